/*
 * midman_hip.h -- C ABI of libmidman_hip.so, the MI355X (gfx950) implementation
 * of midman-ai's decoder forward + cross-entropy loss, the autograd matmul
 * backward, the full decoder backward, the clip + AdamW training step,
 * safetensors checkpoints to and from the device, and token shards with the
 * seeded batcher feeding training and evaluation.
 *
 * Conventions follow the reference's own C ABI (crates/midman-api/src/ffi.rs:5-32):
 *   - Handles, not pointers, for library objects (contexts, models). A stale or
 *     invented handle is an error status, never undefined behaviour.
 *   - The caller owns its input buffers; outputs go to caller buffers.
 *   - Every function returns an int32 status (codes below); the message of the
 *     last failure on the calling thread is read with mmh_error_ptr/len.
 *     Nothing unwinds across the boundary.
 *   - One thread per context: a context (and the models on it) must be used
 *     from one thread at a time.
 *   - A model config is 10 doubles in the reference order (ffi.rs:27-32,68-79):
 *     [vocab_size, d_model, n_layers, n_heads, n_kv_heads, d_ff, max_seq_len,
 *      rope_theta, norm_eps, tie_embeddings].
 *
 * Device-buffer entry points (mmh_gemm_*, mmh_rms_norm, ...) take device
 * pointers from mmh_alloc and are asynchronous on the context's HIP stream.
 * Token ids and targets are always host arrays: they are validated on the host
 * (id < V, as ops_shape.rs:250-252 and ops_reduce.rs:250-252 do) before any
 * launch, so an out-of-range id is MMH_ERR_INDEX and nothing runs.
 *
 * Numerics: all arithmetic is IEEE f32 as in the reference; GEMM sums are
 * formed by fp32 MFMA in a different order from the reference's sequential
 * p-ascending loop, so results agree within a tolerance, not bit for bit
 * (see each function). Embedding, RoPE, token and index handling are bit-exact.
 */
#ifndef MIDMAN_HIP_H
#define MIDMAN_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MMH_ABI_VERSION 1u

/* Status codes: the values of ffi.rs:44-61 plus one for the device. */
#define MMH_OK 0
#define MMH_STOPPED 1
#define MMH_ERR_ARGUMENT (-1) /* null pointer, bad handle, value out of range */
#define MMH_ERR_CONFIG (-2)   /* invalid model config (config.rs:106-138) */
#define MMH_ERR_SHAPE (-3)    /* sizes that do not fit */
#define MMH_ERR_INDEX (-4)    /* token id or target >= vocab */
#define MMH_ERR_OTHER (-5)    /* any other library error */
#define MMH_ERR_DEVICE (-6)   /* a HIP runtime error (no reference counterpart) */
#define MMH_ERR_PANIC (-99)   /* an internal exception caught at the boundary */

typedef int64_t mmh_handle;

/* ---- library ---------------------------------------------------------- */

/* ffi.rs:42 ABI_VERSION. */
uint32_t mmh_abi_version(void);
/* ffi.rs midman_error_ptr/midman_error_len: the calling thread's last error
 * message (not NUL-terminated; valid until the next call on this thread). */
const char *mmh_error_ptr(void);
uint32_t mmh_error_len(void);

/* ---- context: one HIP device + one stream ------------------------------ */

/* No reference counterpart (the reference has no device); the analogue of
 * midman_lab_create's handle table (ffi.rs:473). */
int32_t mmh_context_create(int32_t device, mmh_handle *out_ctx);
int32_t mmh_context_destroy(mmh_handle ctx);
/* Waits for all work queued on the context's stream. */
int32_t mmh_synchronize(mmh_handle ctx);
/* Device name (NUL-terminated, truncated to cap) and compute-unit count. */
int32_t mmh_device_info(mmh_handle ctx, char *name, uint32_t cap, int32_t *cu_count);
/* Diagnostic with no reference counterpart: how the fused forward (see
 * MMH_PATH_AUTO) gives its workgroups their per-XCD team slots on this
 * context. *teams = 1 when the context's probe found 8 XCDs dealt equal
 * shares (else the fused launch is not used). *round_robin = 1 when the probe
 * also found the dispatch dealing workgroup b to XCD (b + o) % 8 with o fixed
 * per launch, so a workgroup's slot is b / 8 with no atomic (each launch still
 * checks that all its workgroups saw one offset, else the forward is redone on
 * the per-operation kernels); 0: one returning atomic per workgroup. The
 * environment variable MMH_FUSED_ATOMIC_SLOTS=1 at context creation forces
 * the atomic slots. Either pointer may be NULL. */
int32_t mmh_context_fused_slots(mmh_handle ctx, int32_t *teams, int32_t *round_robin);
/* Diagnostic with no reference counterpart: the fp32 MFMA rate the whole chip
 * sustains on register operands with no memory traffic (4 independent
 * 32x32x2 chains per wave, 4 waves per SIMD, operands with pseudo-random
 * mantissas changing every MFMA as a GEMM's do), in TFLOP/s: the practical
 * ceiling under the published 157.3 TFLOP/s for the GEMM kernels (the clock
 * the matrix cores hold drops with the operand bits they toggle). */
int32_t mmh_mfma_peak_probe(mmh_handle ctx, double *tflops);

/* Device memory owned by the caller through the context. */
int32_t mmh_alloc(mmh_handle ctx, uint64_t bytes, void **out_dev);
int32_t mmh_free(mmh_handle ctx, void *dev);
/* Synchronous copies host <-> device, ordered after queued work. */
int32_t mmh_upload(mmh_handle ctx, void *dst_dev, const void *src_host, uint64_t bytes);
int32_t mmh_download(mmh_handle ctx, void *dst_host, const void *src_dev, uint64_t bytes);
/* HIP-event timing of the context's stream: start records, stop records and
 * waits, and returns the milliseconds between the two. */
int32_t mmh_timer_start(mmh_handle ctx);
int32_t mmh_timer_stop(mmh_handle ctx, float *ms);

/* Tensor::randn(shape, std, &mut Rng::seed_from_u64(seed)) (tensor.rs:158-162,
 * rng.rs:36-84) into a host array of n values: the reference's bits. */
int32_t mmh_randn(uint64_t seed, float std, float *out_host, int64_t n);

/* ---- the GEMM seam: midman-tensor/src/kernels.rs:49-84 ------------------ */

/* All matrices row-major f32. accumulate != 0 adds into C (the reference
 * kernels always accumulate, kernels.rs:48); accumulate == 0 overwrites C.
 * Tolerance against the reference order: |diff| <= 1e-5 * sum_p |a_p b_p|. */

/* kernels.rs:49 gemm_nn: C[m,n] (+)= A[m,k] B[k,n] */
int32_t mmh_gemm_nn(mmh_handle ctx, const float *a, const float *b, float *c, int64_t m,
                    int64_t k, int64_t n, int32_t accumulate);
/* kernels.rs:66 gemm_nt: C[m,n] (+)= A[m,k] B[n,k]^T (no transpose is materialized) */
int32_t mmh_gemm_nt(mmh_handle ctx, const float *a, const float *b, float *c, int64_t m,
                    int64_t k, int64_t n, int32_t accumulate);
/* kernels.rs:78 gemm_tn: C[m,n] (+)= A[k,m]^T B[k,n] */
int32_t mmh_gemm_tn(mmh_handle ctx, const float *a, const float *b, float *c, int64_t m,
                    int64_t k, int64_t n, int32_t accumulate);
/* mmh_gemm_nn / _nt / _tn (form MMH_GEMM_NN, _NT, _TN) without any device
 * allocation. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). The same kernels and split choices as the
 * three entry points above, so the same bits; the split-K partials live in a
 * fixed 16 MiB device array per GPU instead of the context's workspace. A
 * product whose partials need more is refused with MMH_ERR_SHAPE before
 * anything runs: a K split needs splits x m x n x 4 bytes (chosen only when
 * the output tiles cannot fill the chip; every product of the benchmark sweep
 * fits), the 128x128 kernel's tail balance 64 KiB per piece of its last
 * tiles (a grid of q x CUs + R tiles cut into s pieces each: R x s x 64 KiB).
 * The split choices never depend on the array, so an accepted call gives the
 * allocating entry point's bits. The array is shared by every call on a
 * GPU: calls that overlap on one GPU (other streams, contexts or threads) race
 * on it. */
#define MMH_GEMM_NN 0
#define MMH_GEMM_NT 1
#define MMH_GEMM_TN 2
int32_t mmh_gemm_noalloc(mmh_handle ctx, int32_t form, const float *a, const float *b,
                         float *c, int64_t m, int64_t k, int64_t n, int32_t accumulate);
/* ops_matmul.rs:87-96, batched form: C[i] = A[i] B[i] for i < batch, each
 * [m,k] x [k,n], contiguous. */
int32_t mmh_matmul_batched(mmh_handle ctx, const float *a, const float *b, float *c,
                           int64_t batch, int64_t m, int64_t k, int64_t n);
/* ops_matmul.rs:62-74, the shared-rhs matmul backward: for C[rows,n] =
 * A[rows,k] B[k,n], dA = dC B^T ([rows,k]) and dB = A^T dC ([k,n]). A NULL
 * output is "not needed" (the reference's need flags). Outputs overwritten. */
int32_t mmh_matmul_backward(mmh_handle ctx, const float *a, const float *b, const float *dc,
                            float *da, float *db, int64_t rows, int64_t k, int64_t n);

/* ---- layer ops: midman-nn/src/lib.rs:45-56 ------------------------------ */

/* ops_shape.rs:230-257: out[i,:] = table[ids[i],:]; ids on the host. Bit-exact. */
int32_t mmh_embedding(mmh_handle ctx, const float *table, int64_t vocab, int64_t d,
                      const int32_t *ids_host, int64_t n, float *out);
/* norm.rs:21-39: out = x * (mean(x^2) + eps)^(-1/2) * w over rows of d. */
int32_t mmh_rms_norm(mmh_handle ctx, const float *x, const float *w, int64_t rows, int64_t d,
                     float eps, float *out);
/* rope.rs:54-85: cos/sin tables [max_seq_len, head_dim/2] (angles in f64,
 * stored f32; bit-exact), written to device buffers. */
int32_t mmh_rope_tables(mmh_handle ctx, int64_t head_dim, int64_t max_seq_len, float theta,
                        float *cos_dev, float *sin_dev);
/* rope.rs:20-33 / :114-128: x [bh, t, hd], positions 0..t-1. Bit-exact. */
int32_t mmh_apply_rope(mmh_handle ctx, const float *x, int64_t bh, int64_t t, int64_t hd,
                       const float *cos_dev, const float *sin_dev, float *out);
/* attention.rs:97-101: q [B,H,T,hd], k/v [B,Hkv,T,hd] (already rotated),
 * out [B,H,T,hd]; head j reads kv head j / (H/Hkv). hd 4, 8, 16, 32, 64 or
 * 128 runs on its own kernels; any other even hd below 128 on the next of
 * those, through copies of the heads padded with zero columns (the scale
 * stays 1/sqrt(hd)); hd above 128 is MMH_ERR_SHAPE. The backward likewise. */
int32_t mmh_causal_attention(mmh_handle ctx, const float *q, const float *k, const float *v,
                             int64_t b, int64_t h, int64_t hkv, int64_t t, int64_t hd,
                             float *out);
/* Backward closures of the layer seam (autograd.rs:69-125 through the ops each
 * layer is composed of). Outputs are overwritten.
 * rms_norm (norm.rs:36-38 via ops_elementwise.rs:123-198,287,309,335 and
 * ops_reduce.rs:34-92): dx = d(loss)/dx, dw summed over rows. */
int32_t mmh_rms_norm_backward(mmh_handle ctx, const float *x, const float *w, const float *dy,
                              int64_t rows, int64_t d, float eps, float *dx, float *dw);
/* apply_rope (rope.rs:28-32): dx1 = dy1*cos + dy2*sin, dx2 = dy2*cos - dy1*sin.
 * Bit-exact. dx may equal dy. */
int32_t mmh_apply_rope_backward(mmh_handle ctx, const float *dy, int64_t bh, int64_t t,
                                int64_t hd, const float *cos_dev, const float *sin_dev,
                                float *dx);
/* causal_attention (attention.rs:79-101 with ops_matmul.rs:100-125,
 * ops_reduce.rs:144-175, ops_shape.rs:209-219): dq [B,H,T,hd], dk/dv
 * [B,Hkv,T,hd] from dout [B,H,T,hd]; the copies of a kv head are summed. */
int32_t mmh_causal_attention_backward(mmh_handle ctx, const float *q, const float *k,
                                      const float *v, const float *dout, int64_t b, int64_t h,
                                      int64_t hkv, int64_t t, int64_t hd, float *dq, float *dk,
                                      float *dv);
/* Tensor::cross_entropy backward (ops_reduce.rs:261-275) for loss gradient 1:
 * dlogits = (softmax - onehot) / N (may equal logits); loss_host may be NULL. */
int32_t mmh_cross_entropy_backward(mmh_handle ctx, const float *logits,
                                   const int32_t *targets_host, int64_t n, int64_t vocab,
                                   float *dlogits, float *loss_host);
/* attention.rs:146-170: x [B,T,d] -> out [B,T,d]; weights [d,d],[d,kv],[d,kv],[d,d]. */
int32_t mmh_attention_forward(mmh_handle ctx, const float *x, const float *wq, const float *wk,
                              const float *wv, const float *wo, const float *cos_dev,
                              const float *sin_dev, int64_t b, int64_t t, int64_t d,
                              int64_t h, int64_t hkv, float *out);
/* mlp.rs:20-24: out = (silu(x Wg) * (x Wu)) Wd; x [rows,d]. */
int32_t mmh_swiglu(mmh_handle ctx, const float *x, const float *wg, const float *wu,
                   const float *wd, int64_t rows, int64_t d, int64_t ff, float *out);
/* ops_elementwise.rs:249-259 same-shape add: out = a + b. Bit-exact. */
int32_t mmh_add(mmh_handle ctx, const float *a, const float *b, float *out, int64_t n);
/* ops_reduce.rs:236-259: mean over rows of max + ln(sum exp(z - max)) - z[t],
 * accumulated in f64; targets on the host; the loss is returned to the host. */
int32_t mmh_cross_entropy(mmh_handle ctx, const float *logits, const int32_t *targets_host,
                          int64_t n, int64_t vocab, float *loss_host);

/* ---- model: midman-model/src/model.rs ---------------------------------- */

/* model.rs:51-83 with weights given by the caller in the reference parameter
 * order (docs/midman-model.md:20): embed; per block attn_norm, q, k, v, o,
 * mlp_norm, gate, up, down; final_norm; lm_head if untied. The config checks
 * are config.rs:106-138's (MMH_ERR_CONFIG), plus a head width of at most 128
 * (d_model / n_heads; every even width up to it is taken). */
int32_t mmh_model_create(mmh_handle ctx, const double config[10], const float *weights_host,
                         int64_t n_weights, mmh_handle *out_model);
/* MidManModel::with_init_std(config, std, &mut Rng::seed_from_u64(seed))
 * (model.rs:51-83): the same weights bit for bit. The model keeps the Rng
 * after the draws for mmh_model_lab_tokens. */
int32_t mmh_model_create_seeded(mmh_handle ctx, const double config[10], uint64_t seed,
                                float std, mmh_handle *out_model);
/* Lab::new's task (lab.rs:194-203): continues the model's Rng with batch
 * sequences of seq+1 draws of below(vocab); inputs = tokens[..seq],
 * targets = tokens[1..]. Bit-exact. */
int32_t mmh_model_lab_tokens(mmh_handle model, int64_t batch, int64_t seq, int32_t *inputs,
                             int32_t *targets);
int32_t mmh_model_param_count(mmh_handle model, int64_t *out);
/* Copies the weights back in the reference parameter order. */
int32_t mmh_model_download_weights(mmh_handle model, float *out_host, int64_t n);
/* model.rs:103: logits [B,T,V] to the host. */
int32_t mmh_model_forward(mmh_handle model, const int32_t *ids_host, int64_t batch, int64_t seq,
                          float *logits_host);
/* model.rs:174: the mean next-token cross-entropy. */
int32_t mmh_model_loss(mmh_handle model, const int32_t *inputs_host,
                       const int32_t *targets_host, int64_t batch, int64_t seq,
                       float *loss_host);
/* forward + loss in one pass; logits_host may be NULL. Tolerances against the
 * reference CPU path: loss <= 1e-4 relative; logits max|diff| per row
 * <= 1e-3 * max|row|. */
int32_t mmh_model_forward_loss(mmh_handle model, const int32_t *inputs_host,
                               const int32_t *targets_host, int64_t batch, int64_t seq,
                               float *logits_host, float *loss_host);
int32_t mmh_model_destroy(mmh_handle model);
/* Diagnostic with no reference counterpart (the guard-band checks of
 * kernels_avx.rs:368-390, on the device): the model's activation and training
 * buffers are carved into slots separated by guard words of 0x7FC0DEAD, set
 * when the buffers are allocated; this waits for queued work and counts the
 * guard words that no longer hold that value (0 unless a kernel wrote outside
 * its output: the logits, the loss partials of the head GEMM, the saved
 * gate/up pairs, ...). */
int32_t mmh_model_check_guards(mmh_handle model, uint64_t *broken_words);

/* Device-resident steps (no reference counterpart: the reference has no
 * device; these split model.rs:174's loss into upload / run / read so a caller
 * can keep the tokens in HBM and queue steps without host round trips).
 * stage validates the ids on the host (MMH_ERR_INDEX for id >= V) and copies
 * them into the model's token buffers; run_staged queues forward + loss on
 * them and returns without waiting; read_loss waits and returns the loss of
 * the last staged run. On the per-operation kernels run_staged runs the
 * first call for a (batch, seq) eagerly, captures the second into a HIP graph
 * (kernel launches only) and replays it afterwards; a new shape or
 * re-allocated activations start over. The fused forward (one kernel, see
 * mmh_model_set_forward_path) is launched directly on every call. */
int32_t mmh_model_stage(mmh_handle model, const int32_t *inputs_host,
                        const int32_t *targets_host, int64_t batch, int64_t seq);
int32_t mmh_model_run_staged(mmh_handle model, int64_t batch, int64_t seq);
int32_t mmh_model_read_loss(mmh_handle model, float *loss_host);

/* Which kernels a loss-only forward (mmh_model_loss, run_staged, evaluation)
 * runs on (no reference counterpart: the reference has one CPU path).
 * MMH_PATH_AUTO (the default): one persistent launch for the whole forward +
 * loss where the model fits it (heads of 16 or 32, d_model a multiple of 32
 * up to 256, d_ff a multiple of 4, at most 16384 tokens: the smoke and tiny
 * presets), the per-operation kernels otherwise. MMH_PATH_PER_OP: always the
 * per-operation kernels. The two agree within the forward's tolerance. The
 * fused launch needs every CU of the GPU at once (one workgroup per CU, 8
 * XCDs dealt equal shares: checked when the context is created, else AUTO
 * means PER_OP); kernels of other streams or processes that hold CUs delay
 * it, and two fused launches on different streams of one GPU can hold each
 * other's CUs until a wait gives up. Every wait is bounded (2^18 polls), and
 * a fused launch that gave up is redone on the per-operation kernels from the
 * ids and targets still staged in HBM, before mmh_model_loss returns or
 * before mmh_model_read_loss reads the loss (or when new ids are staged
 * first): the loss returned is always that of a complete forward. Logits-producing
 * forwards, mmh_model_profile and training always use the per-operation
 * kernels. */
#define MMH_PATH_AUTO 0
#define MMH_PATH_PER_OP 1
int32_t mmh_model_set_forward_path(mmh_handle model, int32_t path);
/* 1 in *fused when the model's last queued forward (or the graph that
 * mmh_model_run_staged replays) is the fused launch, else 0 (no reference
 * counterpart; lets a caller or a test see which path MMH_PATH_AUTO took).
 * After a fused launch was redone on the per-operation kernels this is 0. */
int32_t mmh_model_last_forward_fused(mmh_handle model, int32_t *fused);
/* How many fused launches of this model gave up and were redone on the
 * per-operation kernels, and the error word of the last one (bit 0: a
 * dependency wait reached its bound; bit 1: more workgroups landed on one XCD
 * than its team holds; bit 2: row blocks were left uncombined; higher bits:
 * set by mmh_model_inject_fused_error). last_error may be NULL. No reference
 * counterpart. */
int32_t mmh_model_fused_fallbacks(mmh_handle model, int64_t *redone, int32_t *last_error);
/* Diagnostic with no reference counterpart: the next fused launch of this
 * model (eager or a graph replay) starts with `bits` (> 0) in its error word,
 * so its waits give up as they do when the launch's workgroups are not all
 * resident; every workgroup still runs to its end. The failure handling
 * above (the redo, the cleared counters) can then be exercised without
 * making the GPU wait. */
int32_t mmh_model_inject_fused_error(mmh_handle model, int32_t bits);
/* Diagnostic with no reference counterpart (a timing analogue of
 * forward_traced, model.rs:116-125, for the fused launch, whose kernels
 * mmh_model_profile cannot separate): runs the staged loss-only forward
 * `reps` times (1..100000) as the fused launch, back to back, with every
 * workgroup recording the device's constant-rate wall clock at its start and
 * end; per launch the duration is the last end minus the first start. Fills
 * the median (and, when min_us is not NULL, the minimum) in microseconds;
 * the staged loss is then that of the last launch. MMH_ERR_ARGUMENT when
 * nothing is staged for (batch, seq) or the fused launch does not take this
 * model and shape; MMH_ERR_DEVICE when a timed launch gave up (its forward is
 * redone first). */
int32_t mmh_model_fused_duration(mmh_handle model, int64_t batch, int64_t seq, int32_t reps,
                                 float *median_us, float *min_us);

/* Kernel classes timed by mmh_model_profile. */
#define MMH_PROF_EMBEDDING 0
#define MMH_PROF_RMS_NORM 1
#define MMH_PROF_GEMM_QKV 2
#define MMH_PROF_GEMM_O 3
#define MMH_PROF_GEMM_GATE_UP 4
#define MMH_PROF_GEMM_DOWN 5
#define MMH_PROF_GEMM_HEAD 6
#define MMH_PROF_ATTENTION 7
#define MMH_PROF_LOSS 8
#define MMH_PROF_CLASSES 9
/* One staged forward + loss with a HIP event pair around every launch (the
 * analogue of forward_traced for timing, model.rs:116-125): per class, the
 * summed milliseconds and the number of launches. Arrays hold
 * MMH_PROF_CLASSES entries. */
int32_t mmh_model_profile(mmh_handle model, int64_t batch, int64_t seq, float *class_ms,
                          int32_t *class_launches);

/* ---- Training: backward, global-norm clip, AdamW, schedule ----------------
 * model.loss(..).backward() + gather_gradients (model.rs:174-183,
 * autograd.rs:69-125, clip.rs:17-27): forward + loss + the gradient of every
 * parameter, kept on the device in the reference parameter order. loss_host
 * may be NULL. Tolerance against the reference: each parameter's gradient
 * max|diff| <= 2e-3 * max|grad| of that parameter, the global norm <= 1e-4
 * relative. */
int32_t mmh_model_backward(mmh_handle model, const int32_t *inputs_host,
                           const int32_t *targets_host, int64_t batch, int64_t seq,
                           float *loss_host);
/* The gradients of the last backward or training step, reference order. */
int32_t mmh_model_download_grads(mmh_handle model, float *out_host, int64_t n);
/* global_norm of those gradients (clip.rs:30-33): f64 sum of squares. */
int32_t mmh_model_grad_norm(mmh_handle model, float *norm_host);
/* AdamW::new(beta1, beta2, eps, weight_decay) (adamw.rs:48-66) together with
 * the clip limit of Lab/Trainer (lab.rs:185-190, clip.rs:42-47). Replaces any
 * earlier optimizer: moments and the step count start from zero. */
int32_t mmh_model_set_optimizer(mmh_handle model, float beta1, float beta2, float eps,
                                float weight_decay, float clip_norm);
/* Lab::step_once (lab.rs:263-283) / Trainer::update (trainer.rs:185-205) at
 * learning rate lr: loss, backward, clip_global_norm (clip.rs:42-60) and
 * AdamW::step (adamw.rs:180-214), all on the device. loss_host and
 * grad_norm_host (the norm before clipping) may be NULL. When the loss or the
 * gradient norm is not finite, returns MMH_STOPPED with the reference's
 * message and changes nothing (weights, moments, step count). */
int32_t mmh_model_train_step(mmh_handle model, const int32_t *inputs_host,
                             const int32_t *targets_host, int64_t batch, int64_t seq, float lr,
                             float *loss_host, float *grad_norm_host);
/* The same split for callers that keep one batch on the device (Lab trains
 * on a fixed task): stage_train validates and uploads ids and targets and
 * builds the embedding-backward index; train_staged runs one step on them. */
int32_t mmh_model_stage_train(mmh_handle model, const int32_t *inputs_host,
                              const int32_t *targets_host, int64_t batch, int64_t seq);
int32_t mmh_model_train_staged(mmh_handle model, int64_t batch, int64_t seq, float lr,
                               float *loss_host, float *grad_norm_host);
/* AdamW::step_count (adamw.rs:69-71). */
int32_t mmh_model_optimizer_steps(mmh_handle model, uint64_t *out);
/* WarmupCosine::new + lr(step) (schedule.rs:25-66), f64 inside, f32 out. */
int32_t mmh_warmup_cosine_lr(float max_lr, float min_lr, uint64_t warmup_steps,
                             uint64_t total_steps, uint64_t step, float *lr_out);

/* DecoderBlock::forward (block.rs:67-81): out = h + mlp(mlp_norm(h)) with
 * h = x + attn(attn_norm(x)), on device buffers. block_weights holds the
 * block's parameters in DecoderBlock::parameters order (block.rs:85-93):
 * attn_norm [d], q [d,d], k [d,kv], v [d,kv], o [d,d], mlp_norm [d],
 * gate [d,ff], up [d,ff], down [ff,d] (kv = hkv * d/h). x, out [b,t,d]; out
 * may be x itself but must not otherwise overlap it. cos/sin are the rotary
 * tables (mmh_rope_tables) for at least t positions. Tolerance as
 * mmh_attention_forward + mmh_swiglu. */
int32_t mmh_block_forward(mmh_handle ctx, const float *x, const float *block_weights,
                          const float *cos_dev, const float *sin_dev, int64_t b, int64_t t,
                          int64_t d, int64_t h, int64_t hkv, int64_t ff, float eps, float *out);

/* Backward of swiglu (mlp.rs:20-24: out = (silu(x Wg) * (x Wu)) Wd) for the
 * incoming dout [rows, d]: dx [rows, d], dwg, dwu [d, ff], dwd [ff, d], all
 * overwritten (g, u and h are recomputed from x). The silu*mul closure
 * (ops_elementwise.rs:287, :355-364) is elementwise-exact; the products
 * carry the GEMM tolerance. */
int32_t mmh_swiglu_backward(mmh_handle ctx, const float *x, const float *wg, const float *wu,
                            const float *wd, const float *dout, int64_t rows, int64_t d,
                            int64_t ff, float *dx, float *dwg, float *dwu, float *dwd);
/* Backward of embedding (ops_shape.rs:261-269): dtable [vocab, d] = zeros,
 * plus for each position i the row dy[i] added to dtable[ids[i]], in position
 * order (no atomics: bit-exact). ids on the host (MMH_ERR_INDEX for >= vocab). */
int32_t mmh_embedding_backward(mmh_handle ctx, const int32_t *ids_host, int64_t n,
                               const float *dy, int64_t vocab, int64_t d, float *dtable);

/* ---- Checkpoints: midman-checkpoint (safetensors.rs, params.rs) -----------
 * TensorFile (safetensors.rs:68-330): named F32 tensors + string metadata,
 * read with the reference's validation (8-byte length, <= 100 MB header of
 * restricted JSON, F32 only, offsets tiling the data exactly) and written
 * byte-identically (tensors sorted by name, __metadata__ first with sorted
 * keys, serde_json string escapes, header space-padded to a multiple of 8).
 * Host-only: no device is needed. Names and strings are (pointer, length). */
int32_t mmh_tensorfile_create(mmh_handle *out);                       /* TensorFile::new */
int32_t mmh_tensorfile_parse(const uint8_t *bytes, uint64_t len, mmh_handle *out); /* from_bytes */
/* TensorFile::push: copies the values; the name must be new and not __metadata__. */
int32_t mmh_tensorfile_push(mmh_handle tf, const char *name, uint32_t name_len,
                            const uint64_t *shape, int32_t rank, const float *data, uint64_t n);
int32_t mmh_tensorfile_set_metadata(mmh_handle tf, const char *key, uint32_t key_len,
                                    const char *value, uint32_t value_len);
int32_t mmh_tensorfile_count(mmh_handle tf, int64_t *n_tensors, int64_t *n_metadata);
/* Tensor i (insertion order, or file order for a parsed file). */
int32_t mmh_tensorfile_tensor(mmh_handle tf, int64_t i, char *name, uint32_t name_cap,
                              uint32_t *name_len, int32_t *rank, uint64_t *shape,
                              int32_t shape_cap, uint64_t *numel);
int32_t mmh_tensorfile_read(mmh_handle tf, int64_t i, float *out, uint64_t n);
/* Metadata entry i in key order. */
int32_t mmh_tensorfile_metadata(mmh_handle tf, int64_t i, char *key, uint32_t key_cap,
                                uint32_t *key_len, char *value, uint32_t value_cap,
                                uint32_t *value_len);
/* TensorFile::to_bytes; out may be NULL to learn *len. */
int32_t mmh_tensorfile_serialize(mmh_handle tf, uint8_t *out, uint64_t cap, uint64_t *len);
int32_t mmh_tensorfile_destroy(mmh_handle tf);

/* save_parameters (params.rs:36-80, safetensors.rs:220-250) from the device:
 * one tensor per parameter under the reference's names (embed_tokens.weight,
 * blocks.{i}.attn_norm.weight, blocks.{i}.attn.{q,k,v,o}_proj.weight,
 * blocks.{i}.mlp_norm.weight, blocks.{i}.mlp.{gate,up,down}_proj.weight,
 * final_norm.weight, lm_head.weight), metadata format = "midman-checkpoint",
 * checkpoint_version = "1" plus the caller's pairs (those two keys are
 * reserved). The bytes stream device -> pinned staging -> <path>.tmp, which is
 * flushed and renamed over path. The file is byte-identical to the reference
 * writer's for the same weights. */
int32_t mmh_model_save_checkpoint(mmh_handle model, const char *path, const char *const *keys,
                                  const char *const *values, int64_t n_metadata);
/* check_header + load_parameters (params.rs:82-210) straight into HBM: strict
 * (every parameter with its shape, nothing else, format and version checked)
 * and all or nothing (the old weights stay unless the whole file was read). */
int32_t mmh_model_load_checkpoint(mmh_handle model, const char *path);
/* A model built from a checkpoint file (config as mmh_model_create). */
int32_t mmh_model_create_from_checkpoint(mmh_handle ctx, const double config[10],
                                         const char *path, mmh_handle *out_model);

/* ---- Training data: midman-data (hash.rs, shard.rs, batch.rs) -------------
 * Host-only except the two model entry points at the end. Errors carry the
 * reference's messages: MMH_ERR_ARGUMENT for Error::InvalidArgument,
 * MMH_ERR_OTHER for Error::Parse, Error::UnsupportedVersion and Error::Io.
 * A batcher is not safe to use from two threads at once. */

/* sha256 (hash.rs) of len bytes into digest[32]. */
int32_t mmh_sha256(const uint8_t *data, uint64_t len, uint8_t *digest);
/* Sha256::new / update / finalize (hash.rs); finalize frees the handle. */
int32_t mmh_sha256_new(mmh_handle *out);
int32_t mmh_sha256_update(mmh_handle hasher, const uint8_t *data, uint64_t len);
int32_t mmh_sha256_finalize(mmh_handle hasher, uint8_t *digest);
/* The compression path (no reference counterpart): mode 0 = the best the CPU
 * has, 1 = portable, 2 = the x86 SHA extensions if present; *in_use = 1 or 2. */
int32_t mmh_sha256_select(int32_t mode, int32_t *in_use);

/* TokenShard::new (shard.rs:66-83): copies the n tokens. */
int32_t mmh_shard_create(uint32_t vocab_size, uint32_t eos, const uint32_t *tokens, uint64_t n,
                         mmh_handle *out);
/* TokenShard::from_bytes (shard.rs:146-223): magic, version, the width for
 * the vocabulary, eos, the exact length, the SHA-256 and every id checked. */
int32_t mmh_shard_parse(const uint8_t *bytes, uint64_t len, mmh_handle *out);
/* TokenShard::load / save (shard.rs:233-260); save writes <path>.tmp, fsyncs
 * it and renames it over path. */
int32_t mmh_shard_load(const char *path, mmh_handle *out);
int32_t mmh_shard_save(mmh_handle shard, const char *path);
/* vocab_size, eos, len, token_width (shard.rs:86-115) and the file size; any
 * output may be NULL. */
int32_t mmh_shard_info(mmh_handle shard, uint32_t *vocab_size, uint32_t *eos, uint64_t *len,
                       uint32_t *token_width, uint64_t *file_bytes);
/* TokenShard::tokens: n must be the shard's length. */
int32_t mmh_shard_tokens(mmh_handle shard, uint32_t *out, uint64_t n);
/* TokenShard::to_bytes (shard.rs:112-135); out may be NULL to learn *len. */
int32_t mmh_shard_serialize(mmh_handle shard, uint8_t *out, uint64_t cap, uint64_t *len);
int32_t mmh_shard_destroy(mmh_handle shard);

/* Sequences::new (batch.rs:45-70) over n_shards shard handles (the shards are
 * shared, not copied; destroying a shard handle later is fine). */
int32_t mmh_sequences_create(const mmh_handle *shards, int64_t n_shards, uint64_t seq_len,
                             mmh_handle *out);
/* len, seq_len, vocab_size (-1 with no shards) (batch.rs:73-93). */
int32_t mmh_sequences_info(mmh_handle seqs, uint64_t *len, uint64_t *seq_len,
                           int64_t *vocab_size);
/* Sequences::window (batch.rs:96-104): seq_len + 1 ids into out;
 * MMH_ERR_INDEX where the reference returns None. */
int32_t mmh_sequences_window(mmh_handle seqs, uint64_t index, uint32_t *out);
int32_t mmh_sequences_destroy(mmh_handle seqs);

/* Batcher::new (batch.rs:161-172). */
int32_t mmh_batcher_create(mmh_handle seqs, uint64_t batch_size, uint64_t seed,
                           mmh_handle *out);
/* batches_per_epoch, epoch, position (batch.rs:175-190), batch size and
 * seq_len; any output may be NULL. */
int32_t mmh_batcher_info(mmh_handle batcher, uint64_t *batches_per_epoch, uint64_t *epoch,
                         uint64_t *position, uint64_t *batch_size, uint64_t *seq_len);
/* Batcher::seek (batch.rs:196-208). */
int32_t mmh_batcher_seek(mmh_handle batcher, uint64_t epoch, uint64_t batches_done);
/* Batcher::next_batch (batch.rs:211-239): batch_size * seq_len inputs and
 * targets, row after row; the batch's epoch and index (either may be NULL). */
int32_t mmh_batcher_next(mmh_handle batcher, uint32_t *inputs, uint32_t *targets,
                         uint64_t *epoch, uint64_t *index);
int32_t mmh_batcher_destroy(mmh_handle batcher);

/* Trainer::step (trainer.rs:162-183) at learning rate lr: the batcher's next
 * batch through mmh_model_train_step. The data must fit the model (Trainer::new,
 * trainer.rs:83-108: seq_len <= max_seq_len, the same vocabulary). A step that
 * fails (MMH_STOPPED for a non-finite loss or norm, or any error) changes
 * nothing and puts the batcher back where it was. epoch and index report the
 * batch used (either may be NULL). */
int32_t mmh_model_train_next(mmh_handle model, mmh_handle batcher, float lr, float *loss_host,
                             float *grad_norm_host, uint64_t *epoch, uint64_t *index);
/* Trainer::evaluate (trainer.rs:218-258): at most max_batches batches of
 * min(batch_size, len) sequences, row k of all rows being sequence
 * k * len / rows; the mean of the batch losses (f64 sum). */
int32_t mmh_model_evaluate(mmh_handle model, mmh_handle seqs, uint64_t batch_size,
                           uint64_t max_batches, float *loss_host, uint64_t *batches,
                           uint64_t *tokens);

#ifdef __cplusplus
}
#endif

#endif
