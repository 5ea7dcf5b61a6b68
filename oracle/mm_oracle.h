/*
 * mm_oracle.h -- CPU restatement of midman-ai's decoder forward, loss and
 * matmul backward, used ONLY as the parity checker and as the CPU timing
 * baseline.
 *
 * TEST INFRASTRUCTURE. Nothing in the product (libmidman_hip.so, the Python
 * host package) links, loads or calls this library. Only tests/, the smoke()
 * check in __graft_entry__.py and bench.py's cpu_baseline leg may use it.
 *
 * Every function restates one reference function, op for op, in the same
 * floating-point order (the reference is Rust without FMA contraction; this
 * file is compiled with -ffp-contract=off and no fast-math, and calls the same
 * glibc expf/logf/powf/log/sqrt/sin/cos/pow). File:line citations point into
 * the reference tree (MidManStudio/midman-ai).
 *
 * Pinning (which check fixes which function):
 *   rng            -> KATs rng.rs:127-157 (seeds 0/42 next_u64, below seed 7,
 *                     next_f32 seed 5)
 *   param_count    -> presets.rs:125-138 (six exact totals)
 *   init + forward + loss (whole chain) -> golden loss 2.493498 of the Lab
 *                     config at seed 2024 (web/lab/test/engine.test.mjs:20-26),
 *                     golden first loss 5.5674 of the smoke preset at seed
 *                     2024, B4 T32 (scripts/fixtures/train_smoke_real_run.txt:11)
 *   lab tokens     -> inputs[0] = [9,6,2,3,3,7,8,7,0,5,3,5]
 *                     (engine.test.mjs:118)
 *   gemm nn/nt/tn  -> hand KAT ops_matmul.rs:137-156; bit-identity with the
 *                     reference's own C twin mmb_matmul_ikj (built from
 *                     benches/midman-bench/c/baseline_kernels.c into
 *                     oracle/_ref); float64 brute force
 *   matmul backward-> finite differences of sum(W*(A.B)); float64 brute force
 *   rms_norm       -> known row norm.rs:105-114, eps case :117-125
 *   rope           -> formula rope.rs:320-331, norm preservation
 *   attention      -> score-scaling KAT attention.rs:305-337, single position
 *                     attends to itself (:296-303), GQA = copied heads
 *   swiglu         -> known value mlp.rs:90-98
 *   cross_entropy  -> ln 2 and ln 2 / 2 KATs ops_reduce.rs:363-377
 *   forward_backward (every backward closure together) -> golden gradient
 *                     norm 1.0999628 of the Lab config at seed 2024
 *                     (engine.test.mjs:26); per-op backward -> central
 *                     finite differences in float64 of the forward op
 *   clip + AdamW + schedule + backward over five steps -> golden losses
 *                     and gradient norms of steps 1..4 (engine.test.mjs:25-26);
 *                     AdamW alone -> its three-step table (adamw.rs:234-259);
 *                     schedule -> lr[0] = max/15, lr[14] = max
 *                     (engine.test.mjs:123-131) and schedule.rs tests
 *   fork           -> stream 0 reduces to seed(next_u64()) (pinned above);
 *                     the stream multiplier is floor(2^64/phi), checked
 *                     against the integer square root of 5; the xor that
 *                     combines them is pinned only structurally (the
 *                     reference's rng.rs:231-241 independence test)
 *   shuffle / permutation -> the draws-to-permutation map is a bijection
 *                     over all n! draw tuples for n <= 5 (brute force);
 *                     the reference's batch.rs tests (one pass uses each
 *                     sequence at most once, seeds and passes differ);
 *                     PARITY UNPINNED in absolute terms: the reference
 *                     holds no fixed permutation of a known seed (its one
 *                     batch digest, data-smoke-results.json, needs the
 *                     out-of-scope tokenizer and corpus)
 */
#ifndef MM_ORACLE_H
#define MM_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes, the same values as the reference C ABI
 * (crates/midman-api/src/ffi.rs:44-61). */
#define MMO_OK 0
#define MMO_ERR_ARGUMENT (-1)
#define MMO_ERR_CONFIG (-2)
#define MMO_ERR_SHAPE (-3)
#define MMO_ERR_INDEX (-4)

/* ---- RNG: crates/midman-foundation/src/rng.rs:16-120 ---- */
typedef struct mmo_rng {
    uint64_t s[4];
    int32_t has_spare;
    float spare;
} mmo_rng;

void mmo_rng_seed(mmo_rng *r, uint64_t seed);          /* rng.rs:36-41 */
uint64_t mmo_rng_next_u64(mmo_rng *r);                  /* rng.rs:44-55 */
float mmo_rng_next_f32(mmo_rng *r);                     /* rng.rs:58-60 */
double mmo_rng_next_f64(mmo_rng *r);                    /* rng.rs:63-65 */
float mmo_rng_normal(mmo_rng *r);                       /* rng.rs:74-84 */
uint64_t mmo_rng_below(mmo_rng *r, uint64_t n);         /* rng.rs:91-105 */
/* Rng::fork (rng.rs:117-119): a generator for stream `stream`; advances r. */
void mmo_rng_fork(mmo_rng *r, uint64_t stream, mmo_rng *out);
/* Rng::shuffle (rng.rs:108-113): Fisher-Yates from the end, j = below(i+1). */
void mmo_rng_shuffle_u64(mmo_rng *r, uint64_t *items, uint64_t n);
/* The Batcher's order of pass `epoch` (batch.rs:244-248):
 * Rng::seed_from_u64(seed).fork(epoch).shuffle(0..n). */
void mmo_permutation(uint64_t n, uint64_t seed, uint64_t epoch, uint64_t *out);
/* Tensor::randn (tensor.rs:158-162): dst[i] = std * normal(), in order. */
void mmo_randn(mmo_rng *r, float *dst, int64_t n, float std);

/* ---- Config: crates/midman-model-config/src/config.rs:20-43 ---- */
typedef struct mmo_config {
    int64_t vocab_size, d_model, n_layers, n_heads, n_kv_heads, d_ff, max_seq_len;
    float rope_theta, norm_eps;
    int32_t tie_embeddings;
} mmo_config;

int32_t mmo_config_validate(const mmo_config *c);       /* config.rs:106-138 */
int64_t mmo_param_count(const mmo_config *c);           /* config.rs:158-185; <0 on error */
/* 0 smoke, 1 tiny, 2 small, 3 base, 4 medium, 5 large (presets.rs:61-83). */
int32_t mmo_preset(int32_t which, mmo_config *out);

/* ---- Init: model.rs:51-83 draw order, parameters in Module order ----
 * Flat layout (reference parameter order, docs/midman-model.md:20):
 *   embed [V,d]; per block: attn_norm [d], q [d,d], k [d,kv], v [d,kv],
 *   o [d,d], mlp_norm [d], gate [d,ff], up [d,ff], down [ff,d];
 *   final_norm [d]; lm_head [d,V] only when untied. */
int32_t mmo_init_weights(const mmo_config *c, float std, mmo_rng *r, float *w, int64_t n);
/* The same weights with the Box-Muller arithmetic spread over nthreads
 * threads (draws still taken in stream order): identical bits. */
int32_t mmo_init_weights_mt(const mmo_config *c, float std, mmo_rng *r, float *w, int64_t n,
                            int32_t nthreads);
/* Lab::new token scheme (crates/midman-api/src/lab.rs:194-203). */
void mmo_lab_tokens(mmo_rng *r, int64_t vocab, int64_t batch, int64_t seq,
                    int32_t *inputs, int32_t *targets);

/* ---- GEMM kernels (C accumulates): kernels.rs:49-108 ---- */
/* C[m,n] += A[m,k] B[k,n] */
void mmo_gemm_nn(const float *a, const float *b, float *c, int64_t m, int64_t k, int64_t n,
                 int32_t nthreads);
/* C[m,n] += A[m,k] B[n,k]^T (B copied to [k,n] first, kernels.rs:66-75) */
void mmo_gemm_nt(const float *a, const float *b, float *c, int64_t m, int64_t k, int64_t n,
                 int32_t nthreads);
/* C[m,n] += A[k,m]^T B[k,n] (kernels.rs:78-84, scalar :100-108) */
void mmo_gemm_tn(const float *a, const float *b, float *c, int64_t m, int64_t k, int64_t n,
                 int32_t nthreads);
/* The shared-rhs matmul backward closure (ops_matmul.rs:62-74): for the
 * forward C[rows,n] = A[rows,k] B[k,n], dA = dC B^T and dB = A^T dC. Either
 * output may be NULL ("not needed"). Outputs are overwritten. */
void mmo_matmul_backward(const float *a, const float *b, const float *dc, float *da, float *db,
                         int64_t rows, int64_t k, int64_t n, int32_t nthreads);

/* ---- Layer ops ---- */
int32_t mmo_embedding(const float *table, int64_t v, int64_t d, const int32_t *ids, int64_t n,
                      float *out);                                   /* ops_shape.rs:230-257 */
void mmo_rms_norm(const float *x, const float *w, int64_t rows, int64_t d, float eps,
                  float *out);                                       /* norm.rs:21-39 */
void mmo_rope_tables(int64_t head_dim, int64_t max_seq_len, float theta, float *cos_t,
                     float *sin_t);                                  /* rope.rs:54-85 */
/* x [BH, T, hd] -> out, positions 0..T-1 (rope.rs:20-33, 114-128) */
void mmo_apply_rope(const float *x, int64_t bh, int64_t t, int64_t hd, const float *cos_t,
                    const float *sin_t, float *out);
/* q [B,H,T,hd], k/v [B,Hkv,T,hd] -> out [B,H,T,hd] (attention.rs:79-101) */
void mmo_causal_attention(const float *q, const float *k, const float *v, int64_t b, int64_t h,
                          int64_t hkv, int64_t t, int64_t hd, float *out, int32_t nthreads);
/* x [B,T,d] -> out [B,T,d] (attention.rs:146-170); tables [>=T, hd/2] */
void mmo_attention_forward(const float *x, const float *wq, const float *wk, const float *wv,
                           const float *wo, const float *cos_t, const float *sin_t, int64_t b,
                           int64_t t, int64_t d, int64_t h, int64_t hkv, float *out,
                           int32_t nthreads);
/* x [rows,d] -> out [rows,d] (mlp.rs:20-24) */
void mmo_swiglu(const float *x, const float *wg, const float *wu, const float *wd, int64_t rows,
                int64_t d, int64_t ff, float *out, int32_t nthreads);
/* mean CE over rows, f64 accumulation (ops_reduce.rs:236-259) */
int32_t mmo_cross_entropy(const float *logits, const int32_t *targets, int64_t n, int64_t v,
                          float *loss);
/* Per-row CE terms max + ln(sum) - z[t] as the reference forms them (f32). */
int32_t mmo_cross_entropy_rows(const float *logits, const int32_t *targets, int64_t n,
                               int64_t v, float *row_loss);
/* One pre-norm block (block.rs:77-81); bw points at the block's weights in
 * the flat layout above. x,out [B,T,d]. */
int32_t mmo_block_forward(const mmo_config *c, const float *bw, const float *cos_t,
                          const float *sin_t, const float *x, int64_t b, int64_t t, float *out,
                          int32_t nthreads);
/* Logits [B,T,V] (model.rs:127-165). */
int32_t mmo_forward(const mmo_config *c, const float *w, const int32_t *ids, int64_t b,
                    int64_t t, float *logits, int32_t nthreads);
/* Forward + mean CE (model.rs:174-183). logits may be NULL. */
int32_t mmo_forward_loss(const mmo_config *c, const float *w, const int32_t *ids,
                         const int32_t *targets, int64_t b, int64_t t, float *logits,
                         float *loss, int32_t nthreads);

/* ---- Backward (autograd closures) and the training step ---- */
/* ops_reduce.rs:261-275; g is the loss gradient (1 for loss.backward()). */
int32_t mmo_cross_entropy_backward(const float *logits, const int32_t *targets, int64_t n,
                                   int64_t v, float g, float *dlogits);
/* ops_shape.rs:261-269: dtable[id] += g row, in id order (accumulates). */
void mmo_embedding_backward(const int32_t *ids, int64_t n, const float *g, int64_t d,
                            float *dtable);
/* norm.rs:36-38 backward: dx = the norm's share of d(x) (overwritten),
 * dw = sum over rows (overwritten). */
void mmo_rms_norm_backward(const float *x, const float *w, const float *dy, int64_t rows,
                           int64_t d, float eps, float *dx, float *dw);
/* rope.rs:28-32 backward (rotation by -angle). */
void mmo_rope_backward(const float *dy, int64_t bh, int64_t t, int64_t hd, const float *cos_t,
                       const float *sin_t, float *dx);
/* attention.rs:79-101 backward: dout [B,H,T,hd] -> dq [B,H,T,hd],
 * dk/dv [B,Hkv,T,hd] (overwritten). */
void mmo_causal_attention_backward(const float *q, const float *k, const float *v,
                                   const float *dout, int64_t b, int64_t h, int64_t hkv,
                                   int64_t t, int64_t hd, float *dq, float *dk, float *dv,
                                   int32_t nthreads);
/* h = silu(g)*u backward (mlp.rs:20-24, ops_elementwise.rs:355-364). */
void mmo_silu_mul_backward(const float *gate, const float *up, const float *dh, int64_t n,
                           float *dgate, float *dup);
/* Offsets, sizes and ranks of the parameters in the flat layout; returns the
 * count (at most 9*L + 3). */
int64_t mmo_param_segments(const mmo_config *c, int64_t *offsets, int64_t *sizes,
                           int32_t *ranks);
/* Loss and the gradient of every parameter, flat layout (model.rs:174-183 +
 * loss.backward()). */
int32_t mmo_forward_backward(const mmo_config *c, const float *w, const int32_t *ids,
                             const int32_t *targets, int64_t b, int64_t t, float *loss,
                             float *grads, int32_t nthreads);
float mmo_global_norm(const float *g, int64_t n);                       /* clip.rs:30-33 */
int32_t mmo_clip_global_norm(float *g, int64_t n, float max_norm, float *norm_out); /* :42-60 */
float mmo_warmup_cosine_lr(float max_lr, float min_lr, uint64_t warmup, uint64_t total,
                           uint64_t step);                              /* schedule.rs:54-66 */
/* adamw.rs:180-214 for one parameter at step t (from 1); decays = rank >= 2. */
void mmo_adamw_update(float *w, const float *g, float *m, float *v, int64_t n, int32_t decays,
                      uint64_t t, float lr, float beta1, float beta2, float eps,
                      float weight_decay);
/* AdamW::step over the flat list (rank >= 2 decays); *steps increments. */
int32_t mmo_adamw_step(const mmo_config *c, float *w, const float *g, float *m, float *v,
                       float lr, float beta1, float beta2, float eps, float weight_decay,
                       uint64_t *steps);
/* Lab::new + Lab::step (lab.rs:159-283). hyper = {max_lr, min_lr, warmup,
 * total, weight_decay, clip_norm, beta1, beta2}. Outputs per step may be NULL. */
int32_t mmo_lab_train(const mmo_config *c, const double *hyper, uint64_t seed, int64_t batch,
                      int64_t seq, int64_t steps, float *losses, float *grad_norms, float *lrs,
                      float *weights, int32_t nthreads);

#ifdef __cplusplus
}
#endif

#endif
