// MidManModel on the device (midman-model/src/model.rs): seeded init,
// device-resident weights, forward and forward + cross-entropy loss.
//
// Per block (block.rs:77-81, attention.rs:146-170, mlp.rs:20-24) the device
// runs seven kernels instead of the reference's ~60 ops:
//   rms_norm(x)                         -> xn
//   GEMM xn . [Wq|Wk|Wv]                -> qkv [N, d+2kv]   (one fused GEMM)
//   fused causal attention, RoPE inside -> ctx [N, d]       (heads merged by layout)
//   GEMM ctx . Wo, added into x         -> x                (residual epilogue)
//   rms_norm(x)                         -> xn
//   GEMM xn . [Wg|Wu], silu(g)*u        -> h [N, ff]        (SwiGLU epilogue)
//   GEMM h . Wd, added into x           -> x                (residual epilogue)
// then the final norm, the tied head x . E^T (read as the nt form, E^T never
// exists) and the loss (row log-sum-exp + f64 mean).
//
// Weights live in one device buffer in a device layout that differs from the
// reference parameter order only inside a block: per block attn_norm, Wqkv
// (the q|k|v columns side by side, so QKV is one GEMM), Wo, mlp_norm, Wgu
// (gate column f at 2f and up column f at 2f+1, zero columns up to ff_pad, so
// the SwiGLU epilogue finds g and u in one lane) and Wd. Gradients and the
// AdamW moments use the same layout, so a training step writes the weight
// gradients of the packed matrices in place and updates them with no copies;
// the reference order exists only at the boundary (creation, downloads,
// checkpoints), converted on the device.
//
// Training (Lab::step_once, lab.rs:263-283; Trainer::update, trainer.rs:185-205)
// runs the same forward with every value the backward reads kept per layer
// (block input, both norm outputs, rotated QKV, attention output and its
// log-sum-exp, the post-attention residual, the gate/up pre-activations and
// h), then per layer in reverse:
//   GEMM dx . Wd^T with the SwiGLU-backward epilogue -> d(gate, up), in place
//   GEMM h^T . dx -> dWd;  d(gate,up) . Wgu^T -> d(xn2);  xn2^T . d(gate,up) -> dWg, dWu
//   RMSNorm backward (adds into dx, dw);  dx . Wo^T -> d(ctx);  ctx^T . dx -> dWo
//   attention backward (dq, dk, dv, RoPE backward) -> d(qkv)
//   d(qkv) . Wqkv^T -> d(xn1);  xn1^T . d(qkv) -> dWq, dWk, dWv;  RMSNorm backward
// then the embedding scatter. The global norm (f64) and one clip + AdamW pass
// over every parameter follow on the device; the host reads back only the
// loss and the norm.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>

#include "mmh_checkpoint.h"
#include "mmh_data.h"
#include "mmh_internal.h"

namespace mmh {

namespace {

struct Config {
    int64_t vocab = 0, d = 0, layers = 0, heads = 0, kv_heads = 0, ff = 0, max_seq = 0;
    float theta = 0.f, eps = 0.f;
    bool tie = true;
    int64_t hd() const { return d / heads; }
    int64_t kv() const { return kv_heads * hd(); }
    int64_t block_params() const { return 2 * d + 2 * d * d + 2 * d * kv() + 3 * d * ff; }
    int64_t param_count() const {
        return vocab * d + layers * block_params() + d + (tie ? 0 : vocab * d);
    }
};

// ffi.rs:186-200 (config_from) and config.rs:106-138 (validate).
Config parse_config(const double *v) {
    if (!v) fail(MMH_ERR_ARGUMENT, "config is a null pointer");
    static const char *names[10] = {"vocab_size", "d_model", "n_layers", "n_heads",
                                    "n_kv_heads", "d_ff", "max_seq_len", "rope_theta",
                                    "norm_eps", "tie_embeddings"};
    int64_t counts[7];
    for (int i = 0; i < 7; ++i) {
        const double x = v[i];
        if (!(std::isfinite(x) && x >= 0.0 && x == std::floor(x) && x <= 4294967295.0))
            fail(MMH_ERR_ARGUMENT, std::string(names[i]) +
                                       " must be a whole number from 0 to 4294967295");
        counts[i] = (int64_t)x;
    }
    for (int i = 7; i < 9; ++i)
        if (!(std::isfinite(v[i]) && std::fabs(v[i]) <= 3.4028234663852886e38))
            fail(MMH_ERR_ARGUMENT, std::string(names[i]) + " must be a finite number that fits in f32");
    Config c;
    c.vocab = counts[0];
    c.d = counts[1];
    c.layers = counts[2];
    c.heads = counts[3];
    c.kv_heads = counts[4];
    c.ff = counts[5];
    c.max_seq = counts[6];
    c.theta = (float)v[7];
    c.eps = (float)v[8];
    c.tie = v[9] != 0.0;
    for (int i = 0; i < 7; ++i)
        if (counts[i] <= 0) fail(MMH_ERR_CONFIG, std::string(names[i]) + " must be at least 1");
    if (!(std::isfinite(c.theta) && c.theta > 0.f))
        fail(MMH_ERR_CONFIG, "rope_theta must be positive and finite");
    if (!(std::isfinite(c.eps) && c.eps > 0.f))
        fail(MMH_ERR_CONFIG, "norm_eps must be positive and finite");
    if (c.d % c.heads) fail(MMH_ERR_CONFIG, "d_model is not divisible by n_heads");
    if (c.heads % c.kv_heads) fail(MMH_ERR_CONFIG, "n_heads is not divisible by n_kv_heads");
    if (c.hd() & 1) fail(MMH_ERR_CONFIG, "head dimension must be even for rotary embeddings");
    // every even head width the reference accepts (config.rs:130-135) up to
    // 128: 4, 8, 16, 32, 64 and 128 on their own kernels, the others on the
    // next of those through zero-padded heads
    if (c.hd() > 128)
        fail(MMH_ERR_CONFIG, "head dimension " + std::to_string(c.hd()) +
                                 " is above the device attention's 128");
    return c;
}

// One pre-norm block (block.rs:77-81) on packed weights: x += attn(rms(x)),
// then x += mlp(rms(x)), the residual adds fused into the O and down GEMMs,
// SwiGLU into the gate/up GEMM, and the two norms and the q, k rotation
// handed to the QKV and gate/up GEMMs, which fold them in where they can
// (the norms at small widths; the rotation for heads of up to 32 columns on
// the small tiles and of 64 or 128 on the 128x128 tiles) and run them as
// kernels of their own otherwise. timed(class, launch) wraps each launch.
struct BlockRun {
    const float *attn_norm = nullptr, *wqkv = nullptr, *wo = nullptr;
    const float *mlp_norm = nullptr, *wgu = nullptr, *wd = nullptr;
    const float *cos_t = nullptr, *sin_t = nullptr;
    float *x = nullptr;  // [n, d], updated in place
    float *xn = nullptr, *qkv = nullptr, *cb = nullptr, *h = nullptr;
    int64_t batch = 0, seq = 0, d = 0, heads = 0, kv_heads = 0, ff = 0, ff_pad = 0;
    float eps = 0.0f;
};

template <class Timed>
void enqueue_block(Context &c, const BlockRun &r, Timed &&timed) {
    const int64_t n = r.batch * r.seq, d = r.d, hd = d / r.heads, kv = r.kv_heads * hd;
    const int64_t qc = d + 2 * kv;
    // attn_norm and the q, k rotation ride on the QKV product where the GEMM
    // folds them in; otherwise they run (and are timed) as their own kernels
    GemmDesc g;
    g.a = r.x;
    g.norm_w = r.attn_norm;
    g.norm_eps = r.eps;
    g.b = r.wqkv;
    g.c = r.qkv;
    g.m = n;
    g.k = d;
    g.n = qc;
    g.lda = d;
    g.ldb = qc;
    g.ldc = qc;
    g.rope_cos = r.cos_t;
    g.rope_sin = r.sin_t;
    g.rope_seq = r.seq;
    g.rope_hd = hd;
    g.rope_cols = d + kv;
    const GemmFusion fq = gemm_fusion(c, g);
    if (!fq.norm) {
        timed(MMH_PROF_RMS_NORM,
              [&] { launch_rms_norm(c, r.x, r.attn_norm, n, d, r.eps, r.xn); });
        g.a = r.xn;
        g.norm_w = nullptr;
    }
    if (!fq.rope) g.rope_cos = g.rope_sin = nullptr;
    timed(MMH_PROF_GEMM_QKV, [&] { gemm(c, g); });

    AttnDesc a{};
    a.q = r.qkv;
    a.k = r.qkv + d;
    a.v = r.qkv + d + kv;
    a.out = r.cb;
    a.sqb = a.skb = a.svb = r.seq * qc;
    a.sqh = a.skh = a.svh = hd;
    a.sqt = a.skt = a.svt = qc;
    a.sob = r.seq * d;
    a.soh = hd;
    a.sot = d;
    a.b = r.batch;
    a.h = r.heads;
    a.hkv = r.kv_heads;
    a.t = r.seq;
    a.hd = hd;
    if (!fq.rope) {  // attention() rotates q and k first
        a.cos_t = r.cos_t;
        a.sin_t = r.sin_t;
    }
    timed(MMH_PROF_ATTENTION, [&] { attention(c, a); });

    GemmDesc o;
    o.a = r.cb;
    o.b = r.wo;
    o.c = r.x;
    o.m = n;
    o.k = d;
    o.n = d;
    o.lda = d;
    o.ldb = d;
    o.ldc = d;
    o.epi = EPI_ACCUM;
    timed(MMH_PROF_GEMM_O, [&] { gemm(c, o); });

    GemmDesc gu;
    gu.a = r.x;
    gu.norm_w = r.mlp_norm;
    gu.norm_eps = r.eps;
    gu.b = r.wgu;
    gu.c = r.h;
    gu.m = n;
    gu.k = d;
    gu.n = 2 * r.ff_pad;
    gu.lda = d;
    gu.ldb = 2 * r.ff_pad;
    gu.ldc = r.ff;
    gu.epi = EPI_SWIGLU;
    gu.swiglu_ff = r.ff;
    if (!gemm_fusion(c, gu).norm) {
        timed(MMH_PROF_RMS_NORM, [&] { launch_rms_norm(c, r.x, r.mlp_norm, n, d, r.eps, r.xn); });
        gu.a = r.xn;
        gu.norm_w = nullptr;
    }
    timed(MMH_PROF_GEMM_GATE_UP, [&] { gemm(c, gu); });

    GemmDesc dn;
    dn.a = r.h;
    dn.b = r.wd;
    dn.c = r.x;
    dn.m = n;
    dn.k = r.ff;
    dn.n = d;
    dn.lda = r.ff;
    dn.ldb = d;
    dn.ldc = d;
    dn.epi = EPI_ACCUM;
    timed(MMH_PROF_GEMM_DOWN, [&] { gemm(c, dn); });
}

// Activation blocks are carved into slots with a guard band of kGuardFloats
// words before the first slot, between slots and after the last, set to
// kGuardBits when the block is allocated; mmh_model_check_guards counts the
// words that no longer hold it (a kernel that wrote past its output).
constexpr int64_t kGuardFloats = 64;
constexpr uint32_t kGuardBits = 0x7FC0DEADu;

// Allocates sum(sizes) floats plus the bands, writes each slot's base into
// bases[i] and the bands' addresses into bands.
float *alloc_guarded(Context &c, const int64_t *sizes, int nslots, float **bases,
                     std::vector<float *> &bands, const char *what) {
    int64_t total = (nslots + 1) * kGuardFloats;
    for (int i = 0; i < nslots; ++i) total += sizes[i];
    float *mem = nullptr;
    check_hip(hipMalloc(&mem, (size_t)total * 4), what);
    bands.clear();
    float *p = mem;
    for (int i = 0; i < nslots; ++i) {
        bands.push_back(p);
        p += kGuardFloats;
        bases[i] = p;
        p += sizes[i];
    }
    bands.push_back(p);
    for (float *b : bands)
        check_hip(hipMemsetD32Async(reinterpret_cast<hipDeviceptr_t>(b), (int)kGuardBits,
                                    (size_t)kGuardFloats, c.stream),
                  "guard fill");
    return mem;
}

struct Model {
    mmh_handle ctx_handle = 0;
    Context *ctx = nullptr;
    Config cfg;
    int64_t n_params = 0;
    float *w = nullptr;        // the device layout, n_dev floats
    int64_t n_dev = 0;
    int64_t ff_pad = 0;        // ff rounded up to a multiple of 32
    float *cos_t = nullptr, *sin_t = nullptr;
    HostRng rng{};
    bool has_rng = false;
    // Activations for up to cap rows.
    int64_t cap = 0;
    float *act = nullptr;
    std::vector<float *> act_bands, tr_bands;  // guard bands of act and tr.mem
    float *x = nullptr, *xn = nullptr, *qkv = nullptr, *cb = nullptr, *h = nullptr,
          *logits = nullptr, *row_loss = nullptr, *loss = nullptr, *ce_part = nullptr,
          *ce_zt = nullptr;
    int32_t *ids = nullptr, *tgt = nullptr;
    int64_t staged_n = 0;
    bool staged_targets = false;
    // The staged forward + loss of one (batch, seq) as a HIP graph: launch-bound
    // small presets replay ~30 kernels with one call. Valid while the
    // activation buffer and the context's split-K scratch it was captured on
    // are the current ones (other calls on the context may grow the scratch).
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    int64_t graph_b = 0, graph_t = 0, warm_b = 0, warm_t = 0;
    const void *graph_act = nullptr, *warm_act = nullptr, *graph_ws = nullptr,
               *graph_pad = nullptr;
    // The fused loss-only forward (fused_forward.hip): its arena, laid out for
    // (fused_b, fused_t); forward_path 1 keeps every forward on the
    // per-operation kernels. fused_check: a fused launch ran since the error
    // word was last read. last_fused: the last queued forward (or the graph
    // the staged runs replay) was the fused launch.
    float *fused_arena = nullptr;
    int64_t fused_floats = 0, fused_b = 0, fused_t = 0;
    int forward_path = 0;
    bool fused_check = false;
    bool last_fused = false;
    // A fused launch whose error word comes back nonzero is redone on the
    // per-operation kernels: fused_fallbacks counts those redos, fused_last_error
    // keeps the last word seen. fused_inject: bits the host writes into the
    // error word before the next fused launch (a diagnostic: the kernel's waits
    // then give up as under contention, every workgroup still exits).
    // run_b, run_t: the shape of the last staged run, for its redo.
    int64_t fused_fallbacks = 0;
    int32_t fused_last_error = 0, fused_inject = 0;
    int64_t run_b = 0, run_t = 0;
    uint64_t *fused_stamps = nullptr;  // clock stamps for the next fused launch (diagnostic)

    // ---- training state, allocated on the first training call ----
    struct TrainBuf {
        int64_t cap = 0;
        float *mem = nullptr;
        float *xs = nullptr, *xn1 = nullptr, *qkv = nullptr, *cb = nullptr, *lse = nullptr,
              *hres = nullptr, *xn2 = nullptr, *gu = nullptr, *h = nullptr, *xnf = nullptr,
              *dx = nullptr, *dy = nullptr, *dxn = nullptr, *dctx = nullptr, *dqkv = nullptr,
              *dvec = nullptr, *rms = nullptr, *norm = nullptr,
              *apart = nullptr;  // attention backward's per-head dK, dV (GQA)
        double *norm_scratch = nullptr;
        int32_t *uniq = nullptr, *start = nullptr, *order = nullptr;
        int64_t n_unique = 0;
    } tr;
    bool staged_index = false;  // the embedding-backward index matches the staged ids
    float *grad = nullptr, *mom1 = nullptr, *mom2 = nullptr;
    int64_t *ranges = nullptr;  // [start, end) of the parameters without weight decay
    int nranges = 0;
    int64_t ranges_worst = 0;
    bool has_grad = false;
    bool has_opt = false;
    float beta1 = 0.9f, beta2 = 0.999f, adam_eps = 1e-8f, weight_decay = 0.0f, clip_norm = 1.0f;
    uint64_t opt_steps = 0;

    void drop_graph() {
        if (graph_exec) (void)hipGraphExecDestroy(graph_exec);
        if (graph) (void)hipGraphDestroy(graph);
        graph_exec = nullptr;
        graph = nullptr;
        graph_b = graph_t = 0;
        graph_act = graph_ws = graph_pad = nullptr;
    }

    int64_t qkv_cols() const { return cfg.d + 2 * cfg.kv(); }
    // The device layout: embed [V,d]; per block attn_norm [d], Wqkv [d, qc],
    // Wo [d,d], mlp_norm [d], Wgu [d, 2*ff_pad], Wd [ff,d]; final_norm [d];
    // lm_head [d,V] when untied.
    int64_t dev_block() const {
        const int64_t d = cfg.d;
        return 2 * d + d * qkv_cols() + d * d + 2 * d * ff_pad + cfg.ff * d;
    }
    int64_t dev_count() const {
        return cfg.vocab * cfg.d + cfg.layers * dev_block() + cfg.d +
               (cfg.tie ? 0 : cfg.d * cfg.vocab);
    }
    int64_t off_block(int64_t l) const { return cfg.vocab * cfg.d + l * dev_block(); }
    int64_t off_wqkv(int64_t l) const { return off_block(l) + cfg.d; }
    int64_t off_wo(int64_t l) const { return off_wqkv(l) + cfg.d * qkv_cols(); }
    int64_t off_mlp_norm(int64_t l) const { return off_wo(l) + cfg.d * cfg.d; }
    int64_t off_wgu(int64_t l) const { return off_mlp_norm(l) + cfg.d; }
    int64_t off_wd(int64_t l) const { return off_wgu(l) + 2 * cfg.d * ff_pad; }
    int64_t off_final_norm() const { return off_block(cfg.layers); }
    const float *embed() const { return w; }
    const float *attn_norm(int64_t l) const { return w + off_block(l); }
    const float *wqkv(int64_t l) const { return w + off_wqkv(l); }
    const float *wo(int64_t l) const { return w + off_wo(l); }
    const float *mlp_norm(int64_t l) const { return w + off_mlp_norm(l); }
    const float *wgu(int64_t l) const { return w + off_wgu(l); }
    const float *wd(int64_t l) const { return w + off_wd(l); }
    const float *final_norm() const { return w + off_final_norm(); }
    const float *lm_head() const { return final_norm() + cfg.d; }

    // Reference parameter order (docs/midman-model.md:20) <-> the device
    // layout, device to device (ref and dev are parameter-sized buffers).
    void ref_to_dev(const float *ref, float *dev) {
        const int64_t d = cfg.d, kv = cfg.kv(), ff = cfg.ff, V = cfg.vocab, qc = qkv_cols();
        auto copy = [&](float *dst, const float *src, int64_t n) {
            check_hip(hipMemcpyAsync(dst, src, (size_t)n * 4, hipMemcpyDeviceToDevice,
                                     ctx->stream),
                      "weights copy");
        };
        copy(dev, ref, V * d);
        for (int64_t l = 0; l < cfg.layers; ++l) {
            const float *r = ref + V * d + l * cfg.block_params();
            const float *an = r, *wq = an + d, *wk = wq + d * d, *wv = wk + d * kv;
            const float *wo_ = wv + d * kv, *mn = wo_ + d * d, *wg = mn + d, *wu = wg + d * ff;
            const float *wd_ = wu + d * ff;
            copy(dev + off_block(l), an, d);
            launch_pack_cols(*ctx, wq, d, d, dev + off_wqkv(l), qc, 0);
            launch_pack_cols(*ctx, wk, d, kv, dev + off_wqkv(l), qc, d);
            launch_pack_cols(*ctx, wv, d, kv, dev + off_wqkv(l), qc, d + kv);
            copy(dev + off_wo(l), wo_, d * d);
            copy(dev + off_mlp_norm(l), mn, d);
            launch_pack_gate_up(*ctx, wg, wu, d, ff, ff_pad, dev + off_wgu(l));
            copy(dev + off_wd(l), wd_, ff * d);
        }
        const float *rf = ref + V * d + cfg.layers * cfg.block_params();
        copy(dev + off_final_norm(), rf, d);
        if (!cfg.tie) copy(dev + off_final_norm() + d, rf + d, d * V);
    }
    void dev_to_ref(const float *dev, float *ref) {
        const int64_t d = cfg.d, kv = cfg.kv(), ff = cfg.ff, V = cfg.vocab, qc = qkv_cols();
        auto copy = [&](float *dst, const float *src, int64_t n) {
            check_hip(hipMemcpyAsync(dst, src, (size_t)n * 4, hipMemcpyDeviceToDevice,
                                     ctx->stream),
                      "weights copy");
        };
        copy(ref, dev, V * d);
        for (int64_t l = 0; l < cfg.layers; ++l) {
            float *r = ref + V * d + l * cfg.block_params();
            float *an = r, *wq = an + d, *wk = wq + d * d, *wv = wk + d * kv;
            float *wo_ = wv + d * kv, *mn = wo_ + d * d, *wg = mn + d, *wu = wg + d * ff;
            float *wd_ = wu + d * ff;
            copy(an, dev + off_block(l), d);
            launch_unpack_cols(*ctx, dev + off_wqkv(l), qc, 0, d, d, wq);
            launch_unpack_cols(*ctx, dev + off_wqkv(l), qc, d, d, kv, wk);
            launch_unpack_cols(*ctx, dev + off_wqkv(l), qc, d + kv, d, kv, wv);
            copy(wo_, dev + off_wo(l), d * d);
            copy(mn, dev + off_mlp_norm(l), d);
            launch_unpack_gate_up(*ctx, dev + off_wgu(l), d, ff, ff_pad, wg, wu);
            copy(wd_, dev + off_wd(l), ff * d);
        }
        float *rf = ref + V * d + cfg.layers * cfg.block_params();
        copy(rf, dev + off_final_norm(), d);
        if (!cfg.tie) copy(rf + d, dev + off_final_norm() + d, d * V);
    }

    // A temporary device buffer of n floats, freed when it goes out of scope
    // (after the stream has drained).
    struct DevTemp {
        Context *c;
        float *p = nullptr;
        DevTemp(Context *cx, int64_t n) : c(cx) {
            check_hip(hipMalloc(&p, (size_t)std::max<int64_t>(n, 1) * 4), "staging alloc");
        }
        ~DevTemp() {
            if (p) {
                (void)hipStreamSynchronize(c->stream);
                (void)hipFree(p);
            }
        }
    };

    // Weights given in the reference order on the device.
    void set_weights_from_ref(const float *ref_dev) {
        ref_to_dev(ref_dev, w);
        check_hip(hipStreamSynchronize(ctx->stream), "weights conversion sync");
    }
    // A device buffer (weights or gradients) to the host in the reference order.
    void download_ref(const float *dev, float *host) {
        DevTemp t(ctx, n_params);
        dev_to_ref(dev, t.p);
        check_hip(hipMemcpyAsync(host, t.p, (size_t)n_params * 4, hipMemcpyDeviceToHost,
                                 ctx->stream),
                  "download");
        check_hip(hipStreamSynchronize(ctx->stream), "download sync");
    }

    void release() {
        ctx->select();
        (void)hipStreamSynchronize(ctx->stream);
        drop_graph();
        for (void *p : {(void *)w, (void *)cos_t, (void *)sin_t, (void *)act, (void *)tr.mem,
                        (void *)grad, (void *)mom1, (void *)mom2, (void *)ranges,
                        (void *)fused_arena})
            if (p) (void)hipFree(p);
        w = cos_t = sin_t = act = fused_arena = nullptr;
        tr.mem = grad = mom1 = mom2 = nullptr;
        ranges = nullptr;
    }

    void ensure(int64_t n) {
        if (n <= cap) return;
        if (act) {
            check_hip(hipStreamSynchronize(ctx->stream), "sync");
            check_hip(hipFree(act), "free activations");
            // nothing points into the old buffer any more, also when the
            // allocation below fails
            act = nullptr;
            cap = 0;
            staged_n = 0;
        }
        const int64_t d = cfg.d;
        auto al = [](int64_t v) { return (v + 63) / 64 * 64; };
        // the loss folded into the head GEMM: (max, sum) per row and 128-column tile
        const int64_t ce_tiles = (cfg.vocab + 127) / 128;
        const int64_t sizes[] = {al(n * d),     al(n * d),         al(n * qkv_cols()),
                                 al(n * d),     al(n * cfg.ff),    al(n * cfg.vocab),
                                 al(n),         64,                al(n * ce_tiles * 2),
                                 al(n),         al(n),             al(n)};
        float *base[12];
        act = alloc_guarded(*ctx, sizes, 12, base, act_bands, "activation alloc");
        float **slots[] = {&x, &xn, &qkv, &cb, &h, &logits, &row_loss, &loss, &ce_part, &ce_zt};
        for (int i = 0; i < 10; ++i) *slots[i] = base[i];
        ids = reinterpret_cast<int32_t *>(base[10]);
        tgt = reinterpret_cast<int32_t *>(base[11]);
        cap = n;
        staged_n = 0;
    }

    // The rotary tables (rope.rs:71-79, f64 on the host) into HBM.
    void init_tables() {
        const size_t tab = (size_t)(cfg.max_seq * (cfg.hd() / 2));
        std::vector<float> c(tab), s(tab);
        rope_tables_host(cfg.hd(), cfg.max_seq, cfg.theta, c.data(), s.data());
        check_hip(hipMalloc(&cos_t, tab * 4), "rope alloc");
        check_hip(hipMalloc(&sin_t, tab * 4), "rope alloc");
        check_hip(hipMemcpyAsync(cos_t, c.data(), tab * 4, hipMemcpyHostToDevice, ctx->stream), "rope upload");
        check_hip(hipMemcpyAsync(sin_t, s.data(), tab * 4, hipMemcpyHostToDevice, ctx->stream), "rope upload");
        check_hip(hipStreamSynchronize(ctx->stream), "rope tables sync");
    }

    FusedShape fused_shape(int64_t batch, int64_t seq) const {
        FusedShape f;
        f.batch = batch;
        f.seq = seq;
        f.d = cfg.d;
        f.heads = cfg.heads;
        f.kv_heads = cfg.kv_heads;
        f.ff = cfg.ff;
        f.ff_pad = ff_pad;
        f.vocab = cfg.vocab;
        f.layers = cfg.layers;
        f.max_seq = cfg.max_seq;
        f.tie = cfg.tie;
        f.eps = cfg.eps;
        f.weight_floats = n_dev;
        return f;
    }
    bool use_fused(int64_t batch, int64_t seq, bool with_loss, bool want_logits) const {
        return forward_path == 0 && with_loss && !want_logits &&
               fused_forward_fits(*ctx, fused_shape(batch, seq));
    }
    // The arena laid out for (batch, seq): zeroed (counters, error word) with
    // the rotary tables copied in. Never inside a graph capture: the first
    // run of a shape is eager and prepares it.
    void ensure_fused(int64_t batch, int64_t seq) {
        if (fused_arena && fused_b == batch && fused_t == seq) return;
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        check_hip(hipStreamIsCapturing(ctx->stream, &cs), "capture status");
        if (cs != hipStreamCaptureStatusNone)
            fail(MMH_ERR_OTHER, "fused forward: arena not prepared before capture");
        const FusedLayout f = fused_layout(fused_shape(batch, seq));
        // every fill and copy below stays inside the arena, and the table
        // copies read no more than the tables hold
        const int64_t tab_have = cfg.max_seq * (cfg.hd() / 2);
        bool inside = f.nbands > 0 && f.tab_floats == tab_have && f.o_cos >= 0 &&
                      f.o_sin >= f.o_cos + f.tab_floats && f.o_sin + f.tab_floats <= f.floats &&
                      f.o_err >= 0 && f.o_err + 1 <= f.floats && f.o_ctl >= 0 &&
                      f.o_ctl + f.ctl_ints <= f.floats;
        for (int i = 0; i < f.nbands; ++i)
            inside = inside && f.bands[i] >= 0 && f.bands[i] + FusedLayout::kBand <= f.floats;
        if (!inside) fail(MMH_ERR_OTHER, "fused forward: arena layout out of bounds");
        check_hip(hipStreamSynchronize(ctx->stream), "sync");
        if (f.floats > fused_floats) {
            if (fused_arena) (void)hipFree(fused_arena);
            fused_arena = nullptr;
            fused_floats = 0;
            fused_b = fused_t = 0;
            check_hip(hipMalloc(&fused_arena, (size_t)f.floats * 4), "fused arena alloc");
            fused_floats = f.floats;
        }
        check_hip(hipMemsetAsync(fused_arena, 0, (size_t)f.floats * 4, ctx->stream), "arena clear");
        for (int i = 0; i < f.nbands; ++i)
            check_hip(hipMemsetD32Async(reinterpret_cast<hipDeviceptr_t>(fused_arena + f.bands[i]),
                                        (int)kGuardBits, (size_t)FusedLayout::kBand, ctx->stream),
                      "arena guard fill");
        const size_t tab = (size_t)f.tab_floats * 4;
        check_hip(hipMemcpyAsync(fused_arena + f.o_cos, cos_t, tab, hipMemcpyDeviceToDevice,
                                 ctx->stream),
                  "arena tables");
        check_hip(hipMemcpyAsync(fused_arena + f.o_sin, sin_t, tab, hipMemcpyDeviceToDevice,
                                 ctx->stream),
                  "arena tables");
        check_hip(hipStreamSynchronize(ctx->stream), "arena sync");
        fused_b = batch;
        fused_t = seq;
        fused_check = false;
    }
    // The error bits of the fused launches since the last check (0: none, or
    // no fused launch ran); waits for queued work. A nonzero word is cleared
    // together with the counters, so the next launch starts clean.
    int32_t take_fused_error() {
        if (!fused_check || !fused_arena) return 0;
        const FusedLayout f = fused_layout(fused_shape(fused_b, fused_t));
        int32_t e = 0;
        check_hip(hipMemcpyAsync(&e, fused_arena + f.o_err, 4, hipMemcpyDeviceToHost, ctx->stream),
                  "fused error word");
        check_hip(hipStreamSynchronize(ctx->stream), "fused error sync");
        fused_check = false;
        if (e == 0) return 0;
        check_hip(hipMemsetAsync(fused_arena + f.o_ctl, 0, (size_t)f.ctl_ints * 4, ctx->stream),
                  "fused reset");
        check_hip(hipMemsetAsync(fused_arena + f.o_err, 0, 4, ctx->stream), "fused reset");
        check_hip(hipStreamSynchronize(ctx->stream), "fused reset sync");
        return e;
    }
    // When the fused launch of the last loss-only forward (batch x seq) gave
    // up (a dependency wait past its bound: the team's workgroups were not all
    // resident at once, as when other work holds CUs), the same forward runs
    // again on the per-operation kernels from the staged ids and targets,
    // which are still in HBM; the loss buffer then holds its loss. True when
    // that happened. Waits for queued work.
    bool redo_if_fused_failed(int64_t batch, int64_t seq) {
        const int32_t e = take_fused_error();
        if (e == 0) return false;
        fused_last_error = e;
        ++fused_fallbacks;
        enqueue(batch, seq, true, false, nullptr, true);
        check_hip(hipStreamSynchronize(ctx->stream), "fused redo sync");
        return true;
    }
    // Settles a staged fused run whose loss has not been read before its ids,
    // targets or loss are replaced.
    void settle_fused() {
        if (fused_check && staged_n > 0 && staged_n == run_b * run_t && staged_targets)
            (void)redo_if_fused_failed(run_b, run_t);
        else
            (void)take_fused_error();
    }
    // The diagnostic error bits into the arena's error word, outside any
    // capture (a graph holds kernel launches only); kept pending until a
    // fused arena exists.
    void apply_fused_inject() {
        if (!fused_inject || !fused_arena) return;
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        check_hip(hipStreamIsCapturing(ctx->stream, &cs), "capture status");
        if (cs != hipStreamCaptureStatusNone) return;
        const FusedLayout f = fused_layout(fused_shape(fused_b, fused_t));
        check_hip(hipMemsetD32Async(reinterpret_cast<hipDeviceptr_t>(fused_arena + f.o_err),
                                    fused_inject, 1, ctx->stream),
                  "fused error preset");
        fused_inject = 0;
    }

    // Checks of model.rs:134-148 and the id ranges (ops_shape.rs:250-252,
    // ops_reduce.rs:250-252), then the ids go to the model's token buffers.
    void stage(const int32_t *inputs, const int32_t *targets, int64_t batch, int64_t seq) {
        if (batch <= 0 || seq <= 0)
            fail(MMH_ERR_ARGUMENT, "forward: batch and seq must be at least 1");
        if (batch > (int64_t(1) << 40) / seq)
            fail(MMH_ERR_ARGUMENT, "forward: batch x seq is too large");
        if (seq > cfg.max_seq)
            fail(MMH_ERR_ARGUMENT, "forward: sequence length " + std::to_string(seq) +
                                       " exceeds max_seq_len " + std::to_string(cfg.max_seq));
        const int64_t n = batch * seq;
        check_ids(inputs, n, cfg.vocab, "token id");
        if (targets) check_ids(targets, n, cfg.vocab, "target class");
        ctx->select();
        settle_fused();
        ensure(n);
        check_hip(hipMemcpyAsync(ids, inputs, (size_t)n * 4, hipMemcpyHostToDevice, ctx->stream),
                  "ids upload");
        if (targets)
            check_hip(hipMemcpyAsync(tgt, targets, (size_t)n * 4, hipMemcpyHostToDevice,
                                     ctx->stream),
                      "targets upload");
        staged_n = n;
        staged_targets = targets != nullptr;
        staged_index = false;
    }

    // Per-launch HIP events, summed per kernel class after the run.
    struct Prof {
        std::vector<std::pair<int, std::pair<hipEvent_t, hipEvent_t>>> marks;
    };
    template <class F>
    void timed(Prof *prof, int cls, F &&launch) {
        if (!prof) {
            launch();
            return;
        }
        hipEvent_t e0, e1;
        check_hip(hipEventCreate(&e0), "event");
        check_hip(hipEventCreate(&e1), "event");
        check_hip(hipEventRecord(e0, ctx->stream), "event record");
        launch();
        check_hip(hipEventRecord(e1, ctx->stream), "event record");
        prof->marks.push_back({cls, {e0, e1}});
    }

    // model.rs:127-165 on the staged ids, then model.rs:174-183 when with_loss.
    // Without want_logits the loss folds into the head GEMM where it can
    // (EPI_CE) and the logits are never written. Queued on the context
    // stream; nothing waits.
    void enqueue(int64_t batch, int64_t seq, bool with_loss, bool want_logits,
                 Prof *prof = nullptr, bool per_op = false) {
        const int64_t n = batch * seq;
        if (n != staged_n || n > cap)
            fail(MMH_ERR_ARGUMENT, "no tokens staged for batch " + std::to_string(batch) +
                                       " x seq " + std::to_string(seq));
        if (seq > cfg.max_seq) fail(MMH_ERR_ARGUMENT, "forward: sequence length exceeds max_seq_len");
        if (with_loss && !staged_targets) fail(MMH_ERR_ARGUMENT, "no targets staged");
        Context &c = *ctx;
        const int64_t d = cfg.d, V = cfg.vocab;
        last_fused = !prof && !per_op && use_fused(batch, seq, with_loss, want_logits);
        if (last_fused) {
            ensure_fused(batch, seq);
            apply_fused_inject();
            FusedArgs fa;
            fa.shape = fused_shape(batch, seq);
            fa.w = w;
            fa.off_block0 = off_block(0);
            fa.block_floats = dev_block();
            fa.off_final_norm = off_final_norm();
            fa.ids = ids;
            fa.tgt = tgt;
            fa.loss = loss;
            fa.arena = fused_arena;
            fa.stamps = fused_stamps;
            launch_fused_forward(c, fa);
            fused_check = true;
            return;
        }
        timed(prof, MMH_PROF_EMBEDDING, [&] { launch_embedding(c, embed(), d, ids, n, x); });
        BlockRun r;
        r.cos_t = cos_t;
        r.sin_t = sin_t;
        r.x = x;
        r.xn = xn;
        r.qkv = qkv;
        r.cb = cb;
        r.h = h;
        r.batch = batch;
        r.seq = seq;
        r.d = d;
        r.heads = cfg.heads;
        r.kv_heads = cfg.kv_heads;
        r.ff = cfg.ff;
        r.ff_pad = ff_pad;
        r.eps = cfg.eps;
        for (int64_t l = 0; l < cfg.layers; ++l) {
            r.attn_norm = attn_norm(l);
            r.wqkv = wqkv(l);
            r.wo = wo(l);
            r.mlp_norm = mlp_norm(l);
            r.wgu = wgu(l);
            r.wd = wd(l);
            enqueue_block(c, r, [&](int cls, auto &&launch) { timed(prof, cls, launch); });
        }
        timed(prof, MMH_PROF_RMS_NORM,
              [&] { launch_rms_norm(c, x, final_norm(), n, d, cfg.eps, xn); });
        GemmDesc hg;
        hg.a = xn;
        hg.c = logits;
        hg.m = n;
        hg.k = d;
        hg.n = V;
        hg.lda = d;
        hg.ldc = V;
        if (cfg.tie) {  // x . E^T with E [V, d] read in place
            hg.b = embed();
            hg.tb = true;
            hg.ldb = d;
        } else {
            hg.b = lm_head();
            hg.ldb = V;
        }
        const int64_t ce_tiles = with_loss && !want_logits ? gemm_ce_tiles(c, hg) : 0;
        if (ce_tiles > 0) {
            hg.epi = EPI_CE;
            hg.ce_targets = tgt;
            hg.ce_part = ce_part;
            hg.ce_zt = ce_zt;
            timed(prof, MMH_PROF_GEMM_HEAD, [&] { gemm(c, hg); });
            timed(prof, MMH_PROF_LOSS,
                  [&] { launch_ce_combine(c, ce_part, ce_tiles, ce_zt, n, row_loss, loss); });
            return;
        }
        timed(prof, MMH_PROF_GEMM_HEAD, [&] { gemm(c, hg); });
        if (with_loss)
            timed(prof, MMH_PROF_LOSS,
                  [&] { launch_cross_entropy(c, logits, tgt, n, V, row_loss, loss); });
    }

    // First call for a shape: eager (every workspace reaches its size). Second:
    // capture the same launches into a graph. Later calls replay the graph.
    // The graph holds no memset or allocation: only kernel launches.
    void run_staged(int64_t batch, int64_t seq) {
        run_b = batch;
        run_t = seq;
        // The fused forward is one kernel: it is launched directly every time
        // (a graph around one launch only added to the time between
        // launches: 0.1664 -> 0.1615 ms per tiny step).
        if (use_fused(batch, seq, true, false)) {
            drop_graph();
            enqueue(batch, seq, true, false);
            warm_b = warm_t = 0;
            warm_act = nullptr;
            return;
        }
        if (graph_exec && graph_b == batch && graph_t == seq && graph_act == act &&
            graph_ws == ctx->ws[0] && graph_pad == ctx->ws[Context::kPadSlot] &&
            staged_n == batch * seq && staged_targets) {
            check_hip(hipGraphLaunch(graph_exec, ctx->stream), "graph launch");
            last_fused = false;
            return;
        }
        // eager first for a new shape or new activations
        if (!(warm_b == batch && warm_t == seq && warm_act == act)) {
            enqueue(batch, seq, true, false);
            warm_b = batch;
            warm_t = seq;
            warm_act = act;
            return;
        }
        drop_graph();
        check_hip(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal), "capture");
        try {
            enqueue(batch, seq, true, false);
        } catch (...) {
            hipGraph_t g = nullptr;
            (void)hipStreamEndCapture(ctx->stream, &g);
            if (g) (void)hipGraphDestroy(g);
            throw;
        }
        check_hip(hipStreamEndCapture(ctx->stream, &graph), "end capture");
        check_hip(hipGraphInstantiate(&graph_exec, graph, nullptr, nullptr, 0), "instantiate");
        graph_b = batch;
        graph_t = seq;
        graph_act = act;
        graph_ws = ctx->ws[0];
        graph_pad = ctx->ws[Context::kPadSlot];
        check_hip(hipGraphLaunch(graph_exec, ctx->stream), "graph launch");
    }

    // The fused launch's own duration: `reps` eager launches on the staged ids,
    // back to back, each workgroup stamping the device's constant-rate clock
    // at its start and end; per launch, last end - first start. Fills the
    // median and the minimum in microseconds.
    void fused_duration(int64_t batch, int64_t seq, int reps, float *median_us, float *min_us) {
        if (reps < 1 || reps > 100000) fail(MMH_ERR_ARGUMENT, "reps must be 1 to 100000");
        if (staged_n != batch * seq || staged_n == 0 || !staged_targets)
            fail(MMH_ERR_ARGUMENT, "no tokens and targets staged for batch " +
                                       std::to_string(batch) + " x seq " + std::to_string(seq));
        if (!use_fused(batch, seq, true, false))
            fail(MMH_ERR_ARGUMENT, "the fused launch does not take this model and shape");
        settle_fused();
        int khz = 0;
        check_hip(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, ctx->device),
                  "wall clock rate");
        if (khz <= 0) fail(MMH_ERR_DEVICE, "the device reports no wall clock rate");
        const size_t per = 2 * (size_t)ctx->cu_count;
        std::vector<uint64_t> h((size_t)reps * per);
        uint64_t *st = nullptr;
        check_hip(hipMalloc(&st, h.size() * 8), "stamps alloc");
        try {
            for (int r = 0; r < reps; ++r) {
                fused_stamps = st + (size_t)r * per;
                enqueue(batch, seq, true, false);
            }
            fused_stamps = nullptr;
            check_hip(hipMemcpyAsync(h.data(), st, h.size() * 8, hipMemcpyDeviceToHost, ctx->stream),
                      "stamps download");
            check_hip(hipStreamSynchronize(ctx->stream), "stamps sync");
        } catch (...) {
            fused_stamps = nullptr;
            (void)hipStreamSynchronize(ctx->stream);
            (void)hipFree(st);
            throw;
        }
        (void)hipFree(st);
        run_b = batch;
        run_t = seq;
        if (redo_if_fused_failed(batch, seq))
            fail(MMH_ERR_DEVICE, "a timed fused launch gave up (error bits " +
                                     std::to_string(fused_last_error) +
                                     "): its duration is not the kernel's");
        std::vector<double> span((size_t)reps);
        for (int r = 0; r < reps; ++r) {
            uint64_t lo = UINT64_MAX, hi = 0;
            for (size_t g = 0; g < per; g += 2) {
                lo = std::min(lo, h[(size_t)r * per + g]);
                hi = std::max(hi, h[(size_t)r * per + g + 1]);
            }
            span[(size_t)r] = hi > lo ? (double)(hi - lo) * 1000.0 / (double)khz : 0.0;
        }
        std::sort(span.begin(), span.end());
        *median_us = (float)span[span.size() / 2];
        if (min_us) *min_us = (float)span[0];
    }

    // The loss of the last staged run (read_loss): a fused run that gave up is
    // redone on the per-operation kernels first.
    void read_staged_loss(float *out) {
        check_hip(hipMemcpyAsync(out, loss, 4, hipMemcpyDeviceToHost, ctx->stream), "loss download");
        check_hip(hipStreamSynchronize(ctx->stream), "loss sync");
        if (staged_n > 0 && staged_n == run_b * run_t && staged_targets &&
            redo_if_fused_failed(run_b, run_t)) {
            check_hip(hipMemcpyAsync(out, loss, 4, hipMemcpyDeviceToHost, ctx->stream),
                      "loss download");
            check_hip(hipStreamSynchronize(ctx->stream), "loss sync");
        } else {
            (void)take_fused_error();
        }
    }

    void run(const int32_t *inputs, const int32_t *targets, int64_t batch, int64_t seq,
             float *logits_out, float *loss_out) {
        stage(inputs, loss_out ? targets : nullptr, batch, seq);
        enqueue(batch, seq, loss_out != nullptr, logits_out != nullptr);
        Context &c = *ctx;
        if (loss_out)
            check_hip(hipMemcpyAsync(loss_out, loss, 4, hipMemcpyDeviceToHost, c.stream),
                      "loss download");
        if (logits_out)
            check_hip(hipMemcpyAsync(logits_out, logits, (size_t)(batch * seq * cfg.vocab) * 4,
                                     hipMemcpyDeviceToHost, c.stream),
                      "logits download");
        check_hip(hipStreamSynchronize(c.stream), "forward sync");
        run_b = batch;
        run_t = seq;
        if (redo_if_fused_failed(batch, seq) && loss_out) {
            check_hip(hipMemcpyAsync(loss_out, loss, 4, hipMemcpyDeviceToHost, c.stream),
                      "loss download");
            check_hip(hipStreamSynchronize(c.stream), "forward sync");
        }
    }

    // ---------------------------------------------------------------- training
    int64_t lse_rows(int64_t n) const { return n * cfg.heads; }

    // Saved activations and backward scratch for up to n rows. Per-layer
    // slices are cap rows apart.
    void ensure_train(int64_t n) {
        if (n <= tr.cap) return;
        if (tr.mem) {
            check_hip(hipStreamSynchronize(ctx->stream), "sync");
            check_hip(hipFree(tr.mem), "free training activations");
            tr.mem = nullptr;
            tr.cap = 0;
        }
        const int64_t d = cfg.d, L = cfg.layers, qc = qkv_cols(), ffp2 = 2 * ff_pad;
        auto al = [](int64_t v) { return (v + 63) / 64 * 64; };
        const int64_t sizes[] = {
            al((L + 1) * n * d),            // xs
            al(L * n * d),                  // xn1
            al(L * n * qc),                 // qkv
            al(L * n * d),                  // cb
            al(L * lse_rows(n)),            // lse
            al(L * n * d),                  // hres
            al(L * n * d),                  // xn2
            al(L * n * ffp2),               // gu
            al(L * n * cfg.ff),             // h
            al(n * d),                      // xnf
            al(n * d),                      // dx
            al(n * d),                      // dy
            al(n * d),                      // dxn
            al(n * d),                      // dctx
            al(n * qc),                     // dqkv
            al(lse_rows(n)),                // dvec
            al(rms_norm_backward_scratch(n, d)),  // rms
            64,                             // norm
            al(attention_backward_scratch_floats(1, cfg.heads, cfg.kv_heads, n, cfg.hd())),
            al(global_norm_scratch_bytes() / 4),  // norm_scratch (doubles)
            al(n), al(n + 1), al(n),        // uniq, start, order (int32)
        };
        constexpr int nslots = (int)(sizeof(sizes) / sizeof(sizes[0]));
        static_assert(nslots == 23, "training slots");
        float *base[nslots];
        tr.mem = alloc_guarded(*ctx, sizes, nslots, base, tr_bands, "training activation alloc");
        float **slots[] = {&tr.xs,   &tr.xn1, &tr.qkv,  &tr.cb,   &tr.lse,  &tr.hres, &tr.xn2,
                           &tr.gu,   &tr.h,   &tr.xnf,  &tr.dx,   &tr.dy,   &tr.dxn,  &tr.dctx,
                           &tr.dqkv, &tr.dvec, &tr.rms, &tr.norm, &tr.apart};
        for (int i = 0; i < 19; ++i) *slots[i] = base[i];
        tr.norm_scratch = reinterpret_cast<double *>(base[19]);
        tr.uniq = reinterpret_cast<int32_t *>(base[20]);
        tr.start = reinterpret_cast<int32_t *>(base[21]);
        tr.order = reinterpret_cast<int32_t *>(base[22]);
        tr.cap = n;
        staged_index = false;
    }

    // Stages ids and targets (stage()) and the embedding-backward index: the
    // distinct ids in ascending order, and for each the positions holding it
    // in ascending order (a counting sort).
    void stage_train(const int32_t *inputs, const int32_t *targets, int64_t batch, int64_t seq) {
        if (!targets) fail(MMH_ERR_ARGUMENT, "training needs targets");
        stage(inputs, targets, batch, seq);
        const int64_t n = batch * seq;
        ensure_train(n);
        std::vector<int32_t> count((size_t)cfg.vocab + 1, 0);
        for (int64_t i = 0; i < n; ++i) count[(size_t)inputs[i] + 1]++;
        std::vector<int32_t> uniq, start, order((size_t)n);
        uniq.reserve((size_t)n);
        start.reserve((size_t)n + 1);
        std::vector<int32_t> at((size_t)cfg.vocab, 0);
        int32_t run = 0;
        for (int64_t v = 0; v < cfg.vocab; ++v) {
            const int32_t c = count[(size_t)v + 1];
            if (c) {
                uniq.push_back((int32_t)v);
                start.push_back(run);
            }
            at[(size_t)v] = run;
            run += c;
        }
        start.push_back(run);
        for (int64_t i = 0; i < n; ++i) order[(size_t)at[(size_t)inputs[i]]++] = (int32_t)i;
        tr.n_unique = (int64_t)uniq.size();
        // The copies run on the stream before this function returns; the
        // vectors are synchronised below so the host memory outlives them.
        check_hip(hipMemcpyAsync(tr.uniq, uniq.data(), uniq.size() * 4, hipMemcpyHostToDevice,
                                 ctx->stream), "index upload");
        check_hip(hipMemcpyAsync(tr.start, start.data(), start.size() * 4, hipMemcpyHostToDevice,
                                 ctx->stream), "index upload");
        check_hip(hipMemcpyAsync(tr.order, order.data(), order.size() * 4, hipMemcpyHostToDevice,
                                 ctx->stream), "index upload");
        check_hip(hipStreamSynchronize(ctx->stream), "index upload sync");
        staged_index = true;
    }

    float *grad_of(const float *param) { return grad + (param - w); }

    GemmDesc desc(const float *a, bool ta, int64_t lda, const float *b, bool tb, int64_t ldb,
                  float *c, int64_t ldc, int64_t m, int64_t k, int64_t n) const {
        GemmDesc g;
        g.a = a;
        g.ta = ta;
        g.lda = lda;
        g.b = b;
        g.tb = tb;
        g.ldb = ldb;
        g.c = c;
        g.ldc = ldc;
        g.m = m;
        g.k = k;
        g.n = n;
        return g;
    }

    // Forward keeping what the backward reads, the loss, and dlogits in place.
    void enqueue_train_forward(int64_t batch, int64_t seq) {
        const int64_t n = batch * seq;
        Context &c = *ctx;
        const int64_t d = cfg.d, kv = cfg.kv(), hd = cfg.hd(), V = cfg.vocab, qc = qkv_cols();
        const int64_t cap = tr.cap, ffp2 = 2 * ff_pad;
        launch_embedding(c, embed(), d, ids, n, tr.xs);
        for (int64_t l = 0; l < cfg.layers; ++l) {
            float *x = tr.xs + l * cap * d, *xn1 = tr.xn1 + l * cap * d;
            float *qkvl = tr.qkv + l * cap * qc, *cbl = tr.cb + l * cap * d;
            float *hres = tr.hres + l * cap * d, *xn2 = tr.xn2 + l * cap * d;
            float *gu = tr.gu + l * cap * ffp2, *hl = tr.h + l * cap * cfg.ff;
            float *xnext = tr.xs + (l + 1) * cap * d;
            launch_rms_norm(c, x, attn_norm(l), n, d, cfg.eps, xn1);
            // q, k rotated by the QKV GEMM (in its epilogue or right after it)
            GemmDesc q = desc(xn1, false, d, wqkv(l), false, qc, qkvl, qc, n, d, qc);
            q.rope_cos = cos_t;
            q.rope_sin = sin_t;
            q.rope_seq = seq;
            q.rope_hd = hd;
            q.rope_cols = d + kv;
            gemm(c, q);
            AttnDesc a{};
            a.q = qkvl;
            a.k = qkvl + d;
            a.v = qkvl + d + kv;
            a.out = cbl;
            a.sqb = a.skb = a.svb = seq * qc;
            a.sqh = a.skh = a.svh = hd;
            a.sqt = a.skt = a.svt = qc;
            a.sob = seq * d;
            a.soh = hd;
            a.sot = d;
            a.b = batch;
            a.h = cfg.heads;
            a.hkv = cfg.kv_heads;
            a.t = seq;
            a.hd = hd;
            a.lse = tr.lse + l * lse_rows(cap);
            attention(c, a);
            GemmDesc o = desc(cbl, false, d, wo(l), false, d, hres, d, n, d, d);
            o.epi = EPI_ACCUM;
            o.resid = x;
            gemm(c, o);
            launch_rms_norm(c, hres, mlp_norm(l), n, d, cfg.eps, xn2);
            GemmDesc gg = desc(xn2, false, d, wgu(l), false, ffp2, hl, cfg.ff, n, d, ffp2);
            gg.epi = EPI_SWIGLU;
            gg.swiglu_ff = cfg.ff;
            gg.aux = gu;
            gg.ldaux = ffp2;
            gemm(c, gg);
            GemmDesc dn = desc(hl, false, cfg.ff, wd(l), false, d, xnext, d, n, cfg.ff, d);
            dn.epi = EPI_ACCUM;
            dn.resid = hres;
            gemm(c, dn);
        }
        launch_rms_norm(c, tr.xs + cfg.layers * cap * d, final_norm(), n, d, cfg.eps, tr.xnf);
        if (cfg.tie)
            gemm(c, desc(tr.xnf, false, d, embed(), true, d, logits, V, n, d, V));
        else
            gemm(c, desc(tr.xnf, false, d, lm_head(), false, V, logits, V, n, d, V));
        launch_cross_entropy_fwd_bwd(c, logits, tgt, n, V, 1.0f, row_loss, loss);
    }

    // Every parameter gradient into grad (reference order), from dlogits.
    void enqueue_backward(int64_t batch, int64_t seq) {
        const int64_t n = batch * seq;
        Context &c = *ctx;
        const int64_t d = cfg.d, kv = cfg.kv(), hd = cfg.hd(), V = cfg.vocab, qc = qkv_cols();
        const int64_t cap = tr.cap, ffp2 = 2 * ff_pad, ff = cfg.ff;
        // head: logits = xnf . E^T (tied) or xnf . W_head
        if (cfg.tie) {
            gemm(c, desc(logits, false, V, embed(), false, d, tr.dy, d, n, V, d));
            gemm(c, desc(logits, true, V, tr.xnf, false, d, grad, d, V, n, d));
        } else {
            gemm(c, desc(logits, false, V, lm_head(), true, V, tr.dy, d, n, V, d));
            gemm(c, desc(tr.xnf, true, d, logits, false, V, grad_of(lm_head()), V, d, n, V));
        }
        launch_rms_norm_backward(c, tr.xs + cfg.layers * cap * d, final_norm(), tr.dy, n, d,
                                 cfg.eps, tr.dx, false, grad_of(final_norm()), tr.rms);
        for (int64_t l = cfg.layers - 1; l >= 0; --l) {
            float *x = tr.xs + l * cap * d, *xn1 = tr.xn1 + l * cap * d;
            float *qkvl = tr.qkv + l * cap * qc, *cbl = tr.cb + l * cap * d;
            float *hres = tr.hres + l * cap * d, *xn2 = tr.xn2 + l * cap * d;
            float *gu = tr.gu + l * cap * ffp2, *hl = tr.h + l * cap * ff;
            // MLP: y = hres + h . Wd, h = silu(gate) * up
            GemmDesc dh = desc(tr.dx, false, d, wd(l), true, d, gu, ffp2, n, d, ff);
            dh.epi = EPI_SWIGLU_BWD;
            dh.aux = gu;
            dh.ldaux = ffp2;
            gemm(c, dh);  // gu now holds (dgate, dup) pairs
            gemm(c, desc(hl, true, ff, tr.dx, false, d, grad_of(wd(l)), d, ff, n, d));
            gemm(c, desc(gu, false, ffp2, wgu(l), true, ffp2, tr.dxn, d, n, ffp2, d));
            // the packed (gate, up) gradient straight into its place (columns
            // past ff: zero pre-activations, so zero gradients)
            gemm(c, desc(xn2, true, d, gu, false, ffp2, grad_of(wgu(l)), ffp2, d, n, ffp2));
            launch_rms_norm_backward(c, hres, mlp_norm(l), tr.dxn, n, d, cfg.eps, tr.dx, true,
                                     grad_of(mlp_norm(l)), tr.rms);
            // attention: hres = x + ctx . Wo
            gemm(c, desc(tr.dx, false, d, wo(l), true, d, tr.dctx, d, n, d, d));
            gemm(c, desc(cbl, true, d, tr.dx, false, d, grad_of(wo(l)), d, d, n, d));
            AttnBwdDesc ab{};
            ab.q = qkvl;
            ab.k = qkvl + d;
            ab.v = qkvl + d + kv;
            ab.o = cbl;
            ab.dout = tr.dctx;
            ab.lse = tr.lse + l * lse_rows(cap);
            ab.dq = tr.dqkv;
            ab.dk = tr.dqkv + d;
            ab.dv = tr.dqkv + d + kv;
            ab.dvec = tr.dvec;
            ab.sqb = ab.skb = ab.svb = seq * qc;
            ab.sqh = ab.skh = ab.svh = hd;
            ab.sqt = ab.skt = ab.svt = qc;
            ab.sob = seq * d;
            ab.soh = hd;
            ab.sot = d;
            ab.b = batch;
            ab.h = cfg.heads;
            ab.hkv = cfg.kv_heads;
            ab.t = seq;
            ab.hd = hd;
            ab.cos_t = cos_t;
            ab.sin_t = sin_t;
            ab.scratch = cfg.kv_heads < cfg.heads ? tr.apart : nullptr;
            attention_backward(c, ab);
            gemm(c, desc(tr.dqkv, false, qc, wqkv(l), true, qc, tr.dxn, d, n, qc, d));
            gemm(c, desc(xn1, true, d, tr.dqkv, false, qc, grad_of(wqkv(l)), qc, d, n, qc));
            launch_rms_norm_backward(c, x, attn_norm(l), tr.dxn, n, d, cfg.eps, tr.dx, true,
                                     grad_of(attn_norm(l)), tr.rms);
        }
        // embedding: the tied table already holds the head's share
        if (!cfg.tie) launch_fill(c, grad, cfg.vocab * d, 0.0f);
        launch_embedding_backward(c, tr.dx, d, tr.uniq, tr.start, tr.order, tr.n_unique, grad,
                                  true);
        (void)V;
    }

    void ensure_grad() {
        if (!grad) check_hip(hipMalloc(&grad, (size_t)n_dev * 4), "gradient alloc");
    }

    // Forward + loss + backward on the staged batch; gradients stay on the device.
    void backward_staged(int64_t batch, int64_t seq) {
        const int64_t n = batch * seq;
        if (n != staged_n || !staged_targets || !staged_index || n > tr.cap)
            fail(MMH_ERR_ARGUMENT, "no training batch staged for batch " + std::to_string(batch) +
                                       " x seq " + std::to_string(seq));
        ensure_grad();
        enqueue_train_forward(batch, seq);
        enqueue_backward(batch, seq);
        launch_global_norm(*ctx, grad, n_dev, tr.norm_scratch, tr.norm);
        has_grad = true;
    }

    void ensure_optimizer_state() {
        if (!has_opt) fail(MMH_ERR_ARGUMENT, "no optimizer set (mmh_model_set_optimizer)");
        for (float **mom : {&mom1, &mom2}) {  // each on its own: a failed second alloc
            if (*mom) continue;                // leaves the first, which stays valid
            check_hip(hipMalloc(mom, (size_t)n_dev * 4), "moment alloc");
            launch_fill(*ctx, *mom, n_dev, 0.0f);
        }
        if (!ranges) {
            // rank-1 parameters: the two norms of every block and the final norm
            std::vector<int64_t> r;
            const int64_t d = cfg.d;
            for (int64_t l = 0; l < cfg.layers; ++l) {
                const int64_t a = attn_norm(l) - w, m = mlp_norm(l) - w;
                r.insert(r.end(), {a, a + d, m, m + d});
            }
            const int64_t f = final_norm() - w;
            r.insert(r.end(), {f, f + d});
            int64_t *dev = nullptr;
            check_hip(hipMalloc(&dev, r.size() * 8), "range alloc");
            const hipError_t e1 = hipMemcpyAsync(dev, r.data(), r.size() * 8,
                                                 hipMemcpyHostToDevice, ctx->stream);
            const hipError_t e2 = e1 == hipSuccess ? hipStreamSynchronize(ctx->stream) : e1;
            if (e2 != hipSuccess) {
                (void)hipFree(dev);
                check_hip(e2, "range upload");
            }
            ranges = dev;  // set only once the ranges are on the device
            nranges = (int)(r.size() / 2);
            ranges_worst = adamw_max_ranges_per_chunk(r.data(), nranges, n_dev);
        }
    }

    // clip + AdamW at lr for optimizer step opt_steps + 1 (adamw.rs:180-188),
    // gated on the device by the loss and norm being finite. The packed
    // matrices are the weights themselves: nothing is copied afterwards.
    void enqueue_update(float lr) {
        if (!(std::isfinite(lr) && lr >= 0.0f))
            fail(MMH_ERR_ARGUMENT, "adamw: lr must be finite and not negative, got " +
                                       std::to_string(lr));
        ensure_optimizer_state();
        const double t = (double)(opt_steps + 1);
        AdamArgs a;
        a.lr = lr;
        a.beta1 = beta1;
        a.beta2 = beta2;
        a.eps = adam_eps;
        a.weight_decay = weight_decay;
        a.clip_norm = clip_norm;
        const float bias1 = (float)(1.0 - std::pow((double)beta1, t));
        a.bias2_sqrt = (float)std::sqrt(1.0 - std::pow((double)beta2, t));
        a.step_size = lr / bias1;
        launch_adamw(*ctx, w, grad, mom1, mom2, n_dev, ranges, nranges, ranges_worst, a, loss,
                     tr.norm);
    }

    // Guard words of the activation blocks that no longer hold kGuardBits.
    uint64_t count_broken_guards() {
        check_hip(hipStreamSynchronize(ctx->stream), "guard check sync");
        uint64_t broken = 0;
        std::vector<uint32_t> host((size_t)kGuardFloats);
        std::vector<float *> arena_bands;
        if (fused_arena) {
            const FusedLayout f = fused_layout(fused_shape(fused_b, fused_t));
            for (int i = 0; i < f.nbands; ++i) arena_bands.push_back(fused_arena + f.bands[i]);
        }
        static_assert(FusedLayout::kBand == kGuardFloats, "one guard band size");
        for (const auto *bands : {&act_bands, &tr_bands, &arena_bands})
            for (float *b : *bands) {
                check_hip(hipMemcpy(host.data(), b, (size_t)kGuardFloats * 4,
                                    hipMemcpyDeviceToHost),
                          "guard download");
                for (uint32_t v : host) broken += v != kGuardBits;
            }
        return broken;
    }

    // Reads the loss and the norm; true when both are finite.
    bool read_step(float *loss_out, float *norm_out) {
        float host[2];
        check_hip(hipMemcpyAsync(&host[0], loss, 4, hipMemcpyDeviceToHost, ctx->stream),
                  "loss download");
        check_hip(hipMemcpyAsync(&host[1], tr.norm, 4, hipMemcpyDeviceToHost, ctx->stream),
                  "norm download");
        check_hip(hipStreamSynchronize(ctx->stream), "step sync");
        if (loss_out) *loss_out = host[0];
        if (norm_out) *norm_out = host[1];
        return std::isfinite(host[0]) && std::isfinite(host[1]);
    }

    // Lab::step_once / Trainer::update on the staged batch. Returns false (and
    // changes nothing) when the loss or the gradient norm is not finite.
    bool train_staged(int64_t batch, int64_t seq, float lr, float *loss_out, float *norm_out) {
        ensure_optimizer_state();
        if (!(std::isfinite(lr) && lr >= 0.0f))
            fail(MMH_ERR_ARGUMENT, "adamw: lr must be finite and not negative");
        backward_staged(batch, seq);
        enqueue_update(lr);
        const bool ok = read_step(loss_out, norm_out);
        if (ok) ++opt_steps;
        return ok;
    }
};

std::mutex g_models_mutex;
std::vector<std::unique_ptr<Model>> g_models;  // handle = index + 1

Model &model(mmh_handle h) {
    std::lock_guard<std::mutex> lock(g_models_mutex);
    if (h <= 0 || (size_t)h > g_models.size() || !g_models[(size_t)h - 1])
        fail(MMH_ERR_ARGUMENT, "invalid model handle " + std::to_string(h));
    Model &m = *g_models[(size_t)h - 1];
    (void)context(m.ctx_handle);  // the context must still exist
    return m;
}

mmh_handle register_model(std::unique_ptr<Model> m) {
    std::lock_guard<std::mutex> lock(g_models_mutex);
    g_models.push_back(std::move(m));
    return (mmh_handle)g_models.size();
}

std::unique_ptr<Model> new_model(mmh_handle ctx, const double *config) {
    auto m = std::make_unique<Model>();
    m->ctx_handle = ctx;
    m->ctx = &context(ctx);
    m->cfg = parse_config(config);
    m->n_params = m->cfg.param_count();
    m->ff_pad = (m->cfg.ff + 31) / 32 * 32;
    m->n_dev = m->dev_count();
    check_hip(hipMalloc(&m->w, (size_t)m->n_dev * 4), "weights alloc");
    try {
        // zero padding (Wgu's columns past ff) before any conversion fills the rest
        launch_fill(*m->ctx, m->w, m->n_dev, 0.0f);
        m->init_tables();
    } catch (...) {
        m->release();
        throw;
    }
    return m;
}

// Runs fill(m) on a model not yet registered; on any failure the model's
// device memory is released before the error propagates (a Model frees
// nothing by itself: its memory goes back through release()).
template <class F>
void fill_or_release(Model &m, F &&fill) {
    try {
        fill(m);
    } catch (...) {
        m.release();
        throw;
    }
}

}  // namespace

void release_models_of(mmh_handle ctx) {
    std::vector<std::unique_ptr<Model>> dead;
    {
        std::lock_guard<std::mutex> lock(g_models_mutex);
        for (auto &m : g_models)
            if (m && m->ctx_handle == ctx) dead.push_back(std::move(m));
    }
    for (auto &m : dead) {
        m->drop_graph();
        for (void *p : {(void *)m->w, (void *)m->cos_t, (void *)m->sin_t, (void *)m->act,
                        (void *)m->tr.mem, (void *)m->grad, (void *)m->mom1, (void *)m->mom2,
                        (void *)m->ranges})
            if (p) (void)hipFree(p);
    }
}

}  // namespace mmh

using namespace mmh;

extern "C" {

int32_t mmh_model_create(mmh_handle ctx, const double config[10], const float *weights_host,
                         int64_t n_weights, mmh_handle *out_model) {
    return guard([&] {
        if (!out_model) fail(MMH_ERR_ARGUMENT, "out_model is a null pointer");
        if (!weights_host) fail(MMH_ERR_ARGUMENT, "weights is a null pointer");
        auto m = new_model(ctx, config);
        fill_or_release(*m, [&](Model &mm) {
            if (n_weights != mm.n_params)
                fail(MMH_ERR_SHAPE, "the config has " + std::to_string(mm.n_params) +
                                        " parameters but " + std::to_string(n_weights) +
                                        " weights were given");
            Model::DevTemp ref(mm.ctx, mm.n_params);
            check_hip(hipMemcpyAsync(ref.p, weights_host, (size_t)n_weights * 4,
                                     hipMemcpyHostToDevice, mm.ctx->stream),
                      "weights upload");
            mm.set_weights_from_ref(ref.p);
        });
        *out_model = register_model(std::move(m));
        return MMH_OK;
    });
}

int32_t mmh_model_create_seeded(mmh_handle ctx, const double config[10], uint64_t seed,
                                float std_, mmh_handle *out_model) {
    return guard([&] {
        if (!out_model) fail(MMH_ERR_ARGUMENT, "out_model is a null pointer");
        if (!(std::isfinite(std_) && std_ > 0.f))
            fail(MMH_ERR_ARGUMENT, "init std must be positive and finite");
        auto m = new_model(ctx, config);
        fill_or_release(*m, [&](Model &mm) {
            const Config &c = mm.cfg;
            // model.rs:51-83 draw order; norms are ones (norm.rs:60).
            std::vector<float> host((size_t)mm.n_params);
            HostRng rng = HostRng::seed(seed);
            const float out_std = std_ / std::sqrt(2.0f * (float)c.layers);  // init.rs:38
            const int64_t d = c.d, kv = c.kv(), ff = c.ff;
            float *p = host.data();
            auto ones = [&](int64_t n) {
                std::fill(p, p + n, 1.0f);
                p += n;
            };
            auto draw = [&](int64_t n, float s) {
                randn_parallel(rng, p, n, s);
                p += n;
            };
            draw(c.vocab * d, std_);
            for (int64_t l = 0; l < c.layers; ++l) {
                ones(d);
                draw(d * d, std_);
                draw(d * kv, std_);
                draw(d * kv, std_);
                draw(d * d, out_std);
                ones(d);
                draw(d * ff, std_);
                draw(d * ff, std_);
                draw(ff * d, out_std);
            }
            ones(d);
            if (!c.tie) draw(d * c.vocab, std_);
            if (p - host.data() != mm.n_params) fail(MMH_ERR_OTHER, "init: parameter count mismatch");
            {
                Model::DevTemp ref(mm.ctx, mm.n_params);
                check_hip(hipMemcpyAsync(ref.p, host.data(), host.size() * 4, hipMemcpyHostToDevice,
                                         mm.ctx->stream),
                          "weights upload");
                mm.set_weights_from_ref(ref.p);
            }
            mm.rng = rng;
            mm.has_rng = true;
        });
        *out_model = register_model(std::move(m));
        return MMH_OK;
    });
}

int32_t mmh_model_lab_tokens(mmh_handle model_h, int64_t batch, int64_t seq, int32_t *inputs,
                             int32_t *targets) {
    return guard([&] {
        Model &m = model(model_h);
        if (!inputs || !targets) fail(MMH_ERR_ARGUMENT, "inputs/targets is a null pointer");
        if (batch <= 0 || seq <= 0) fail(MMH_ERR_ARGUMENT, "batch and seq must be at least 1");
        if (!m.has_rng) fail(MMH_ERR_ARGUMENT, "the model was not created from a seed");
        std::vector<int32_t> tok((size_t)seq + 1);
        for (int64_t b = 0; b < batch; ++b) {  // lab.rs:198-202
            for (int64_t i = 0; i <= seq; ++i) tok[(size_t)i] = (int32_t)m.rng.below((uint64_t)m.cfg.vocab);
            std::memcpy(inputs + b * seq, tok.data(), (size_t)seq * 4);
            std::memcpy(targets + b * seq, tok.data() + 1, (size_t)seq * 4);
        }
        return MMH_OK;
    });
}

int32_t mmh_model_param_count(mmh_handle model_h, int64_t *out) {
    return guard([&] {
        if (!out) fail(MMH_ERR_ARGUMENT, "out is a null pointer");
        *out = model(model_h).n_params;
        return MMH_OK;
    });
}

int32_t mmh_model_download_weights(mmh_handle model_h, float *out_host, int64_t n) {
    return guard([&] {
        Model &m = model(model_h);
        if (!out_host) fail(MMH_ERR_ARGUMENT, "out is a null pointer");
        if (n != m.n_params) fail(MMH_ERR_SHAPE, "weights: wrong count");
        m.download_ref(m.w, out_host);
        return MMH_OK;
    });
}

int32_t mmh_model_forward(mmh_handle model_h, const int32_t *ids_host, int64_t batch,
                          int64_t seq, float *logits_host) {
    return guard([&] {
        if (!logits_host) fail(MMH_ERR_ARGUMENT, "logits is a null pointer");
        model(model_h).run(ids_host, nullptr, batch, seq, logits_host, nullptr);
        return MMH_OK;
    });
}

int32_t mmh_model_loss(mmh_handle model_h, const int32_t *inputs_host,
                       const int32_t *targets_host, int64_t batch, int64_t seq,
                       float *loss_host) {
    return guard([&] {
        if (!loss_host) fail(MMH_ERR_ARGUMENT, "loss is a null pointer");
        model(model_h).run(inputs_host, targets_host, batch, seq, nullptr, loss_host);
        return MMH_OK;
    });
}

int32_t mmh_model_forward_loss(mmh_handle model_h, const int32_t *inputs_host,
                               const int32_t *targets_host, int64_t batch, int64_t seq,
                               float *logits_host, float *loss_host) {
    return guard([&] {
        if (!loss_host) fail(MMH_ERR_ARGUMENT, "loss is a null pointer");
        model(model_h).run(inputs_host, targets_host, batch, seq, logits_host, loss_host);
        return MMH_OK;
    });
}

int32_t mmh_model_stage(mmh_handle model_h, const int32_t *inputs_host,
                        const int32_t *targets_host, int64_t batch, int64_t seq) {
    return guard([&] {
        Model &m = model(model_h);
        m.stage(inputs_host, targets_host, batch, seq);
        check_hip(hipStreamSynchronize(m.ctx->stream), "stage sync");
        return MMH_OK;
    });
}

int32_t mmh_model_run_staged(mmh_handle model_h, int64_t batch, int64_t seq) {
    return guard([&] {
        Model &m = model(model_h);
        m.run_staged(batch, seq);
        return MMH_OK;
    });
}

int32_t mmh_model_read_loss(mmh_handle model_h, float *loss_host) {
    return guard([&] {
        if (!loss_host) fail(MMH_ERR_ARGUMENT, "loss is a null pointer");
        Model &m = model(model_h);
        if (!m.loss) fail(MMH_ERR_ARGUMENT, "nothing has run on this model");
        m.ctx->select();
        m.read_staged_loss(loss_host);
        return MMH_OK;
    });
}

int32_t mmh_model_fused_fallbacks(mmh_handle model_h, int64_t *redone, int32_t *last_error) {
    return guard([&] {
        if (!redone) fail(MMH_ERR_ARGUMENT, "redone is a null pointer");
        const Model &m = model(model_h);
        *redone = m.fused_fallbacks;
        if (last_error) *last_error = m.fused_last_error;
        return MMH_OK;
    });
}

int32_t mmh_model_fused_duration(mmh_handle model_h, int64_t batch, int64_t seq, int32_t reps,
                                 float *median_us, float *min_us) {
    return guard([&] {
        if (!median_us) fail(MMH_ERR_ARGUMENT, "median_us is a null pointer");
        Model &m = model(model_h);
        m.ctx->select();
        m.fused_duration(batch, seq, reps, median_us, min_us);
        return MMH_OK;
    });
}

int32_t mmh_model_inject_fused_error(mmh_handle model_h, int32_t bits) {
    return guard([&] {
        if (bits <= 0) fail(MMH_ERR_ARGUMENT, "the injected error bits must be positive");
        model(model_h).fused_inject = bits;
        return MMH_OK;
    });
}

int32_t mmh_model_set_forward_path(mmh_handle model_h, int32_t path) {
    return guard([&] {
        if (path != MMH_PATH_AUTO && path != MMH_PATH_PER_OP)
            fail(MMH_ERR_ARGUMENT, "forward path must be MMH_PATH_AUTO or MMH_PATH_PER_OP");
        Model &m = model(model_h);
        if (m.forward_path != path) {
            m.ctx->select();
            (void)hipStreamSynchronize(m.ctx->stream);
            m.drop_graph();
            m.warm_b = m.warm_t = 0;
            m.warm_act = nullptr;
            m.forward_path = path;
        }
        return MMH_OK;
    });
}

int32_t mmh_model_last_forward_fused(mmh_handle model_h, int32_t *fused) {
    return guard([&] {
        if (!fused) fail(MMH_ERR_ARGUMENT, "fused is null");
        *fused = model(model_h).last_fused ? 1 : 0;
        return MMH_OK;
    });
}

int32_t mmh_model_profile(mmh_handle model_h, int64_t batch, int64_t seq, float *class_ms,
                          int32_t *class_launches) {
    return guard([&] {
        if (!class_ms || !class_launches) fail(MMH_ERR_ARGUMENT, "output arrays are null");
        Model &m = model(model_h);
        Model::Prof prof;
        struct Cleanup {
            Model::Prof &p;
            ~Cleanup() {
                for (auto &mk : p.marks) {
                    (void)hipEventDestroy(mk.second.first);
                    (void)hipEventDestroy(mk.second.second);
                }
            }
        } cleanup{prof};
        check_hip(hipStreamSynchronize(m.ctx->stream), "profile sync");
        m.enqueue(batch, seq, true, false, &prof);
        check_hip(hipStreamSynchronize(m.ctx->stream), "profile sync");
        for (int i = 0; i < MMH_PROF_CLASSES; ++i) {
            class_ms[i] = 0.0f;
            class_launches[i] = 0;
        }
        for (auto &mk : prof.marks) {
            float ms = 0.0f;
            check_hip(hipEventElapsedTime(&ms, mk.second.first, mk.second.second), "elapsed");
            class_ms[mk.first] += ms;
            class_launches[mk.first] += 1;
        }
        return MMH_OK;
    });
}

int32_t mmh_model_backward(mmh_handle model_h, const int32_t *inputs_host,
                           const int32_t *targets_host, int64_t batch, int64_t seq,
                           float *loss_host) {
    return guard([&] {
        Model &m = model(model_h);
        m.stage_train(inputs_host, targets_host, batch, seq);
        m.backward_staged(batch, seq);
        m.read_step(loss_host, nullptr);
        return MMH_OK;
    });
}

int32_t mmh_model_download_grads(mmh_handle model_h, float *out_host, int64_t n) {
    return guard([&] {
        Model &m = model(model_h);
        if (!out_host) fail(MMH_ERR_ARGUMENT, "out is a null pointer");
        if (!m.has_grad) fail(MMH_ERR_ARGUMENT, "no gradients yet: run mmh_model_backward first");
        if (n != m.n_params) fail(MMH_ERR_SHAPE, "gradients: wrong count");
        m.download_ref(m.grad, out_host);
        return MMH_OK;
    });
}

int32_t mmh_model_grad_norm(mmh_handle model_h, float *norm_host) {
    return guard([&] {
        Model &m = model(model_h);
        if (!norm_host) fail(MMH_ERR_ARGUMENT, "norm is a null pointer");
        if (!m.has_grad) fail(MMH_ERR_ARGUMENT, "no gradients yet: run mmh_model_backward first");
        float host[2];
        m.read_step(&host[0], &host[1]);
        *norm_host = host[1];
        return MMH_OK;
    });
}

int32_t mmh_model_set_optimizer(mmh_handle model_h, float beta1, float beta2, float eps,
                                float weight_decay, float clip_norm) {
    return guard([&] {
        Model &m = model(model_h);
        // adamw.rs:48-66 and lab.rs:185-190
        if (!(beta1 >= 0.0f && beta1 < 1.0f))
            fail(MMH_ERR_ARGUMENT, "adamw: beta1 must be in [0, 1), got " + std::to_string(beta1));
        if (!(beta2 >= 0.0f && beta2 < 1.0f))
            fail(MMH_ERR_ARGUMENT, "adamw: beta2 must be in [0, 1), got " + std::to_string(beta2));
        if (!(std::isfinite(eps) && eps > 0.0f))
            fail(MMH_ERR_ARGUMENT, "adamw: eps must be positive and finite");
        if (!(std::isfinite(weight_decay) && weight_decay >= 0.0f))
            fail(MMH_ERR_ARGUMENT, "adamw: weight_decay must be finite and not negative");
        if (!(std::isfinite(clip_norm) && clip_norm > 0.0f))
            fail(MMH_ERR_ARGUMENT, "clip_norm must be positive and finite");
        m.beta1 = beta1;
        m.beta2 = beta2;
        m.adam_eps = eps;
        m.weight_decay = weight_decay;
        m.clip_norm = clip_norm;
        m.has_opt = true;
        m.opt_steps = 0;
        if (m.mom1) {  // a new optimizer starts with no moments
            launch_fill(*m.ctx, m.mom1, m.n_dev, 0.0f);
            launch_fill(*m.ctx, m.mom2, m.n_dev, 0.0f);
            check_hip(hipStreamSynchronize(m.ctx->stream), "optimizer reset sync");
        }
        return MMH_OK;
    });
}

int32_t mmh_model_stage_train(mmh_handle model_h, const int32_t *inputs_host,
                              const int32_t *targets_host, int64_t batch, int64_t seq) {
    return guard([&] {
        model(model_h).stage_train(inputs_host, targets_host, batch, seq);
        return MMH_OK;
    });
}

int32_t mmh_model_train_staged(mmh_handle model_h, int64_t batch, int64_t seq, float lr,
                               float *loss_host, float *grad_norm_host) {
    return guard([&] {
        Model &m = model(model_h);
        float l = 0.0f, g = 0.0f;
        const bool ok = m.train_staged(batch, seq, lr, &l, &g);
        if (loss_host) *loss_host = l;
        if (grad_norm_host) *grad_norm_host = g;
        if (!ok) {  // lab.rs:268-271, clip.rs:48-50: nothing was changed
            if (!std::isfinite(l))
                fail(MMH_STOPPED, "the loss is " + std::to_string(l) + ", not a finite number");
            fail(MMH_STOPPED, "clip: the gradient norm is not finite");
        }
        return MMH_OK;
    });
}

int32_t mmh_model_train_step(mmh_handle model_h, const int32_t *inputs_host,
                             const int32_t *targets_host, int64_t batch, int64_t seq, float lr,
                             float *loss_host, float *grad_norm_host) {
    const int32_t st = mmh_model_stage_train(model_h, inputs_host, targets_host, batch, seq);
    if (st != MMH_OK) return st;
    return mmh_model_train_staged(model_h, batch, seq, lr, loss_host, grad_norm_host);
}

namespace {

// The checks Trainer::new and Trainer::evaluate make between the data and the
// model (trainer.rs:83-108, :218-235).
void check_data_for(const Model &m, const Sequences &q) {
    if (q.seq_len > (uint64_t)m.cfg.max_seq)
        fail(MMH_ERR_ARGUMENT, "invalid argument: sequences of " + std::to_string(q.seq_len) +
                                   " tokens are longer than the model's " +
                                   std::to_string(m.cfg.max_seq));
    if (q.vocab() < 0) fail(MMH_ERR_ARGUMENT, "invalid argument: the data has no tokens");
    if (q.vocab() != m.cfg.vocab)
        fail(MMH_ERR_ARGUMENT, "invalid argument: the data has a vocabulary of " +
                                   std::to_string(q.vocab()) + " and the model " +
                                   std::to_string(m.cfg.vocab));
    if (m.cfg.vocab > INT32_MAX) fail(MMH_ERR_ARGUMENT, "the vocabulary does not fit int32 ids");
}

}  // namespace

int32_t mmh_model_train_next(mmh_handle model_h, mmh_handle batcher_h, float lr,
                             float *loss_host, float *grad_norm_host, uint64_t *epoch,
                             uint64_t *index) {
    return guard([&] {
        Model &m = model(model_h);
        Batcher &b = batcher_of(batcher_h);
        check_data_for(m, *b.data);
        const int64_t batch = (int64_t)b.batch, seq = (int64_t)b.data->seq_len;
        std::vector<uint32_t> in((size_t)(batch * seq)), tg((size_t)(batch * seq));
        const uint64_t e0 = b.epoch, p0 = b.position;  // trainer.rs:163
        uint64_t e = 0, i = 0;
        b.next_batch(in.data(), tg.data(), &e, &i);
        try {
            // every id is below the vocabulary, which fits int32
            m.stage_train(reinterpret_cast<const int32_t *>(in.data()),
                          reinterpret_cast<const int32_t *>(tg.data()), batch, seq);
            float l = 0.0f, g = 0.0f;
            const bool ok = m.train_staged(batch, seq, lr, &l, &g);
            if (loss_host) *loss_host = l;
            if (grad_norm_host) *grad_norm_host = g;
            if (!ok) {
                if (!std::isfinite(l))
                    fail(MMH_STOPPED, "the loss is " + std::to_string(l) +
                                          ", not a finite number");
                fail(MMH_STOPPED, "clip: the gradient norm is not finite");
            }
        } catch (...) {
            b.seek(e0, p0);  // trainer.rs:177-181: the batcher goes back
            throw;
        }
        if (epoch) *epoch = e;
        if (index) *index = i;
        return MMH_OK;
    });
}

int32_t mmh_model_evaluate(mmh_handle model_h, mmh_handle sequences_h, uint64_t batch_size,
                           uint64_t max_batches, float *loss_host, uint64_t *batches_out,
                           uint64_t *tokens_out) {
    return guard([&] {
        if (!loss_host) fail(MMH_ERR_ARGUMENT, "loss is a null pointer");
        Model &m = model(model_h);
        std::shared_ptr<const Sequences> q = sequences_of(sequences_h);
        check_data_for(m, *q);
        if (batch_size == 0) fail(MMH_ERR_ARGUMENT, "invalid argument: the batch size is 0");
        if (max_batches == 0 || q->len() == 0)
            fail(MMH_ERR_ARGUMENT, "invalid argument: nothing to evaluate");
        // trainer.rs:236-257: batches of the run's size (or all there is),
        // row k of `rows` is sequence k * len / rows, the mean of the losses.
        const uint64_t len = q->len(), seq = q->seq_len;
        const uint64_t batch = std::min(batch_size, len);
        const uint64_t batches = std::min(max_batches, len / batch);
        const uint64_t rows = batches * batch;
        std::vector<int32_t> in((size_t)(batch * seq)), tg((size_t)(batch * seq));
        double total = 0.0;
        for (uint64_t bi = 0; bi < batches; ++bi) {
            for (uint64_t r = 0; r < batch; ++r) {
                const uint64_t at =
                    (uint64_t)((unsigned __int128)(bi * batch + r) * len / rows);
                const uint32_t *w = q->window(at);
                std::memcpy(&in[(size_t)(r * seq)], w, (size_t)seq * 4);
                std::memcpy(&tg[(size_t)(r * seq)], w + 1, (size_t)seq * 4);
            }
            float l = 0.0f;
            m.run(in.data(), tg.data(), (int64_t)batch, (int64_t)seq, nullptr, &l);
            total += (double)l;
        }
        *loss_host = (float)(total / (double)batches);
        if (batches_out) *batches_out = batches;
        if (tokens_out) *tokens_out = rows * seq;
        return MMH_OK;
    });
}

int32_t mmh_model_optimizer_steps(mmh_handle model_h, uint64_t *out) {
    return guard([&] {
        if (!out) fail(MMH_ERR_ARGUMENT, "out is a null pointer");
        *out = model(model_h).opt_steps;
        return MMH_OK;
    });
}

// ---- checkpoints (midman-checkpoint params.rs) ----------------------------------

namespace {

std::vector<ParamSpec> specs_of(const Model &m) {
    const Config &c = m.cfg;
    return model_param_specs(c.vocab, c.d, c.layers, c.kv(), c.ff, c.tie);
}

// The new weights arrive in a separate buffer and replace the old ones only when
// the whole file has been read (params.rs:126: nothing changes on failure).
void load_into(Model &m, const std::string &path) {
    Model::DevTemp fresh(m.ctx, m.n_params);  // the file's tensors, reference order
    load_checkpoint(*m.ctx, specs_of(m), m.n_params, path, fresh.p, nullptr);
    m.set_weights_from_ref(fresh.p);
}

}  // namespace

int32_t mmh_model_save_checkpoint(mmh_handle model_h, const char *path, const char *const *keys,
                                  const char *const *values, int64_t n_metadata) {
    return guard([&] {
        Model &m = model(model_h);
        if (!path) fail(MMH_ERR_ARGUMENT, "path is a null pointer");
        if (n_metadata < 0 || (n_metadata > 0 && (!keys || !values)))
            fail(MMH_ERR_ARGUMENT, "metadata arrays are null");
        std::map<std::string, std::string> meta;
        for (int64_t i = 0; i < n_metadata; ++i) {
            if (!keys[i] || !values[i]) fail(MMH_ERR_ARGUMENT, "a metadata string is null");
            meta[keys[i]] = values[i];
        }
        m.ctx->select();
        check_hip(hipStreamSynchronize(m.ctx->stream), "checkpoint sync");
        Model::DevTemp ref(m.ctx, m.n_params);  // the weights in the reference order
        m.dev_to_ref(m.w, ref.p);
        check_hip(hipStreamSynchronize(m.ctx->stream), "checkpoint conversion sync");
        save_checkpoint(*m.ctx, ref.p, specs_of(m), meta, path);
        return MMH_OK;
    });
}

int32_t mmh_model_load_checkpoint(mmh_handle model_h, const char *path) {
    return guard([&] {
        Model &m = model(model_h);
        if (!path) fail(MMH_ERR_ARGUMENT, "path is a null pointer");
        m.ctx->select();
        check_hip(hipStreamSynchronize(m.ctx->stream), "checkpoint sync");
        load_into(m, path);
        return MMH_OK;
    });
}

int32_t mmh_model_create_from_checkpoint(mmh_handle ctx, const double config[10],
                                         const char *path, mmh_handle *out_model) {
    return guard([&] {
        if (!out_model) fail(MMH_ERR_ARGUMENT, "out_model is a null pointer");
        if (!path) fail(MMH_ERR_ARGUMENT, "path is a null pointer");
        auto m = new_model(ctx, config);
        fill_or_release(*m, [&](Model &mm) { load_into(mm, path); });
        *out_model = register_model(std::move(m));
        return MMH_OK;
    });
}

int32_t mmh_block_forward(mmh_handle ctx, const float *x, const float *block_weights,
                          const float *cos_dev, const float *sin_dev, int64_t b, int64_t t,
                          int64_t d, int64_t h, int64_t hkv, int64_t ff, float eps, float *out) {
    return guard([&] {
        Context &c = context(ctx);
        for (const void *p : {(const void *)x, (const void *)block_weights, (const void *)cos_dev,
                              (const void *)sin_dev, (const void *)out})
            if (!p) fail(MMH_ERR_ARGUMENT, "block_forward: a null pointer argument");
        for (int64_t v : {b, t, d, h, hkv, ff})
            if (v <= 0) fail(MMH_ERR_ARGUMENT, "block_forward: sizes must be positive");
        if (d % h || h % hkv)
            fail(MMH_ERR_SHAPE, "block_forward: d_model % n_heads or n_heads % n_kv_heads != 0");
        if (!(std::isfinite(eps) && eps > 0.0f))
            fail(MMH_ERR_ARGUMENT, "block_forward: eps must be positive and finite");
        const int64_t hd = d / h, kv = hkv * hd, n = b * t, qc = d + 2 * kv;
        const int64_t ff_pad = (ff + 31) / 32 * 32;
        // DecoderBlock::parameters order (block.rs:85-93)
        const float *an = block_weights, *wq = an + d, *wk = wq + d * d, *wv = wk + d * kv;
        const float *wo = wv + d * kv, *mn = wo + d * d, *wg = mn + d, *wu = wg + d * ff;
        const float *wdn = wu + d * ff;
        auto al = [](int64_t v) { return (v + 63) / 64 * 64; };
        const int64_t sizes[] = {al(d * qc), al(d * 2 * ff_pad), al(n * d), al(n * qc),
                                 al(n * d), al(n * ff)};
        int64_t total = 0;
        for (int64_t v : sizes) total += v;
        float *ws = static_cast<float *>(c.workspace(2, (size_t)total * 4));
        float *wqkv = ws, *wgu = wqkv + sizes[0];
        BlockRun r;
        r.xn = wgu + sizes[1];
        r.qkv = r.xn + sizes[2];
        r.cb = r.qkv + sizes[3];
        r.h = r.cb + sizes[4];
        launch_pack_cols(c, wq, d, d, wqkv, qc, 0);
        launch_pack_cols(c, wk, d, kv, wqkv, qc, d);
        launch_pack_cols(c, wv, d, kv, wqkv, qc, d + kv);
        launch_pack_gate_up(c, wg, wu, d, ff, ff_pad, wgu);
        if (out != x)
            check_hip(hipMemcpyAsync(out, x, (size_t)(n * d) * 4, hipMemcpyDeviceToDevice,
                                     c.stream), "block input copy");
        r.attn_norm = an;
        r.wqkv = wqkv;
        r.wo = wo;
        r.mlp_norm = mn;
        r.wgu = wgu;
        r.wd = wdn;
        r.cos_t = cos_dev;
        r.sin_t = sin_dev;
        r.x = out;
        r.batch = b;
        r.seq = t;
        r.d = d;
        r.heads = h;
        r.kv_heads = hkv;
        r.ff = ff;
        r.ff_pad = ff_pad;
        r.eps = eps;
        enqueue_block(c, r, [](int, auto &&launch) { launch(); });
        return MMH_OK;
    });
}

int32_t mmh_model_destroy(mmh_handle model_h) {
    return guard([&] {
        std::unique_ptr<Model> m;
        {
            std::lock_guard<std::mutex> lock(g_models_mutex);
            if (model_h <= 0 || (size_t)model_h > g_models.size() || !g_models[(size_t)model_h - 1])
                fail(MMH_ERR_ARGUMENT, "invalid model handle " + std::to_string(model_h));
            m = std::move(g_models[(size_t)model_h - 1]);
        }
        m->release();
        return MMH_OK;
    });
}

int32_t mmh_model_check_guards(mmh_handle model_h, uint64_t *broken_words) {
    return guard([&] {
        if (!broken_words) fail(MMH_ERR_ARGUMENT, "broken_words is a null pointer");
        Model &m = model(model_h);
        m.ctx->select();
        *broken_words = m.count_broken_guards();
        return MMH_OK;
    });
}

}  // extern "C"
