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
// Weights keep the reference parameter order in one device buffer; the QKV
// and gate/up matrices are additionally packed once at creation.
#include <cmath>
#include <cstring>
#include <mutex>

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
    const int64_t hd = c.hd();
    if (hd != 4 && hd != 8 && hd != 16 && hd != 32 && hd != 64 && hd != 128)
        fail(MMH_ERR_CONFIG, "head dimension " + std::to_string(hd) +
                                 " is not one of the device attention sizes 4, 8, 16, 32, 64, 128");
    return c;
}

struct Model {
    mmh_handle ctx_handle = 0;
    Context *ctx = nullptr;
    Config cfg;
    int64_t n_params = 0;
    float *w = nullptr;        // reference parameter order
    float *packed = nullptr;   // per layer: Wqkv [d, d+2kv] then Wgu [d, 2*ff_pad]
    int64_t ff_pad = 0;
    float *cos_t = nullptr, *sin_t = nullptr;
    HostRng rng{};
    bool has_rng = false;
    // Activations for up to cap rows.
    int64_t cap = 0;
    float *act = nullptr;
    float *x = nullptr, *xn = nullptr, *qkv = nullptr, *cb = nullptr, *h = nullptr,
          *logits = nullptr, *row_loss = nullptr, *loss = nullptr;
    int32_t *ids = nullptr, *tgt = nullptr;
    int64_t staged_n = 0;
    bool staged_targets = false;
    // The staged forward + loss of one (batch, seq) as a HIP graph: launch-bound
    // small presets replay ~30 kernels with one call. Valid while the
    // activation buffer it was captured on is the current one.
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    int64_t graph_b = 0, graph_t = 0, warm_b = 0, warm_t = 0;
    const void *graph_act = nullptr, *warm_act = nullptr;

    void drop_graph() {
        if (graph_exec) (void)hipGraphExecDestroy(graph_exec);
        if (graph) (void)hipGraphDestroy(graph);
        graph_exec = nullptr;
        graph = nullptr;
        graph_b = graph_t = 0;
        graph_act = nullptr;
    }

    int64_t qkv_cols() const { return cfg.d + 2 * cfg.kv(); }
    const float *embed() const { return w; }
    const float *block(int64_t l) const { return w + cfg.vocab * cfg.d + l * cfg.block_params(); }
    const float *attn_norm(int64_t l) const { return block(l); }
    const float *wo(int64_t l) const {
        const int64_t d = cfg.d, kv = cfg.kv();
        return block(l) + d + d * d + 2 * d * kv;
    }
    const float *mlp_norm(int64_t l) const { return wo(l) + cfg.d * cfg.d; }
    const float *wd(int64_t l) const { return mlp_norm(l) + cfg.d + 2 * cfg.d * cfg.ff; }
    const float *final_norm() const { return block(cfg.layers); }
    const float *lm_head() const { return final_norm() + cfg.d; }
    int64_t packed_per_layer() const { return cfg.d * qkv_cols() + cfg.d * 2 * ff_pad; }
    const float *wqkv(int64_t l) const { return packed + l * packed_per_layer(); }
    const float *wgu(int64_t l) const { return wqkv(l) + cfg.d * qkv_cols(); }

    void release() {
        ctx->select();
        (void)hipStreamSynchronize(ctx->stream);
        drop_graph();
        for (void *p : {(void *)w, (void *)packed, (void *)cos_t, (void *)sin_t, (void *)act})
            if (p) (void)hipFree(p);
        w = packed = cos_t = sin_t = act = nullptr;
    }

    void ensure(int64_t n) {
        if (n <= cap) return;
        if (act) {
            check_hip(hipStreamSynchronize(ctx->stream), "sync");
            check_hip(hipFree(act), "free activations");
            act = nullptr;
        }
        const int64_t d = cfg.d;
        auto al = [](int64_t v) { return (v + 63) / 64 * 64; };
        const int64_t sizes[] = {al(n * d), al(n * d), al(n * qkv_cols()), al(n * d),
                                 al(n * cfg.ff), al(n * cfg.vocab), al(n), 64, al(n), al(n)};
        int64_t total = 0;
        for (int64_t s : sizes) total += s;
        check_hip(hipMalloc(&act, (size_t)total * 4), "activation alloc");
        float *p = act;
        float **slots[] = {&x, &xn, &qkv, &cb, &h, &logits, &row_loss, &loss};
        for (int i = 0; i < 8; ++i) {
            *slots[i] = p;
            p += sizes[i];
        }
        ids = reinterpret_cast<int32_t *>(p);
        p += sizes[8];
        tgt = reinterpret_cast<int32_t *>(p);
        cap = n;
        staged_n = 0;
    }

    void pack() {
        const int64_t d = cfg.d, kv = cfg.kv(), ff = cfg.ff;
        ff_pad = (ff + 31) / 32 * 32;
        check_hip(hipMalloc(&packed, (size_t)(cfg.layers * packed_per_layer()) * 4), "packed alloc");
        for (int64_t l = 0; l < cfg.layers; ++l) {
            const float *wq = block(l) + d, *wk = wq + d * d, *wv = wk + d * kv;
            float *dst = const_cast<float *>(wqkv(l));
            launch_pack_cols(*ctx, wq, d, d, dst, qkv_cols(), 0);
            launch_pack_cols(*ctx, wk, d, kv, dst, qkv_cols(), d);
            launch_pack_cols(*ctx, wv, d, kv, dst, qkv_cols(), d + kv);
            const float *wg = mlp_norm(l) + d, *wu = wg + d * ff;
            launch_pack_gate_up(*ctx, wg, wu, d, ff, ff_pad, const_cast<float *>(wgu(l)));
        }
        const size_t tab = (size_t)(cfg.max_seq * (cfg.hd() / 2));
        std::vector<float> c(tab), s(tab);
        rope_tables_host(cfg.hd(), cfg.max_seq, cfg.theta, c.data(), s.data());
        check_hip(hipMalloc(&cos_t, tab * 4), "rope alloc");
        check_hip(hipMalloc(&sin_t, tab * 4), "rope alloc");
        check_hip(hipMemcpyAsync(cos_t, c.data(), tab * 4, hipMemcpyHostToDevice, ctx->stream), "rope upload");
        check_hip(hipMemcpyAsync(sin_t, s.data(), tab * 4, hipMemcpyHostToDevice, ctx->stream), "rope upload");
        check_hip(hipStreamSynchronize(ctx->stream), "pack sync");
    }

    // Checks of model.rs:134-148 and the id ranges (ops_shape.rs:250-252,
    // ops_reduce.rs:250-252), then the ids go to the model's token buffers.
    void stage(const int32_t *inputs, const int32_t *targets, int64_t batch, int64_t seq) {
        if (batch <= 0 || seq <= 0)
            fail(MMH_ERR_ARGUMENT, "forward: batch and seq must be at least 1");
        if (seq > cfg.max_seq)
            fail(MMH_ERR_ARGUMENT, "forward: sequence length " + std::to_string(seq) +
                                       " exceeds max_seq_len " + std::to_string(cfg.max_seq));
        const int64_t n = batch * seq;
        check_ids(inputs, n, cfg.vocab, "token id");
        if (targets) check_ids(targets, n, cfg.vocab, "target class");
        ctx->select();
        ensure(n);
        check_hip(hipMemcpyAsync(ids, inputs, (size_t)n * 4, hipMemcpyHostToDevice, ctx->stream),
                  "ids upload");
        if (targets)
            check_hip(hipMemcpyAsync(tgt, targets, (size_t)n * 4, hipMemcpyHostToDevice,
                                     ctx->stream),
                      "targets upload");
        staged_n = n;
        staged_targets = targets != nullptr;
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
    // Queued on the context stream; nothing waits.
    void enqueue(int64_t batch, int64_t seq, bool with_loss, Prof *prof = nullptr) {
        const int64_t n = batch * seq;
        if (n != staged_n || n > cap)
            fail(MMH_ERR_ARGUMENT, "no tokens staged for batch " + std::to_string(batch) +
                                       " x seq " + std::to_string(seq));
        if (seq > cfg.max_seq) fail(MMH_ERR_ARGUMENT, "forward: sequence length exceeds max_seq_len");
        if (with_loss && !staged_targets) fail(MMH_ERR_ARGUMENT, "no targets staged");
        Context &c = *ctx;
        const int64_t d = cfg.d, kv = cfg.kv(), hd = cfg.hd(), V = cfg.vocab;
        timed(prof, MMH_PROF_EMBEDDING, [&] { launch_embedding(c, embed(), d, ids, n, x); });
        for (int64_t l = 0; l < cfg.layers; ++l) {
            timed(prof, MMH_PROF_RMS_NORM,
                  [&] { launch_rms_norm(c, x, attn_norm(l), n, d, cfg.eps, xn); });
            GemmDesc g;
            g.a = xn;
            g.b = wqkv(l);
            g.c = qkv;
            g.m = n;
            g.k = d;
            g.n = qkv_cols();
            g.lda = d;
            g.ldb = qkv_cols();
            g.ldc = qkv_cols();
            timed(prof, MMH_PROF_GEMM_QKV, [&] { gemm(c, g); });

            AttnDesc a{};
            const int64_t ld = qkv_cols();
            a.q = qkv;
            a.k = qkv + d;
            a.v = qkv + d + kv;
            a.out = cb;
            a.sqb = a.skb = a.svb = seq * ld;
            a.sqh = a.skh = a.svh = hd;
            a.sqt = a.skt = a.svt = ld;
            a.sob = seq * d;
            a.soh = hd;
            a.sot = d;
            a.b = batch;
            a.h = cfg.heads;
            a.hkv = cfg.kv_heads;
            a.t = seq;
            a.hd = hd;
            a.cos_t = cos_t;
            a.sin_t = sin_t;
            timed(prof, MMH_PROF_ATTENTION, [&] { attention(c, a); });

            GemmDesc o;
            o.a = cb;
            o.b = wo(l);
            o.c = x;
            o.m = n;
            o.k = d;
            o.n = d;
            o.lda = d;
            o.ldb = d;
            o.ldc = d;
            o.epi = EPI_ACCUM;
            timed(prof, MMH_PROF_GEMM_O, [&] { gemm(c, o); });

            timed(prof, MMH_PROF_RMS_NORM,
                  [&] { launch_rms_norm(c, x, mlp_norm(l), n, d, cfg.eps, xn); });
            GemmDesc gu;
            gu.a = xn;
            gu.b = wgu(l);
            gu.c = h;
            gu.m = n;
            gu.k = d;
            gu.n = 2 * ff_pad;
            gu.lda = d;
            gu.ldb = 2 * ff_pad;
            gu.ldc = cfg.ff;
            gu.epi = EPI_SWIGLU;
            gu.swiglu_ff = cfg.ff;
            timed(prof, MMH_PROF_GEMM_GATE_UP, [&] { gemm(c, gu); });

            GemmDesc dn;
            dn.a = h;
            dn.b = wd(l);
            dn.c = x;
            dn.m = n;
            dn.k = cfg.ff;
            dn.n = d;
            dn.lda = cfg.ff;
            dn.ldb = d;
            dn.ldc = d;
            dn.epi = EPI_ACCUM;
            timed(prof, MMH_PROF_GEMM_DOWN, [&] { gemm(c, dn); });
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
        timed(prof, MMH_PROF_GEMM_HEAD, [&] { gemm(c, hg); });
        if (with_loss)
            timed(prof, MMH_PROF_LOSS,
                  [&] { launch_cross_entropy(c, logits, tgt, n, V, row_loss, loss); });
    }

    // First call for a shape: eager (every workspace reaches its size). Second:
    // capture the same launches into a graph. Later calls replay the graph.
    // The graph holds no memset or allocation: only kernel launches.
    void run_staged(int64_t batch, int64_t seq) {
        if (graph_exec && graph_b == batch && graph_t == seq && graph_act == act &&
            staged_n == batch * seq && staged_targets) {
            check_hip(hipGraphLaunch(graph_exec, ctx->stream), "graph launch");
            return;
        }
        if (!(warm_b == batch && warm_t == seq && warm_act == act)) {
            enqueue(batch, seq, true);
            warm_b = batch;
            warm_t = seq;
            warm_act = act;
            return;
        }
        drop_graph();
        check_hip(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal), "capture");
        try {
            enqueue(batch, seq, true);
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
        check_hip(hipGraphLaunch(graph_exec, ctx->stream), "graph launch");
    }

    void run(const int32_t *inputs, const int32_t *targets, int64_t batch, int64_t seq,
             float *logits_out, float *loss_out) {
        stage(inputs, loss_out ? targets : nullptr, batch, seq);
        enqueue(batch, seq, loss_out != nullptr);
        Context &c = *ctx;
        if (loss_out)
            check_hip(hipMemcpyAsync(loss_out, loss, 4, hipMemcpyDeviceToHost, c.stream),
                      "loss download");
        if (logits_out)
            check_hip(hipMemcpyAsync(logits_out, logits, (size_t)(batch * seq * cfg.vocab) * 4,
                                     hipMemcpyDeviceToHost, c.stream),
                      "logits download");
        check_hip(hipStreamSynchronize(c.stream), "forward sync");
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
    check_hip(hipMalloc(&m->w, (size_t)m->n_params * 4), "weights alloc");
    return m;
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
        for (void *p : {(void *)m->w, (void *)m->packed, (void *)m->cos_t, (void *)m->sin_t,
                        (void *)m->act})
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
        if (n_weights != m->n_params) {
            m->release();
            fail(MMH_ERR_SHAPE, "the config has " + std::to_string(m->n_params) +
                                    " parameters but " + std::to_string(n_weights) +
                                    " weights were given");
        }
        check_hip(hipMemcpyAsync(m->w, weights_host, (size_t)n_weights * 4,
                                 hipMemcpyHostToDevice, m->ctx->stream),
                  "weights upload");
        m->pack();
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
        const Config &c = m->cfg;
        // model.rs:51-83 draw order; norms are ones (norm.rs:60).
        std::vector<float> host((size_t)m->n_params);
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
        if (p - host.data() != m->n_params) fail(MMH_ERR_OTHER, "init: parameter count mismatch");
        check_hip(hipMemcpyAsync(m->w, host.data(), host.size() * 4, hipMemcpyHostToDevice,
                                 m->ctx->stream),
                  "weights upload");
        check_hip(hipStreamSynchronize(m->ctx->stream), "weights upload sync");
        m->rng = rng;
        m->has_rng = true;
        m->pack();
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
        check_hip(hipMemcpyAsync(out_host, m.w, (size_t)n * 4, hipMemcpyDeviceToHost,
                                 m.ctx->stream),
                  "weights download");
        check_hip(hipStreamSynchronize(m.ctx->stream), "weights download sync");
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
        check_hip(hipMemcpyAsync(loss_host, m.loss, 4, hipMemcpyDeviceToHost, m.ctx->stream),
                  "loss download");
        check_hip(hipStreamSynchronize(m.ctx->stream), "loss sync");
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
        m.enqueue(batch, seq, true, &prof);
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

}  // extern "C"
