// The C ABI of libmidman_hip.so: handle tables, contexts (one device + one
// stream), device buffers, timers and the op-level entry points (the status
// codes and the error buffer are host_errors.cpp). Boundary rules follow midman-api/src/ffi.rs:5-32, 99-145:
// handles not pointers, status codes, the last error message per thread, and
// nothing unwinds across the boundary (every entry point catches everything).
#include <cmath>
#include <cstring>
#include <mutex>
#include <new>

#include <cstdlib>

#include "mmh_internal.h"

namespace mmh {

namespace {
std::mutex g_mutex;
std::vector<std::unique_ptr<Context>> g_contexts;  // handle = index + 1
}  // namespace

void check_hip(hipError_t e, const char *what) {
    if (e != hipSuccess)
        fail(MMH_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

void *Context::get_scratch(size_t bytes) { return workspace(0, bytes); }

void *Context::workspace(int slot, size_t bytes) {
    if (slot < 0 || slot >= kSlots) fail(MMH_ERR_OTHER, "workspace slot out of range");
    if (bytes == 0) bytes = 256;
    if (bytes > ws_bytes[slot]) {
        if (ws[slot]) {
            // The old buffer may still be read by queued kernels.
            check_hip(hipStreamSynchronize(stream), "workspace sync");
            check_hip(hipFree(ws[slot]), "workspace free");
            ws[slot] = nullptr;
            ws_bytes[slot] = 0;
        }
        const size_t rounded = (bytes + (1u << 20) - 1) & ~size_t((1u << 20) - 1);
        check_hip(hipMalloc(&ws[slot], rounded), "workspace alloc");
        ws_bytes[slot] = rounded;
    }
    return ws[slot];
}

int32_t *Context::stage_ids(const int32_t *host, int64_t n, int which) {
    // Two halves of slot 1: inputs at 0, targets after them.
    const size_t half = ((size_t)n * 4 + 255) & ~size_t(255);
    char *base = static_cast<char *>(workspace(1, 2 * half));
    int32_t *dst = reinterpret_cast<int32_t *>(base + (which ? half : 0));
    check_hip(hipMemcpyAsync(dst, host, (size_t)n * 4, hipMemcpyHostToDevice, stream),
              "ids upload");
    return dst;
}

void Context::select() const { check_hip(hipSetDevice(device), "hipSetDevice"); }

Context &context(mmh_handle h) {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (h <= 0 || (size_t)h > g_contexts.size() || !g_contexts[(size_t)h - 1])
        fail(MMH_ERR_ARGUMENT, "invalid context handle " + std::to_string(h));
    Context &c = *g_contexts[(size_t)h - 1];
    c.select();
    return c;
}

void check_ids(const int32_t *ids, int64_t n, int64_t vocab, const char *what) {
    if (!ids) fail(MMH_ERR_ARGUMENT, std::string(what) + " is a null pointer");
    for (int64_t i = 0; i < n; ++i) {
        if (ids[i] < 0 || ids[i] >= vocab)
            fail(MMH_ERR_INDEX, std::string(what) + " " + std::to_string(ids[i]) +
                                    " is out of range for " + std::to_string(vocab));
    }
}

}  // namespace mmh

using namespace mmh;

namespace {

void need(const void *p, const char *what) {
    if (!p) fail(MMH_ERR_ARGUMENT, std::string(what) + " is a null pointer");
}
void positive(int64_t v, const char *what) {
    if (v <= 0) fail(MMH_ERR_SHAPE, std::string(what) + " must be at least 1, got " + std::to_string(v));
}

}  // namespace

extern "C" {

int32_t mmh_context_create(int32_t device, mmh_handle *out_ctx) {
    return guard([&] {
        need(out_ctx, "out_ctx");
        int count = 0;
        check_hip(hipGetDeviceCount(&count), "hipGetDeviceCount");
        if (device < 0 || device >= count)
            fail(MMH_ERR_ARGUMENT, "device " + std::to_string(device) + " does not exist (" +
                                       std::to_string(count) + " visible)");
        auto c = std::make_unique<Context>();
        c->device = device;
        check_hip(hipSetDevice(device), "hipSetDevice");
        hipDeviceProp_t prop;
        check_hip(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
        c->cu_count = prop.multiProcessorCount;
        c->name = prop.name[0] ? prop.name : prop.gcnArchName;
        check_hip(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "stream create");
        check_hip(hipEventCreate(&c->t0), "event create");
        check_hip(hipEventCreate(&c->t1), "event create");
        c->xcd_teams = probe_xcd_teams(*c);
        if (const char *e = std::getenv("MMH_FUSED_ATOMIC_SLOTS"))
            if (e[0] == '1') c->xcd_rr = false;
        check_hip(hipMalloc(&c->tickets, Context::kTickets * sizeof(int32_t)), "ticket alloc");
        check_hip(hipMemsetAsync(c->tickets, 0, Context::kTickets * sizeof(int32_t), c->stream),
                  "ticket clear");
        check_hip(hipStreamSynchronize(c->stream), "ticket clear sync");
        std::lock_guard<std::mutex> lock(g_mutex);
        g_contexts.push_back(std::move(c));
        *out_ctx = (mmh_handle)g_contexts.size();
        return MMH_OK;
    });
}

int32_t mmh_context_destroy(mmh_handle ctx) {
    return guard([&] {
        std::unique_ptr<Context> c;
        {
            std::lock_guard<std::mutex> lock(g_mutex);
            if (ctx <= 0 || (size_t)ctx > g_contexts.size() || !g_contexts[(size_t)ctx - 1])
                fail(MMH_ERR_ARGUMENT, "invalid context handle " + std::to_string(ctx));
            c = std::move(g_contexts[(size_t)ctx - 1]);
        }
        release_models_of(ctx);
        c->select();
        (void)hipStreamSynchronize(c->stream);
        for (void *p : c->owned) (void)hipFree(p);
        for (int s = 0; s < Context::kSlots; ++s)
            if (c->ws[s]) (void)hipFree(c->ws[s]);
        if (c->tickets) (void)hipFree(c->tickets);
        (void)hipEventDestroy(c->t0);
        (void)hipEventDestroy(c->t1);
        (void)hipStreamDestroy(c->stream);
        return MMH_OK;
    });
}

int32_t mmh_synchronize(mmh_handle ctx) {
    return guard([&] {
        check_hip(hipStreamSynchronize(context(ctx).stream), "synchronize");
        return MMH_OK;
    });
}

int32_t mmh_device_info(mmh_handle ctx, char *name, uint32_t cap, int32_t *cu_count) {
    return guard([&] {
        Context &c = context(ctx);
        if (name && cap > 0) {
            const size_t n = std::min<size_t>(cap - 1, c.name.size());
            std::memcpy(name, c.name.data(), n);
            name[n] = '\0';
        }
        if (cu_count) *cu_count = c.cu_count;
        return MMH_OK;
    });
}

int32_t mmh_context_fused_slots(mmh_handle ctx, int32_t *teams, int32_t *round_robin) {
    return guard([&] {
        Context &c = context(ctx);
        if (teams) *teams = c.xcd_teams ? 1 : 0;
        if (round_robin) *round_robin = c.xcd_teams && c.xcd_rr ? 1 : 0;
        return MMH_OK;
    });
}

int32_t mmh_mfma_peak_probe(mmh_handle ctx, double *tflops) {
    return guard([&] {
        need(tflops, "tflops");
        *tflops = mfma_peak_tflops(context(ctx));
        return MMH_OK;
    });
}

int32_t mmh_alloc(mmh_handle ctx, uint64_t bytes, void **out_dev) {
    return guard([&] {
        need(out_dev, "out_dev");
        Context &c = context(ctx);
        void *p = nullptr;
        check_hip(hipMalloc(&p, bytes ? bytes : 1), "hipMalloc");
        c.owned.push_back(p);
        *out_dev = p;
        return MMH_OK;
    });
}

int32_t mmh_free(mmh_handle ctx, void *dev) {
    return guard([&] {
        Context &c = context(ctx);
        for (size_t i = 0; i < c.owned.size(); ++i) {
            if (c.owned[i] == dev) {
                check_hip(hipStreamSynchronize(c.stream), "sync before free");
                check_hip(hipFree(dev), "hipFree");
                c.owned.erase(c.owned.begin() + (long)i);
                return MMH_OK;
            }
        }
        fail(MMH_ERR_ARGUMENT, "pointer was not allocated by mmh_alloc on this context");
    });
}

int32_t mmh_upload(mmh_handle ctx, void *dst_dev, const void *src_host, uint64_t bytes) {
    return guard([&] {
        Context &c = context(ctx);
        need(dst_dev, "dst_dev");
        need(src_host, "src_host");
        check_hip(hipMemcpyAsync(dst_dev, src_host, bytes, hipMemcpyHostToDevice, c.stream),
                  "upload");
        check_hip(hipStreamSynchronize(c.stream), "upload sync");
        return MMH_OK;
    });
}

int32_t mmh_download(mmh_handle ctx, void *dst_host, const void *src_dev, uint64_t bytes) {
    return guard([&] {
        Context &c = context(ctx);
        need(dst_host, "dst_host");
        need(src_dev, "src_dev");
        check_hip(hipMemcpyAsync(dst_host, src_dev, bytes, hipMemcpyDeviceToHost, c.stream),
                  "download");
        check_hip(hipStreamSynchronize(c.stream), "download sync");
        return MMH_OK;
    });
}

int32_t mmh_timer_start(mmh_handle ctx) {
    return guard([&] {
        Context &c = context(ctx);
        check_hip(hipEventRecord(c.t0, c.stream), "event record");
        return MMH_OK;
    });
}

int32_t mmh_timer_stop(mmh_handle ctx, float *ms) {
    return guard([&] {
        need(ms, "ms");
        Context &c = context(ctx);
        check_hip(hipEventRecord(c.t1, c.stream), "event record");
        check_hip(hipEventSynchronize(c.t1), "event sync");
        check_hip(hipEventElapsedTime(ms, c.t0, c.t1), "elapsed time");
        return MMH_OK;
    });
}

int32_t mmh_randn(uint64_t seed, float std_, float *out_host, int64_t n) {
    return guard([&] {
        need(out_host, "out");
        if (n < 0) fail(MMH_ERR_SHAPE, "randn: negative count");
        if (!std::isfinite(std_)) fail(MMH_ERR_ARGUMENT, "randn: std must be finite");
        HostRng rng = HostRng::seed(seed);
        randn_parallel(rng, out_host, n, std_);
        return MMH_OK;
    });
}

// ---- GEMM seam ----------------------------------------------------------------

static int32_t gemm_entry(mmh_handle ctx, const float *a, const float *b, float *c, int64_t m,
                          int64_t k, int64_t n, int32_t accumulate, bool ta, bool tb) {
    return guard([&] {
        Context &cx = context(ctx);
        need(a, "a");
        need(b, "b");
        need(c, "c");
        positive(m, "m");
        positive(k, "k");
        positive(n, "n");
        GemmDesc d;
        d.a = a;
        d.b = b;
        d.c = c;
        d.m = m;
        d.k = k;
        d.n = n;
        d.ta = ta;
        d.tb = tb;
        d.lda = ta ? m : k;
        d.ldb = tb ? k : n;
        d.ldc = n;
        d.epi = accumulate ? EPI_ACCUM : EPI_STORE;
        d.accumulate_into_c = accumulate != 0;
        gemm(cx, d);
        return MMH_OK;
    });
}

int32_t mmh_gemm_nn(mmh_handle ctx, const float *a, const float *b, float *c, int64_t m,
                    int64_t k, int64_t n, int32_t accumulate) {
    return gemm_entry(ctx, a, b, c, m, k, n, accumulate, false, false);
}

int32_t mmh_gemm_nt(mmh_handle ctx, const float *a, const float *b, float *c, int64_t m,
                    int64_t k, int64_t n, int32_t accumulate) {
    return gemm_entry(ctx, a, b, c, m, k, n, accumulate, false, true);
}

int32_t mmh_gemm_tn(mmh_handle ctx, const float *a, const float *b, float *c, int64_t m,
                    int64_t k, int64_t n, int32_t accumulate) {
    return gemm_entry(ctx, a, b, c, m, k, n, accumulate, true, false);
}

int32_t mmh_matmul_batched(mmh_handle ctx, const float *a, const float *b, float *c,
                           int64_t batch, int64_t m, int64_t k, int64_t n) {
    return guard([&] {
        Context &cx = context(ctx);
        need(a, "a");
        need(b, "b");
        need(c, "c");
        positive(batch, "batch");
        positive(m, "m");
        positive(k, "k");
        positive(n, "n");
        GemmDesc d;
        d.a = a;
        d.b = b;
        d.c = c;
        d.m = m;
        d.k = k;
        d.n = n;
        d.lda = k;
        d.ldb = n;
        d.ldc = n;
        d.batch = batch;
        d.stride_a = m * k;
        d.stride_b = k * n;
        d.stride_c = m * n;
        gemm(cx, d);
        return MMH_OK;
    });
}

int32_t mmh_matmul_backward(mmh_handle ctx, const float *a, const float *b, const float *dc,
                            float *da, float *db, int64_t rows, int64_t k, int64_t n) {
    return guard([&] {
        Context &cx = context(ctx);
        need(dc, "dc");
        positive(rows, "rows");
        positive(k, "k");
        positive(n, "n");
        if (da) {  // dA[rows,k] = dC[rows,n] . B[k,n]^T  (gemm_nt, kernels.rs:66)
            need(b, "b");
            GemmDesc d;
            d.a = dc;
            d.b = b;
            d.c = da;
            d.m = rows;
            d.k = n;
            d.n = k;
            d.lda = n;
            d.tb = true;
            d.ldb = n;
            d.ldc = k;
            gemm(cx, d);
        }
        if (db) {  // dB[k,n] = A[rows,k]^T . dC[rows,n]  (gemm_tn, kernels.rs:78)
            need(a, "a");
            GemmDesc d;
            d.a = a;
            d.b = dc;
            d.c = db;
            d.m = k;
            d.k = rows;
            d.n = n;
            d.ta = true;
            d.lda = k;
            d.ldb = n;
            d.ldc = n;
            gemm(cx, d);
        }
        return MMH_OK;
    });
}

// ---- layer ops --------------------------------------------------------------------

int32_t mmh_embedding(mmh_handle ctx, const float *table, int64_t vocab, int64_t d,
                      const int32_t *ids_host, int64_t n, float *out) {
    return guard([&] {
        Context &cx = context(ctx);
        need(table, "table");
        need(out, "out");
        positive(vocab, "vocab");
        positive(d, "d");
        positive(n, "n");
        check_ids(ids_host, n, vocab, "token id");
        const int32_t *ids = cx.stage_ids(ids_host, n, 0);
        launch_embedding(cx, table, d, ids, n, out);
        return MMH_OK;
    });
}

int32_t mmh_rms_norm(mmh_handle ctx, const float *x, const float *w, int64_t rows, int64_t d,
                     float eps, float *out) {
    return guard([&] {
        Context &cx = context(ctx);
        need(x, "x");
        need(w, "w");
        need(out, "out");
        positive(rows, "rows");
        positive(d, "d");
        if (!(std::isfinite(eps) && eps > 0.0f))
            fail(MMH_ERR_ARGUMENT, "rms_norm: eps must be positive and finite");
        launch_rms_norm(cx, x, w, rows, d, eps, out);
        return MMH_OK;
    });
}

int32_t mmh_rope_tables(mmh_handle ctx, int64_t head_dim, int64_t max_seq_len, float theta,
                        float *cos_dev, float *sin_dev) {
    return guard([&] {
        Context &cx = context(ctx);
        need(cos_dev, "cos_dev");
        need(sin_dev, "sin_dev");
        if (head_dim <= 0 || (head_dim & 1))
            fail(MMH_ERR_ARGUMENT, "rope: head_dim must be even and positive");
        positive(max_seq_len, "max_seq_len");
        if (!(std::isfinite(theta) && theta > 0.0f))
            fail(MMH_ERR_ARGUMENT, "rope: theta must be positive and finite");
        const size_t cnt = (size_t)(max_seq_len * (head_dim / 2));
        std::vector<float> c(cnt), s(cnt);
        rope_tables_host(head_dim, max_seq_len, theta, c.data(), s.data());
        check_hip(hipMemcpyAsync(cos_dev, c.data(), cnt * 4, hipMemcpyHostToDevice, cx.stream),
                  "rope upload");
        check_hip(hipMemcpyAsync(sin_dev, s.data(), cnt * 4, hipMemcpyHostToDevice, cx.stream),
                  "rope upload");
        check_hip(hipStreamSynchronize(cx.stream), "rope sync");
        return MMH_OK;
    });
}

int32_t mmh_apply_rope(mmh_handle ctx, const float *x, int64_t bh, int64_t t, int64_t hd,
                       const float *cos_dev, const float *sin_dev, float *out) {
    return guard([&] {
        Context &cx = context(ctx);
        need(x, "x");
        need(cos_dev, "cos_dev");
        need(sin_dev, "sin_dev");
        need(out, "out");
        positive(bh, "bh");
        positive(t, "t");
        if (hd <= 0 || (hd & 1)) fail(MMH_ERR_SHAPE, "apply_rope: the last axis must be even");
        launch_rope(cx, x, bh, t, hd, cos_dev, sin_dev, out);
        return MMH_OK;
    });
}

int32_t mmh_causal_attention(mmh_handle ctx, const float *q, const float *k, const float *v,
                             int64_t b, int64_t h, int64_t hkv, int64_t t, int64_t hd,
                             float *out) {
    return guard([&] {
        Context &cx = context(ctx);
        need(q, "q");
        need(k, "k");
        need(v, "v");
        need(out, "out");
        positive(b, "batch");
        positive(h, "n_heads");
        positive(hkv, "n_kv_heads");
        positive(t, "time");
        positive(hd, "head_dim");
        if (h % hkv) fail(MMH_ERR_SHAPE, "causal_attention: n_heads is not a multiple of n_kv_heads");
        AttnDesc d{};
        d.q = q;
        d.k = k;
        d.v = v;
        d.out = out;
        d.sqb = h * t * hd;
        d.sqh = t * hd;
        d.sqt = hd;
        d.skb = hkv * t * hd;
        d.skh = t * hd;
        d.skt = hd;
        d.svb = d.skb;
        d.svh = d.skh;
        d.svt = d.skt;
        d.sob = d.sqb;
        d.soh = d.sqh;
        d.sot = d.sqt;
        d.b = b;
        d.h = h;
        d.hkv = hkv;
        d.t = t;
        d.hd = hd;
        attention(cx, d);
        return MMH_OK;
    });
}

int32_t mmh_attention_forward(mmh_handle ctx, const float *x, const float *wq, const float *wk,
                              const float *wv, const float *wo, const float *cos_dev,
                              const float *sin_dev, int64_t b, int64_t t, int64_t d,
                              int64_t h, int64_t hkv, float *out) {
    return guard([&] {
        Context &cx = context(ctx);
        for (const void *p : {(const void *)x, (const void *)wq, (const void *)wk,
                              (const void *)wv, (const void *)wo, (const void *)cos_dev,
                              (const void *)sin_dev, (const void *)out})
            need(p, "attention_forward argument");
        positive(b, "batch");
        positive(t, "time");
        positive(d, "d_model");
        positive(h, "n_heads");
        positive(hkv, "n_kv_heads");
        if (d % h || h % hkv)
            fail(MMH_ERR_SHAPE, "attention_forward: d_model % n_heads or n_heads % n_kv_heads != 0");
        const int64_t hd = d / h, kv = hkv * hd, n = b * t;
        float *ws = static_cast<float *>(cx.workspace(2, (size_t)(2 * n * d + 2 * n * kv) * 4));
        float *qp = ws, *kp = qp + n * d, *vp = kp + n * kv, *cb = vp + n * kv;
        auto proj = [&](const float *w, int64_t cols, float *dst) {
            GemmDesc g;
            g.a = x;
            g.b = w;
            g.c = dst;
            g.m = n;
            g.k = d;
            g.n = cols;
            g.lda = d;
            g.ldb = cols;
            g.ldc = cols;
            gemm(cx, g);
        };
        proj(wq, d, qp);
        proj(wk, kv, kp);
        proj(wv, kv, vp);
        AttnDesc a{};
        a.q = qp;
        a.k = kp;
        a.v = vp;
        a.out = cb;
        a.sqb = t * d;
        a.sqh = hd;
        a.sqt = d;
        a.skb = t * kv;
        a.skh = hd;
        a.skt = kv;
        a.svb = a.skb;
        a.svh = a.skh;
        a.svt = a.skt;
        a.sob = t * d;
        a.soh = hd;
        a.sot = d;
        a.b = b;
        a.h = h;
        a.hkv = hkv;
        a.t = t;
        a.hd = hd;
        a.cos_t = cos_dev;
        a.sin_t = sin_dev;
        attention(cx, a);
        GemmDesc g;
        g.a = cb;
        g.b = wo;
        g.c = out;
        g.m = n;
        g.k = d;
        g.n = d;
        g.lda = d;
        g.ldb = d;
        g.ldc = d;
        gemm(cx, g);
        return MMH_OK;
    });
}

int32_t mmh_swiglu(mmh_handle ctx, const float *x, const float *wg, const float *wu,
                   const float *wd, int64_t rows, int64_t d, int64_t ff, float *out) {
    return guard([&] {
        Context &cx = context(ctx);
        for (const void *p : {(const void *)x, (const void *)wg, (const void *)wu,
                              (const void *)wd, (const void *)out})
            need(p, "swiglu argument");
        positive(rows, "rows");
        positive(d, "d_model");
        positive(ff, "d_ff");
        float *ws = static_cast<float *>(cx.workspace(2, (size_t)(2 * rows * ff) * 4));
        float *g = ws, *u = ws + rows * ff;
        auto mm = [&](const float *a, const float *w, float *c, int64_t kk, int64_t nn) {
            GemmDesc gd;
            gd.a = a;
            gd.b = w;
            gd.c = c;
            gd.m = rows;
            gd.k = kk;
            gd.n = nn;
            gd.lda = kk;
            gd.ldb = nn;
            gd.ldc = nn;
            gemm(cx, gd);
        };
        mm(x, wg, g, d, ff);
        mm(x, wu, u, d, ff);
        launch_silu_mul(cx, g, u, g, rows * ff);
        mm(g, wd, out, ff, d);
        return MMH_OK;
    });
}

int32_t mmh_add(mmh_handle ctx, const float *a, const float *b, float *out, int64_t n) {
    return guard([&] {
        Context &cx = context(ctx);
        need(a, "a");
        need(b, "b");
        need(out, "out");
        positive(n, "n");
        launch_add(cx, a, b, out, n);
        return MMH_OK;
    });
}

int32_t mmh_cross_entropy(mmh_handle ctx, const float *logits, const int32_t *targets_host,
                          int64_t n, int64_t vocab, float *loss_host) {
    return guard([&] {
        Context &cx = context(ctx);
        need(logits, "logits");
        need(loss_host, "loss");
        positive(n, "rows");
        positive(vocab, "vocab");
        check_ids(targets_host, n, vocab, "target class");
        const int32_t *tg = cx.stage_ids(targets_host, n, 1);
        float *rows = static_cast<float *>(cx.workspace(3, (size_t)(n + 64) * 4));
        float *loss_dev = rows + ((n + 63) / 64) * 64;
        launch_cross_entropy(cx, logits, tg, n, vocab, rows, loss_dev);
        check_hip(hipMemcpyAsync(loss_host, loss_dev, 4, hipMemcpyDeviceToHost, cx.stream),
                  "loss download");
        check_hip(hipStreamSynchronize(cx.stream), "loss sync");
        return MMH_OK;
    });
}

// ---- op-level backward (the autograd closures of the layer seam) ----------

int32_t mmh_rms_norm_backward(mmh_handle ctx, const float *x, const float *w, const float *dy,
                              int64_t rows, int64_t d, float eps, float *dx, float *dw) {
    return guard([&] {
        Context &cx = context(ctx);
        need(x, "x");
        need(w, "w");
        need(dy, "dy");
        need(dx, "dx");
        need(dw, "dw");
        positive(rows, "rows");
        positive(d, "d");
        if (!(std::isfinite(eps) && eps > 0.0f))
            fail(MMH_ERR_ARGUMENT, "rms_norm: eps must be positive and finite");
        float *scratch = static_cast<float *>(
            cx.workspace(2, (size_t)rms_norm_backward_scratch(rows, d) * 4 + 256));
        launch_rms_norm_backward(cx, x, w, dy, rows, d, eps, dx, false, dw, scratch);
        return MMH_OK;
    });
}

int32_t mmh_apply_rope_backward(mmh_handle ctx, const float *dy, int64_t bh, int64_t t,
                                int64_t hd, const float *cos_dev, const float *sin_dev,
                                float *dx) {
    return guard([&] {
        Context &cx = context(ctx);
        need(dy, "dy");
        need(dx, "dx");
        need(cos_dev, "cos");
        need(sin_dev, "sin");
        positive(bh, "bh");
        positive(t, "time");
        if (hd <= 0 || (hd & 1)) fail(MMH_ERR_SHAPE, "rope backward: the last axis must be even");
        if (dx != dy)
            check_hip(hipMemcpyAsync(dx, dy, (size_t)(bh * t * hd) * 4, hipMemcpyDeviceToDevice,
                                     cx.stream),
                      "rope copy");
        launch_rope_strided(cx, dx, 0, t * hd, hd, 1, bh, t, hd, cos_dev, sin_dev, true);
        return MMH_OK;
    });
}

int32_t mmh_causal_attention_backward(mmh_handle ctx, const float *q, const float *k,
                                      const float *v, const float *dout, int64_t b, int64_t h,
                                      int64_t hkv, int64_t t, int64_t hd, float *dq, float *dk,
                                      float *dv) {
    return guard([&] {
        Context &cx = context(ctx);
        need(q, "q");
        need(k, "k");
        need(v, "v");
        need(dout, "dout");
        need(dq, "dq");
        need(dk, "dk");
        need(dv, "dv");
        positive(b, "batch");
        positive(h, "n_heads");
        positive(hkv, "n_kv_heads");
        positive(t, "time");
        positive(hd, "head_dim");
        if (h % hkv) fail(MMH_ERR_SHAPE, "causal_attention: n_heads is not a multiple of n_kv_heads");
        // forward output and log-sum-exp, then the backward
        const int64_t rows = b * h * t;
        const size_t o_floats = ((size_t)(rows * hd) + 63) / 64 * 64;
        const size_t r_floats = ((size_t)rows + 63) / 64 * 64;
        const size_t s_floats = (size_t)attention_backward_scratch_floats(b, h, hkv, t, hd);
        float *o = static_cast<float *>(
            cx.workspace(2, (o_floats + 2 * r_floats + s_floats) * 4));
        float *lse = o + o_floats, *dvec = lse + r_floats, *part = dvec + r_floats;
        AttnDesc f{};
        f.q = q;
        f.k = k;
        f.v = v;
        f.out = o;
        f.sqb = h * t * hd;
        f.sqh = t * hd;
        f.sqt = hd;
        f.skb = hkv * t * hd;
        f.skh = t * hd;
        f.skt = hd;
        f.svb = f.skb;
        f.svh = f.skh;
        f.svt = f.skt;
        f.sob = f.sqb;
        f.soh = f.sqh;
        f.sot = f.sqt;
        f.b = b;
        f.h = h;
        f.hkv = hkv;
        f.t = t;
        f.hd = hd;
        f.lse = lse;
        attention(cx, f);
        AttnBwdDesc g{};
        g.q = q;
        g.k = k;
        g.v = v;
        g.o = o;
        g.dout = dout;
        g.lse = lse;
        g.dq = dq;
        g.dk = dk;
        g.dv = dv;
        g.dvec = dvec;
        g.sqb = f.sqb; g.sqh = f.sqh; g.sqt = f.sqt;
        g.skb = f.skb; g.skh = f.skh; g.skt = f.skt;
        g.svb = f.svb; g.svh = f.svh; g.svt = f.svt;
        g.sob = f.sob; g.soh = f.soh; g.sot = f.sot;
        g.b = b;
        g.h = h;
        g.hkv = hkv;
        g.t = t;
        g.hd = hd;
        g.scratch = s_floats ? part : nullptr;
        attention_backward(cx, g);
        return MMH_OK;
    });
}

int32_t mmh_swiglu_backward(mmh_handle ctx, const float *x, const float *wg, const float *wu,
                            const float *wd, const float *dout, int64_t rows, int64_t d,
                            int64_t ff, float *dx, float *dwg, float *dwu, float *dwd) {
    return guard([&] {
        Context &cx = context(ctx);
        for (const void *p : {(const void *)x, (const void *)wg, (const void *)wu,
                              (const void *)wd, (const void *)dout, (const void *)dx,
                              (const void *)dwg, (const void *)dwu, (const void *)dwd})
            need(p, "swiglu_backward argument");
        positive(rows, "rows");
        positive(d, "d_model");
        positive(ff, "d_ff");
        // g = x.Wg, u = x.Wu, h = silu(g)*u recomputed (the forward keeps no
        // intermediates), then the closures of mlp.rs:20-24 in reverse.
        const size_t rf = ((size_t)(rows * ff) + 63) / 64 * 64;
        float *ws = static_cast<float *>(cx.workspace(2, 4 * rf * 4));
        float *g = ws, *u = g + rf, *h = u + rf, *dh = h + rf;
        auto mm = [&](const float *a, bool ta, int64_t lda, const float *b, bool tb, int64_t ldb,
                      float *c, int64_t m, int64_t k, int64_t n, int epi) {
            GemmDesc gd;
            gd.a = a;
            gd.ta = ta;
            gd.lda = lda;
            gd.b = b;
            gd.tb = tb;
            gd.ldb = ldb;
            gd.c = c;
            gd.ldc = n;
            gd.m = m;
            gd.k = k;
            gd.n = n;
            gd.epi = epi;
            gemm(cx, gd);
        };
        mm(x, false, d, wg, false, ff, g, rows, d, ff, EPI_STORE);
        mm(x, false, d, wu, false, ff, u, rows, d, ff, EPI_STORE);
        launch_silu_mul(cx, g, u, h, rows * ff);
        mm(h, true, ff, dout, false, d, dwd, ff, rows, d, EPI_STORE);    // dWd = h^T dout
        mm(dout, false, d, wd, true, d, dh, rows, d, ff, EPI_STORE);    // dh = dout Wd^T
        launch_silu_mul_backward(cx, dh, g, u, g, u, rows * ff);        // g, u <- dg, du
        mm(x, true, d, g, false, ff, dwg, d, rows, ff, EPI_STORE);      // dWg = x^T dg
        mm(x, true, d, u, false, ff, dwu, d, rows, ff, EPI_STORE);      // dWu = x^T du
        mm(g, false, ff, wg, true, ff, dx, rows, ff, d, EPI_STORE);     // dx = dg Wg^T
        mm(u, false, ff, wu, true, ff, dx, rows, ff, d, EPI_ACCUM);     //    + du Wu^T
        return MMH_OK;
    });
}

int32_t mmh_embedding_backward(mmh_handle ctx, const int32_t *ids_host, int64_t n,
                               const float *dy, int64_t vocab, int64_t d, float *dtable) {
    return guard([&] {
        Context &cx = context(ctx);
        need(dy, "dy");
        need(dtable, "dtable");
        positive(n, "n");
        positive(vocab, "vocab");
        positive(d, "d");
        check_ids(ids_host, n, vocab, "token id");
        // the distinct ids ascending, and per id its positions ascending (a
        // counting sort), so each table row sums its gradient rows in
        // position order as ops_shape.rs:261-269 adds them
        std::vector<int32_t> count((size_t)vocab + 1, 0);
        for (int64_t i = 0; i < n; ++i) count[(size_t)ids_host[i] + 1]++;
        std::vector<int32_t> index;  // uniq | start | order
        index.reserve((size_t)(3 * n + 1));
        std::vector<int32_t> at((size_t)vocab, 0);
        int32_t run = 0;
        std::vector<int32_t> uniq, start;
        for (int64_t v = 0; v < vocab; ++v) {
            const int32_t c = count[(size_t)v + 1];
            if (c) {
                uniq.push_back((int32_t)v);
                start.push_back(run);
            }
            at[(size_t)v] = run;
            run += c;
        }
        start.push_back(run);
        std::vector<int32_t> order((size_t)n);
        for (int64_t i = 0; i < n; ++i) order[(size_t)at[(size_t)ids_host[i]]++] = (int32_t)i;
        const int64_t nu = (int64_t)uniq.size();
        index.insert(index.end(), uniq.begin(), uniq.end());
        index.insert(index.end(), start.begin(), start.end());
        index.insert(index.end(), order.begin(), order.end());
        int32_t *dev = static_cast<int32_t *>(cx.workspace(3, index.size() * 4));
        check_hip(hipMemcpyAsync(dev, index.data(), index.size() * 4, hipMemcpyHostToDevice,
                                 cx.stream), "index upload");
        launch_fill(cx, dtable, vocab * d, 0.0f);
        launch_embedding_backward(cx, dy, d, dev, dev + nu, dev + 2 * nu + 1, nu, dtable, false);
        check_hip(hipStreamSynchronize(cx.stream), "index upload sync");
        return MMH_OK;
    });
}

int32_t mmh_cross_entropy_backward(mmh_handle ctx, const float *logits,
                                   const int32_t *targets_host, int64_t n, int64_t vocab,
                                   float *dlogits, float *loss_host) {
    return guard([&] {
        Context &cx = context(ctx);
        need(logits, "logits");
        need(dlogits, "dlogits");
        positive(n, "rows");
        positive(vocab, "vocab");
        check_ids(targets_host, n, vocab, "target class");
        const int32_t *tg = cx.stage_ids(targets_host, n, 1);
        float *rows = static_cast<float *>(cx.workspace(3, (size_t)(n + 64) * 4));
        float *loss_dev = rows + ((n + 63) / 64) * 64;
        if (dlogits != logits)
            check_hip(hipMemcpyAsync(dlogits, logits, (size_t)(n * vocab) * 4,
                                     hipMemcpyDeviceToDevice, cx.stream),
                      "logits copy");
        launch_cross_entropy_fwd_bwd(cx, dlogits, tg, n, vocab, 1.0f, rows, loss_dev);
        if (loss_host) {
            check_hip(hipMemcpyAsync(loss_host, loss_dev, 4, hipMemcpyDeviceToHost, cx.stream),
                      "loss download");
            check_hip(hipStreamSynchronize(cx.stream), "loss sync");
        }
        return MMH_OK;
    });
}

}  // extern "C"
