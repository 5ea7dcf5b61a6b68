// Internal declarations shared by the libmidman_hip translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "../../include/midman_hip.h"
#include "mmh_host.h"

namespace mmh {

// An error that the C-ABI boundary turns into a status code + message.
struct Error {
    int32_t status;
    std::string message;
};

[[noreturn]] void fail(int32_t status, const std::string &message);
void check_hip(hipError_t e, const char *what);

// One device + one stream + growable workspaces.
struct Context {
    static constexpr int kSlots = 4;  // 0 split-K partials, 1 ids, 2 op temporaries, 3 losses
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t t0 = nullptr, t1 = nullptr;
    int cu_count = 0;
    std::string name;
    void *ws[kSlots] = {nullptr, nullptr, nullptr, nullptr};
    size_t ws_bytes[kSlots] = {0, 0, 0, 0};
    // Allocations made through mmh_alloc, freed at destroy.
    std::vector<void *> owned;

    void *get_scratch(size_t bytes);
    // A device buffer of at least `bytes` for this slot; growing it waits for
    // queued work first, since queued kernels may still read the old one.
    void *workspace(int slot, size_t bytes);
    // Copies n host ids into slot 1 (which = 0 inputs, 1 targets).
    int32_t *stage_ids(const int32_t *host, int64_t n, int which);
    void select() const;
};

Context &context(mmh_handle h);

// Runs an entry point body: an Error becomes its status and the thread's
// error message; any other exception becomes MMH_ERR_PANIC.
int32_t guard_impl(const std::function<int32_t()> &body);
template <class F>
int32_t guard(F &&f) {
    return guard_impl(std::function<int32_t()>(std::forward<F>(f)));
}
// Host-side id validation (ops_shape.rs:250-252, ops_reduce.rs:250-252).
void check_ids(const int32_t *ids, int64_t n, int64_t vocab, const char *what);
// Destroys the models created on a context (model.hip).
void release_models_of(mmh_handle ctx);

// ---- GEMM -----------------------------------------------------------------
// C[m,n] = epi(op(A)[m,k] op(B)[k,n]). op(A)(i,p) = A[i*lda+p] (ta=false)
// or A[p*lda+i] (ta=true); op(B)(p,j) = B[p*ldb+j] (tb=false) or B[j*ldb+p].
enum Epilogue : int { EPI_STORE = 0, EPI_ACCUM = 1, EPI_SWIGLU = 2 };

struct GemmDesc {
    const float *a = nullptr;
    const float *b = nullptr;
    float *c = nullptr;
    int64_t m = 0, n = 0, k = 0;
    int64_t lda = 0, ldb = 0, ldc = 0;
    int64_t batch = 1, stride_a = 0, stride_b = 0, stride_c = 0;
    bool ta = false, tb = false;
    int epi = EPI_STORE;
    int64_t swiglu_ff = 0;  // EPI_SWIGLU: output columns (<= n/2)
    int force_splits = 0;   // 0 = heuristic
};

void gemm(Context &ctx, const GemmDesc &d);

// ---- bandwidth kernels ------------------------------------------------------
void launch_embedding(Context &ctx, const float *table, int64_t d, const int32_t *ids_dev,
                      int64_t n, float *out);
void launch_rms_norm(Context &ctx, const float *x, const float *w, int64_t rows, int64_t d,
                     float eps, float *out);
void launch_add(Context &ctx, const float *a, const float *b, float *out, int64_t n);
void launch_silu_mul(Context &ctx, const float *g, const float *u, float *out, int64_t n);
void launch_rope(Context &ctx, const float *x, int64_t bh, int64_t t, int64_t hd,
                 const float *cos_t, const float *sin_t, float *out);
// Row losses then their f64 mean; loss_dev receives one float.
void launch_cross_entropy(Context &ctx, const float *logits, const int32_t *targets_dev,
                          int64_t n, int64_t v, float *row_loss, float *loss_dev);
void launch_pack_cols(Context &ctx, const float *src, int64_t rows, int64_t cols, float *dst,
                      int64_t ld_dst, int64_t col_off);
void launch_pack_gate_up(Context &ctx, const float *wg, const float *wu, int64_t rows,
                         int64_t ff, int64_t ff_pad, float *dst);

// ---- attention --------------------------------------------------------------
// Element (b,h,t,p) of q is q[b*sqb + h*sqh + t*sqt + p] (likewise k, v with
// the kv head, and out with the query head).
struct AttnDesc {
    const float *q, *k, *v;
    float *out;
    int64_t sqb, sqh, sqt;
    int64_t skb, skh, skt;
    int64_t svb, svh, svt;
    int64_t sob, soh, sot;
    int64_t b, h, hkv, t, hd;
    const float *cos_t = nullptr, *sin_t = nullptr;  // non-null: rotate q and k in-kernel
};
void attention(Context &ctx, const AttnDesc &d);

}  // namespace mmh
