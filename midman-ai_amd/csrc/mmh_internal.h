// Internal declarations shared by the libmidman_hip translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "../../include/midman_hip.h"
#include "mmh_error.h"
#include "mmh_host.h"

namespace mmh {

// silu (ops_elementwise.rs:239-241, :355-364): x * (1 / (1 + e^-x)).
__device__ __forceinline__ float silu_f(float x) {
    const float s = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-x)));
    return __fmul_rn(x, s);
}
// silu through the hardware exp2 and reciprocal (a few ulp from silu_f): 5
// VALU instructions instead of ~25 for the libm exp and the IEEE division.
// The VALU's cycles add to the matrix core's on a SIMD, so the 128x128 GEMM
// epilogue that finishes SwiGLU takes this form.
__device__ __forceinline__ float silu_fast(float x) {
    const float e = __builtin_amdgcn_exp2f(x * -1.4426950408889634f);
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// Backward of h = silu(g) * u (mul then silu, ops_elementwise.rs:287, :355-364):
// dsilu = dh*u, du = dh*silu(g), dg = dsilu * s*(1 + g*(1 - s)); returns (dg, du).
__device__ __forceinline__ float2 swiglu_bwd_f(float dh, float g, float u) {
    const float s = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-g)));
    const float sv = __fmul_rn(g, s);
    const float dsilu = __fmul_rn(dh, u);
    const float du = __fmul_rn(dh, sv);
    const float deriv = __fmul_rn(s, __fadd_rn(1.0f, __fmul_rn(g, __fsub_rn(1.0f, s))));
    return make_float2(__fmul_rn(dsilu, deriv), du);
}

// Merges a log-sum-exp pair (m2, s2) into (m, s): the pair (max, sum of
// exp(z - max)) of the union, -inf / 0 standing for an empty set.
__device__ __forceinline__ void lse_merge(float &m, float &s, float m2, float s2) {
    if (m2 == -INFINITY) return;
    if (m == -INFINITY) {
        m = m2;
        s = s2;
        return;
    }
    if (m2 > m) {
        s = s * expf(m - m2) + s2;
        m = m2;
    } else {
        s = s + s2 * expf(m2 - m);
    }
}

void check_hip(hipError_t e, const char *what);

// One device + one stream + growable workspaces.
struct Context {
    // 0 split-K partials, 1 ids, 2 op temporaries, 3 losses, 4 attention heads
    // padded to a kernel width
    static constexpr int kSlots = 5;
    static constexpr int kPadSlot = 4;
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t t0 = nullptr, t1 = nullptr;
    int cu_count = 0;
    // 8 XCDs, each dealt cu_count / 8 of a cu_count-workgroup grid (probed at
    // creation): what the fused forward's per-XCD teams need
    bool xcd_teams = false;
    // the dispatch deals workgroup b to XCD (b + o) % 8 with o fixed per
    // launch (checked at creation): the fused forward's team slots are b / 8
    bool xcd_rr = false;
    std::string name;
    void *ws[kSlots] = {};
    size_t ws_bytes[kSlots] = {};
    // One counter per output tile of a K-split GEMM (zero between launches:
    // the last split of a tile resets its counter), allocated and zeroed
    // with the context.
    static constexpr int kTickets = 4096;
    int32_t *tickets = nullptr;
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

// Host-side id validation (ops_shape.rs:250-252, ops_reduce.rs:250-252).
void check_ids(const int32_t *ids, int64_t n, int64_t vocab, const char *what);
// Destroys the models created on a context (model.hip).
void release_models_of(mmh_handle ctx);

// ---- GEMM -----------------------------------------------------------------
// C[m,n] = epi(op(A)[m,k] op(B)[k,n]). op(A)(i,p) = A[i*lda+p] (ta=false)
// or A[p*lda+i] (ta=true); op(B)(p,j) = B[p*ldb+j] (tb=false) or B[j*ldb+p].
// EPI_STORE: C = acc. EPI_ACCUM: C = R + acc with R = resid, or C itself.
// EPI_SWIGLU: columns (2f, 2f+1) are (gate f, up f); C[row][f] = silu(gate)*up,
// and aux (when set) receives the raw pair. EPI_SWIGLU_BWD: acc is dh [M, ff];
// with (g, u) = aux[row][2f, 2f+1], C[row][2f, 2f+1] = (dg, du) (C may be aux).
// EPI_CE: C is not written; the products are logits, and each 128-column tile
// tn of row i leaves ce_part[(i * tiles + tn) * 2 + {0, 1}] = (max, sum of
// exp(z - max)) over its columns, and the tile holding column ce_targets[i]
// leaves that logit in ce_zt[i] (the head GEMM with the loss folded in; see
// gemm_ce_tiles and launch_ce_combine).
enum Epilogue : int { EPI_STORE = 0, EPI_ACCUM = 1, EPI_SWIGLU = 2, EPI_SWIGLU_BWD = 3,
                      EPI_CE = 4 };

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
    const float *resid = nullptr;  // EPI_ACCUM: residual source (ldc layout); null = C
    float *aux = nullptr;          // EPI_SWIGLU(_BWD): interleaved gate/up pairs
    int64_t ldaux = 0;
    int force_splits = 0;   // 0 = heuristic
    // RMSNorm of A's rows first (norm.rs:21-39; nn form, batch 1): A is x and
    // the product uses (x * inv) * norm_w with inv = (mean(x^2) + eps)^-1/2.
    // Folded into the small-tile kernel's loads when K <= 256; otherwise the
    // norm runs as its own kernel into norm_tmp ([m, k]) first.
    const float *norm_w = nullptr;
    float norm_eps = 0.0f;
    float *norm_tmp = nullptr;
    // RoPE (rope.rs:28-32) on the result's columns [0, rope_cols): heads of
    // rope_hd columns, row r at position r % rope_seq; applied in the small
    // kernel's epilogue when a head fits a wave's 32 columns (EPI_STORE),
    // otherwise by the rope kernel after the product. Same bits either way.
    const float *rope_cos = nullptr, *rope_sin = nullptr;
    int64_t rope_seq = 0, rope_hd = 0, rope_cols = 0;
    // EPI_CE (batch 1, the 128x128 kernel only): targets [m] on the device,
    // partials [m, gemm_ce_tiles, 2] and target logits [m] out.
    const int32_t *ce_targets = nullptr;
    float *ce_part = nullptr, *ce_zt = nullptr;
    // Device memory for the split-K partials supplied by the caller (null: the
    // context's growable workspace). gemm() fails with MMH_ERR_SHAPE when the
    // partials of the split it chooses need more than scratch_bytes.
    float *scratch = nullptr;
    size_t scratch_bytes = 0;
    // With scratch: kTickets zeroed tile counters for the in-kernel split
    // reduction (null: the context's own).
    int32_t *scratch_tickets = nullptr;
    // EPI_ACCUM with the GEMM seam's rule (kernels.rs:48, C += A.B): C's own
    // value starts the sum. Without it EPI_ACCUM is a residual add of a fresh
    // product (block.rs:79-80: x + matmul(..), the product summed from +0).
    // The two differ only in the sign of an exact zero.
    bool accumulate_into_c = false;
};

void gemm(Context &ctx, const GemmDesc &d);
// Whether gemm() folds the A-row norm and the RoPE of d into its kernel (so a
// caller can time or schedule them as kernels of their own otherwise).
struct GemmFusion {
    bool norm = false, rope = false;
};
GemmFusion gemm_fusion(const Context &ctx, const GemmDesc &d);
// Column tiles of an EPI_CE product of d's shape (the partials per row), or 0
// when the loss cannot fold into it (the small-shape kernels, batches).
int64_t gemm_ce_tiles(const Context &ctx, const GemmDesc &d);
// TFLOP/s of an fp32 MFMA issue-rate probe (register operands, no memory
// traffic) over the whole chip; uses the context's scratch and its events.
double mfma_peak_tflops(Context &ctx);

// ---- bandwidth kernels ------------------------------------------------------
void launch_embedding(Context &ctx, const float *table, int64_t d, const int32_t *ids_dev,
                      int64_t n, float *out);
void launch_rms_norm(Context &ctx, const float *x, const float *w, int64_t rows, int64_t d,
                     float eps, float *out);
void launch_add(Context &ctx, const float *a, const float *b, float *out, int64_t n);
void launch_silu_mul(Context &ctx, const float *g, const float *u, float *out, int64_t n);
// (dg, du) of h = silu(g) * u for the incoming dh; dg and du may alias g and u.
void launch_silu_mul_backward(Context &ctx, const float *dh, float *g, float *u, float *dg,
                              float *du, int64_t n);
void launch_rope(Context &ctx, const float *x, int64_t bh, int64_t t, int64_t hd,
                 const float *cos_t, const float *sin_t, float *out);
// Row losses then their f64 mean; loss_dev receives one float.
void launch_cross_entropy(Context &ctx, const float *logits, const int32_t *targets_dev,
                          int64_t n, int64_t v, float *row_loss, float *loss_dev);
// The loss from the partials of an EPI_CE head GEMM: each row's (max, sum)
// pairs merged over its tiles, row loss = max + ln(sum) - z[target], then the
// f64 mean as launch_cross_entropy.
void launch_ce_combine(Context &ctx, const float *part, int64_t tiles, const float *zt,
                       int64_t n, float *row_loss, float *loss_dev);
void launch_pack_cols(Context &ctx, const float *src, int64_t rows, int64_t cols, float *dst,
                      int64_t ld_dst, int64_t col_off);
void launch_pack_gate_up(Context &ctx, const float *wg, const float *wu, int64_t rows,
                         int64_t ff, int64_t ff_pad, float *dst);

// ---- training step ----------------------------------------------------------
// Loss (row terms + f64 mean) and, in place, dlogits = (softmax - onehot) * g/N.
void launch_cross_entropy_fwd_bwd(Context &ctx, float *logits, const int32_t *targets_dev,
                                  int64_t n, int64_t v, float g, float *row_loss,
                                  float *loss_dev);
// Floats of scratch launch_rms_norm_backward needs for (rows, d).
int64_t rms_norm_backward_scratch(int64_t rows, int64_t d);
// dx = [dx +] the norm's share of d(x); dw overwritten.
void launch_rms_norm_backward(Context &ctx, const float *x, const float *w, const float *dy,
                              int64_t rows, int64_t d, float eps, float *dx, bool accumulate,
                              float *dw, float *scratch);
// table[uniq[u]] = [table +] sum of g rows order[start[u] .. start[u+1]).
void launch_embedding_backward(Context &ctx, const float *g, int64_t d, const int32_t *uniq,
                               const int32_t *start, const int32_t *order, int64_t n_unique,
                               float *table, bool accumulate);
void launch_fill(Context &ctx, float *x, int64_t n, float v);
void launch_unpack_cols(Context &ctx, const float *src, int64_t ld_src, int64_t col_off,
                        int64_t rows, int64_t cols, float *dst);
void launch_unpack_gate_up(Context &ctx, const float *src, int64_t rows, int64_t ff,
                           int64_t ff_pad, float *wg, float *wu);
int64_t global_norm_scratch_bytes();
void launch_global_norm(Context &ctx, const float *g, int64_t n, double *scratch, float *norm);
struct AdamArgs {
    float lr, beta1, beta2, eps, weight_decay, clip_norm;
    float step_size, bias2_sqrt;  // lr / (1 - beta1^t), sqrt(1 - beta2^t) (adamw.rs:185-188)
};
// ranges: [start, end) pairs of parameters that do not decay (rank 1).
int64_t adamw_max_ranges_per_chunk(const int64_t *ranges_host, int nranges, int64_t n);
void launch_adamw(Context &ctx, float *w, const float *g, float *m, float *v, int64_t n,
                  const int64_t *ranges_dev, int nranges, int64_t max_per_chunk,
                  const AdamArgs &a, const float *loss_dev, const float *norm_dev);

// ---- fused forward (fused_forward.hip) --------------------------------------
// The loss-only forward of a small model as one persistent launch: per-XCD
// teams of workgroups, each owning the sequences s with s % 8 == its XCD.
struct FusedShape {
    int64_t batch = 0, seq = 0, d = 0, heads = 0, kv_heads = 0, ff = 0, ff_pad = 0, vocab = 0,
            layers = 0, max_seq = 0;
    bool tie = true;
    float eps = 0.0f;
    int64_t weight_floats = 0;  // the device weight layout's size
};
// The fused kernel's arena: every buffer it writes plus a copy of the rotary
// tables, as float offsets of one allocation, each region between guard
// bands (filled with the model's guard word at allocation).
struct FusedLayout {
    static constexpr int64_t kBand = 64;  // guard band floats around each region
    int64_t qc = 0, nrb = 0, smax = 0, nsi = 0, ctl_ints = 0, tab_floats = 0;
    int64_t bands[24] = {};  // float offsets of the guard bands
    int nbands = 0;
    int64_t o_x = 0, o_h = 0, o_qkv = 0, o_part = 0, o_zt = 0, o_rl = 0, o_p64 = 0,
            o_ctl = 0, o_err = 0, o_cos = 0, o_sin = 0, o_op = 0, o_x2 = 0;
    int64_t floats = 0;
};
struct FusedArgs {
    FusedShape shape;
    const float *w = nullptr;
    int64_t off_block0 = 0, block_floats = 0, off_final_norm = 0;
    const int32_t *ids = nullptr, *tgt = nullptr;  // tgt after ids in one allocation
    float *loss = nullptr;
    // fused_layout(shape).floats floats: counters (the exit ticket, the team
    // slots of the 8 XCDs, the task counters) and error word zero before
    // the first launch, the rotary tables at o_cos / o_sin
    float *arena = nullptr;
    // diagnostic: when set, workgroup g stores the device's constant-rate
    // clock at its start and its end into stamps[2g], stamps[2g + 1]
    uint64_t *stamps = nullptr;
};
// Whether the fused kernel takes this shape (heads of 16 or 32, d a multiple
// of 32 up to 256, ff a multiple of 4, at most 16384 rows, 32-bit offsets)
// on this device (ctx.xcd_teams).
bool fused_forward_fits(const Context &ctx, const FusedShape &s);
// Launches one workgroup per CU and checks that 8 XCDs take cu_count / 8 each
// (false on a device partitioned otherwise, or on any error).
bool probe_xcd_teams(Context &ctx);
FusedLayout fused_layout(const FusedShape &s);
// Queues the forward + loss; the loss lands in a.loss, the row losses in
// a.row_loss. The counters are back at zero when the launch ends.
void launch_fused_forward(Context &ctx, const FusedArgs &a);

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
    float *lse = nullptr;  // non-null: per-row log2-sum-exp2 of the scaled scores, [B,H,T]
};
void attention(Context &ctx, const AttnDesc &d);

// Backward of attention() from its saved lse. q and k are the rows the
// forward read (rotated in place when it had tables); o is its output and do
// the output gradient, both with the out strides. dq/dk/dv take the q/k/v
// strides and are overwritten; with tables set, dq and dk are rotated back
// (RoPE backward) at the end. dvec is [B*H*T] scratch (rowsum(dO*O)).
struct AttnBwdDesc {
    const float *q, *k, *v, *o, *dout, *lse;
    float *dq, *dk, *dv, *dvec;
    int64_t sqb, sqh, sqt;
    int64_t skb, skh, skt;
    int64_t svb, svh, svt;
    int64_t sob, soh, sot;
    int64_t b, h, hkv, t, hd;
    const float *cos_t = nullptr, *sin_t = nullptr;
    // Optional, attention_backward_scratch_floats() floats: with GQA the
    // query heads then run as separate workgroups (better balanced) and their
    // partial dK, dV are summed in head order.
    float *scratch = nullptr;
};
int64_t attention_backward_scratch_floats(int64_t b, int64_t h, int64_t hkv, int64_t t,
                                          int64_t hd);
void attention_backward(Context &ctx, const AttnBwdDesc &d);
// In-place RoPE on strided heads; inverse rotates by -angle (the backward).
void launch_rope_strided(Context &ctx, float *x, int64_t sb, int64_t sh, int64_t st, int64_t nb,
                         int64_t nh, int64_t t, int64_t hd, const float *cos_t,
                         const float *sin_t, bool inverse = false);
// q and k heads rotated in place (one launch when k's heads follow q's in each
// row, as in the fused QKV layout).
void rope_qk(Context &ctx, float *q, float *k, int64_t sqb, int64_t sqh, int64_t sqt, int64_t skb,
             int64_t skh, int64_t skt, int64_t b, int64_t h, int64_t hkv, int64_t t, int64_t hd,
             const float *cos_t, const float *sin_t, bool inverse);
// Head widths the attention kernels take directly; kernel_head(hd) is the
// smallest of them >= hd (0 above 128): other even widths run on it through
// zero-padded copies of the heads.
bool native_head(int64_t hd);
int64_t kernel_head(int64_t hd);
// [nb, nh, t, hd] heads at strides (sb, sh, st) into contiguous [nb, nh, t, hp]
// with zeros beyond hd, and back (columns below hd only).
void launch_pad_heads(Context &ctx, const float *src, int64_t sb, int64_t sh, int64_t st,
                      int64_t nb, int64_t nh, int64_t t, int64_t hd, float *dst, int64_t hp);
void launch_unpad_heads(Context &ctx, const float *src, int64_t hp, int64_t nb, int64_t nh,
                        int64_t t, int64_t hd, float *dst, int64_t sb, int64_t sh, int64_t st);

}  // namespace mmh
