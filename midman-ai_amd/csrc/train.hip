// Training-step kernels: the backward closures that are not GEMMs or
// attention, the global gradient norm and the fused clip + AdamW update.
//
//   cross entropy forward + backward (ops_reduce.rs:236-275), one row per
//     workgroup: rows of up to 32768 columns are held in the workgroup's
//     registers (read from HBM once: max, exp and sum, then dlogits written in
//     place over the logits); wider rows take an online max/sum pass and a
//     second pass for dlogits.
//   RMSNorm backward (norm.rs:36-38 through mul, mean_axis, add_scalar, powf):
//     one wave per row with the row in registers; the weight gradient is summed
//     per workgroup into a partial row, then over workgroups in a fixed order.
//   embedding backward (ops_shape.rs:261-269): rows of the same id are added
//     in position order from a host-built index (no atomics).
//   unpacking of the fused QKV and interleaved gate/up weight gradients into
//     the reference's parameter layout.
//   global norm (clip.rs:30-33): f64 sum of squares, fixed reduction tree.
//   clip + AdamW (clip.rs:42-60, adamw.rs:180-214): one pass over every
//     parameter; nothing is written when the loss or the norm is not finite.
// Element-wise arithmetic uses explicitly rounded intrinsics, so the update is
// the reference's operation order with no contraction.
#include <algorithm>

#include "mmh_internal.h"

namespace mmh {
namespace {

typedef float nt4 __attribute__((ext_vector_type(4)));  // the nontemporal builtins take native vectors

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// ---- cross entropy forward + backward ----------------------------------------
// row_loss[row] = max + ln(sum) - z[t]; then z[j] <- exp(z[j] - max) / sum * scale,
// minus scale at the target (ops_reduce.rs:263-272, scale = g / N).
__global__ __launch_bounds__(256) void ce_fwd_bwd_kernel(float *__restrict__ logits,
                                                         const int32_t *__restrict__ targets,
                                                         int64_t v, float scale,
                                                         float *__restrict__ row_loss, int vec) {
    constexpr int CH = 4;
    const int64_t row = blockIdx.x;
    float *z = logits + row * v;
    float4 *z4 = reinterpret_cast<float4 *>(z);
    const int64_t v4 = vec ? v / 4 : 0;
    float m = -INFINITY, s = 0.0f;
    for (int64_t j0 = threadIdx.x; j0 < v4; j0 += 256 * CH) {
        float4 a[CH];
        float cm = -INFINITY;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int64_t j = j0 + 256 * c;
            a[c] = j < v4 ? z4[j] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
            cm = fmaxf(cm, fmaxf(fmaxf(a[c].x, a[c].y), fmaxf(a[c].z, a[c].w)));
        }
        if (cm == -INFINITY) continue;
        if (cm > m) {
            s = s * expf(m - cm);
            m = cm;
        }
        float cs = 0.0f;
#pragma unroll
        for (int c = 0; c < CH; ++c)
            cs += expf(a[c].x - m) + expf(a[c].y - m) + expf(a[c].z - m) + expf(a[c].w - m);
        s += cs;
    }
    for (int64_t k = v4 * 4 + threadIdx.x; k < v; k += 256) {
        const float x = z[k];
        if (x > m) {
            s = (m == -INFINITY) ? 0.0f : s * expf(m - x);
            m = x;
        }
        s += expf(x - m);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float m2 = __shfl_xor(m, off, 64), s2 = __shfl_xor(s, off, 64);
        lse_merge(m, s, m2, s2);
    }
    __shared__ float sm[4], ss[4];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) {
        sm[wave] = m;
        ss[wave] = s;
    }
    __syncthreads();
    float M = sm[0], S = ss[0];
    for (int i = 1; i < 4; ++i) lse_merge(M, S, sm[i], ss[i]);
    const int64_t t = targets[row];
    if (threadIdx.x == 0) row_loss[row] = __fsub_rn(__fadd_rn(M, logf(S)), z[t]);
    __syncthreads();  // z[t] is read before anything is overwritten
    auto grad = [&](float x, int64_t j) {
        const float d = __fmul_rn(__fdiv_rn(expf(__fsub_rn(x, M)), S), scale);
        return j == t ? __fsub_rn(d, scale) : d;
    };
    for (int64_t j = threadIdx.x; j < v4; j += 256) {
        float4 a = z4[j];
        a.x = grad(a.x, 4 * j);
        a.y = grad(a.y, 4 * j + 1);
        a.z = grad(a.z, 4 * j + 2);
        a.w = grad(a.w, 4 * j + 3);
        z4[j] = a;
    }
    for (int64_t k = v4 * 4 + threadIdx.x; k < v; k += 256) z[k] = grad(z[k], k);
}

// The same for rows that fit the workgroup's registers (v <= 4096 * NV, v a
// multiple of 4, 16-byte aligned rows): the row is read from HBM once and
// written once. NT threads, thread l of the workgroup holding float4s l,
// l + NT, ...: the row's max, then e = exp(z - max) kept in place of z and
// their sum, then dlogits = e / sum * scale from the registers.
template <int NT>
__device__ __forceinline__ float block_max(float v, float *red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) m = fmaxf(m, red[i]);
    return m;
}

template <int NT, int NV>
__global__ __launch_bounds__(NT) void ce_fwd_bwd_regs_kernel(float *__restrict__ logits,
                                                                const int32_t *__restrict__ targets,
                                                                int64_t v, float scale,
                                                                float *__restrict__ row_loss) {
    __shared__ float red_m[NT / 64], red_s[NT / 64];
    const int64_t row = blockIdx.x;
    float4 *z4 = reinterpret_cast<float4 *>(logits + row * v);
    const int v4 = (int)(v >> 2), tid = threadIdx.x;
    const int64_t t = targets[row];
    const float zt = tid == 0 ? logits[row * v + t] : 0.0f;
    // the row streams through once each way: nontemporal loads and stores
    // (the logits, hundreds of MB, are read nowhere else; the head's backward
    // products that read the dlogits next are bound by their matrix work)
    float4 e[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int q = tid + NT * i;
        if (q < v4) {
            const nt4 t4 = __builtin_nontemporal_load(reinterpret_cast<const nt4 *>(z4 + q));
            e[i] = make_float4(t4[0], t4[1], t4[2], t4[3]);
        } else {
            e[i] = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        }
    }
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i) m = fmaxf(m, fmaxf(fmaxf(e[i].x, e[i].y), fmaxf(e[i].z, e[i].w)));
    const float M = block_max<NT>(m, red_m);
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        // positions past the row hold -inf: exp gives 0
        e[i].x = expf(__fsub_rn(e[i].x, M));
        e[i].y = expf(__fsub_rn(e[i].y, M));
        e[i].z = expf(__fsub_rn(e[i].z, M));
        e[i].w = expf(__fsub_rn(e[i].w, M));
        sum = __fadd_rn(sum, __fadd_rn(__fadd_rn(e[i].x, e[i].y), __fadd_rn(e[i].z, e[i].w)));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum = __fadd_rn(sum, __shfl_xor(sum, off, 64));
    if ((tid & 63) == 0) red_s[tid >> 6] = sum;
    __syncthreads();
    float S = red_s[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) S = __fadd_rn(S, red_s[i]);
    if (tid == 0) row_loss[row] = __fsub_rn(__fadd_rn(M, logf(S)), zt);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int q = tid + NT * i;
        if (q >= v4) continue;
        float4 d;
        d.x = __fmul_rn(__fdiv_rn(e[i].x, S), scale);
        d.y = __fmul_rn(__fdiv_rn(e[i].y, S), scale);
        d.z = __fmul_rn(__fdiv_rn(e[i].z, S), scale);
        d.w = __fmul_rn(__fdiv_rn(e[i].w, S), scale);
        const int64_t j = 4 * (int64_t)q;
        if (t >= j && t < j + 4) {
            const int c = (int)(t - j);
            if (c == 0) d.x = __fsub_rn(d.x, scale);
            if (c == 1) d.y = __fsub_rn(d.y, scale);
            if (c == 2) d.z = __fsub_rn(d.z, scale);
            if (c == 3) d.w = __fsub_rn(d.w, scale);
        }
        __builtin_nontemporal_store(nt4{d.x, d.y, d.z, d.w}, reinterpret_cast<nt4 *>(z4 + q));
    }
}

__global__ __launch_bounds__(256) void mean_f64_kernel(const float *__restrict__ row_loss,
                                                       int64_t n, float *__restrict__ out) {
    __shared__ double part[256];
    double acc = 0.0;
    for (int64_t i = threadIdx.x; i < n; i += 256) acc += (double)row_loss[i];
    part[threadIdx.x] = acc;
    __syncthreads();
    for (int stride = 128; stride > 0; stride >>= 1) {
        if ((int)threadIdx.x < stride) part[threadIdx.x] += part[threadIdx.x + stride];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[0] = (float)(part[0] / (double)n);
}

// ---- RMSNorm backward ----------------------------------------------------------
// Per row (a = mean(x^2) + eps, inv = a^-1/2 as the forward computes it):
//   dinv = sum_j (dy_j w_j) x_j, ds = dinv * (-0.5 * a^-3/2) * (1/d),
//   share_j = ((dy_j w_j) inv + ds x_j) + ds x_j,  dx_j = [dx_j +] share_j,
//   dw_j += dy_j (x_j inv).
// Workgroup = WPB waves, one row per wave. Each lane holds x, dy (and dx when
// accumulating) of the float4 columns it owns (lane + 64 i) in registers: the
// three row reads are issued together, at unconditional (clamped) addresses,
// so a wave waits for memory once. w, shared by every row, is staged in LDS.
// Each row's weight-gradient term dy (x inv) goes to LDS, and the WPB rows
// are added per column in wave order into one partial row per workgroup.
// float4 columns per lane at width d (d <= 4096)
constexpr int rms_nv(int64_t d) { return d <= 256 ? 1 : d <= 512 ? 2 : d <= 1024 ? 4 : d <= 2048 ? 8 : 16; }
// Waves (rows) per workgroup: 16 when that still leaves a workgroup for every
// CU of the part (fewer partial rows to sum), else 4, else 1; the LDS row
// terms ([WPB][64 NV] float4) stay within 128 KB (8 waves at NV 16).
// Measured at 4096 x 2048: 16 waves 20.8 / 24.6 us (without / with the dx
// accumulate read, partial sum included), 8 waves 20.7 / 25.0, 4 waves
// 21.7 / 27.0.
int rms_wpb(int64_t rows, int nv) {
    const int top = nv == 16 ? 8 : 16;
    return rows >= 256 * top ? top : rows >= 256 * 4 ? 4 : 1;
}

template <int NV, int WPB>
__global__ __launch_bounds__(64 * WPB) void rms_bwd_rows_kernel(const float *__restrict__ x,
                                                                const float *__restrict__ w,
                                                                const float *__restrict__ dy,
                                                                int64_t rows, int d, float eps,
                                                                float *__restrict__ dx,
                                                                int accumulate,
                                                                float *__restrict__ partial) {
    __shared__ float4 ws[64 * NV];
    __shared__ float4 part[WPB][64 * NV];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int d4 = d >> 2;
    const int64_t row = (int64_t)blockIdx.x * WPB + wave;
    const bool live = row < rows;
    const int64_t r = live ? row : rows - 1;  // loads stay in bounds; a dead row adds nothing
    const float4 *x4 = reinterpret_cast<const float4 *>(x + r * d);
    const float4 *g4 = reinterpret_cast<const float4 *>(dy + r * d);
    float4 *o4 = reinterpret_cast<float4 *>(dx + r * d);
    float4 xv[NV], gv[NV], ov[NV];
    // x and dy with the nontemporal hint: read once here, nothing after this
    // kernel reads them again soon (dx, which the next layer's backward reads,
    // keeps the default)
    auto ntl = [](const float4 *q) __attribute__((always_inline)) {
        const nt4 t = __builtin_nontemporal_load(reinterpret_cast<const nt4 *>(q));
        return make_float4(t[0], t[1], t[2], t[3]);
    };
    if (accumulate) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int jc = min(lane + 64 * i, d4 - 1);
            xv[i] = ntl(x4 + jc);
            gv[i] = ntl(g4 + jc);
            ov[i] = o4[jc];
        }
    } else {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int jc = min(lane + 64 * i, d4 - 1);
            xv[i] = ntl(x4 + jc);
            gv[i] = ntl(g4 + jc);
            ov[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    // w after the row loads (the wait for it then covers them too)
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    for (int j = threadIdx.x; j < 64 * NV; j += 64 * WPB)
        ws[j] = j < d4 ? w4[j] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const bool in = live && lane + 64 * i < d4;
        xv[i] = in ? xv[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        gv[i] = in ? gv[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();  // ws
    const float inv_len = __fdiv_rn(1.0f, (float)d);
    float ss = 0.0f, dinv = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const float4 wv = ws[lane + 64 * i];
        ss = __fadd_rn(ss, __fmul_rn(xv[i].x, xv[i].x));
        ss = __fadd_rn(ss, __fmul_rn(xv[i].y, xv[i].y));
        ss = __fadd_rn(ss, __fmul_rn(xv[i].z, xv[i].z));
        ss = __fadd_rn(ss, __fmul_rn(xv[i].w, xv[i].w));
        dinv = __fadd_rn(dinv, __fmul_rn(__fmul_rn(gv[i].x, wv.x), xv[i].x));
        dinv = __fadd_rn(dinv, __fmul_rn(__fmul_rn(gv[i].y, wv.y), xv[i].y));
        dinv = __fadd_rn(dinv, __fmul_rn(__fmul_rn(gv[i].z, wv.z), xv[i].z));
        dinv = __fadd_rn(dinv, __fmul_rn(__fmul_rn(gv[i].w, wv.w), xv[i].w));
    }
    ss = wave_sum(ss);
    dinv = wave_sum(dinv);
    const float a = __fadd_rn(__fmul_rn(ss, inv_len), eps);
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(a));
    const float a32 = __fmul_rn(__fmul_rn(inv, inv), inv);  // a^-3/2
    const float ds = __fmul_rn(__fmul_rn(dinv, __fmul_rn(-0.5f, a32)), inv_len);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int j = lane + 64 * i;
        const float4 wv = ws[j];
        float4 sh, pw;
#define MMH_SHARE(c)                                                                   \
    {                                                                                  \
        const float t = __fmul_rn(ds, xv[i].c);                                        \
        sh.c = __fadd_rn(__fadd_rn(__fmul_rn(__fmul_rn(gv[i].c, wv.c), inv), t), t);   \
        pw.c = __fmul_rn(gv[i].c, __fmul_rn(xv[i].c, inv));                            \
        if (accumulate) sh.c = __fadd_rn(ov[i].c, sh.c);                               \
    }
        MMH_SHARE(x)
        MMH_SHARE(y)
        MMH_SHARE(z)
        MMH_SHARE(w)
#undef MMH_SHARE
        part[wave][j] = pw;
        if (live && j < d4) o4[j] = sh;
    }
    __syncthreads();
    // column sums over the workgroup's rows, in wave (row) order
    float4 *out = reinterpret_cast<float4 *>(partial + (int64_t)blockIdx.x * d);
    for (int j = threadIdx.x; j < d4; j += 64 * WPB) {
        float4 s = part[0][j];
#pragma unroll
        for (int wv = 1; wv < WPB; ++wv) {
            const float4 o = part[wv][j];
            s.x = __fadd_rn(s.x, o.x);
            s.y = __fadd_rn(s.y, o.y);
            s.z = __fadd_rn(s.z, o.z);
            s.w = __fadd_rn(s.w, o.w);
        }
        out[j] = s;
    }
}

// Generic rows (any d): one wave per row, dx and the row's inv; the weight
// gradient is formed afterwards by the column kernel below.
__global__ __launch_bounds__(256) void rms_bwd_generic_kernel(const float *__restrict__ x,
                                                              const float *__restrict__ w,
                                                              const float *__restrict__ dy,
                                                              int64_t rows, int64_t d, float eps,
                                                              float *__restrict__ dx,
                                                              int accumulate,
                                                              float *__restrict__ inv_out) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + row * d, *gr = dy + row * d;
    float *o = dx + row * d;
    float ss = 0.0f, dinv = 0.0f;
    for (int64_t j = lane; j < d; j += 64) {
        ss = __fadd_rn(ss, __fmul_rn(xr[j], xr[j]));
        dinv = __fadd_rn(dinv, __fmul_rn(__fmul_rn(gr[j], w[j]), xr[j]));
    }
    ss = wave_sum(ss);
    dinv = wave_sum(dinv);
    const float inv_len = __fdiv_rn(1.0f, (float)d);
    const float a = __fadd_rn(__fmul_rn(ss, inv_len), eps);
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(a));
    const float a32 = __fmul_rn(__fmul_rn(inv, inv), inv);
    const float ds = __fmul_rn(__fmul_rn(dinv, __fmul_rn(-0.5f, a32)), inv_len);
    for (int64_t j = lane; j < d; j += 64) {
        const float t = __fmul_rn(ds, xr[j]);
        float sh = __fadd_rn(__fadd_rn(__fmul_rn(__fmul_rn(gr[j], w[j]), inv), t), t);
        if (accumulate) sh = __fadd_rn(o[j], sh);
        o[j] = sh;
    }
    if (lane == 0) inv_out[row] = inv;
}

// partial[chunk][j] = sum over the chunk's rows (in order) of dy * (x * inv).
__global__ __launch_bounds__(256) void rms_dw_cols_kernel(const float *__restrict__ x,
                                                          const float *__restrict__ dy,
                                                          const float *__restrict__ inv,
                                                          int64_t rows, int64_t d,
                                                          int64_t rows_per_chunk,
                                                          float *__restrict__ partial) {
    const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (j >= d) return;
    const int64_t r0 = (int64_t)blockIdx.y * rows_per_chunk;
    const int64_t r1 = min(rows, r0 + rows_per_chunk);
    float acc = 0.0f;
    for (int64_t r = r0; r < r1; ++r)
        acc = __fadd_rn(acc, __fmul_rn(dy[r * d + j], __fmul_rn(x[r * d + j], inv[r])));
    partial[(int64_t)blockIdx.y * d + j] = acc;
}

// out[j] = sum over the partial rows: workgroup = 64 columns x 16 waves; wave
// w sums rows w, w+16, w+32, ... in order (sixteen loads in flight: 256 rows
// take one round trip), then the 16 wave sums are added in wave order. Fixed
// order for a given nrows.
constexpr int SUM_WAVES = 16;

__global__ __launch_bounds__(64 * SUM_WAVES) void sum_rows_kernel(const float *__restrict__ partial,
                                                                 int64_t nrows, int64_t d,
                                                                 float *__restrict__ out) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t j = (int64_t)blockIdx.x * 64 + lane;
    float acc = 0.0f;
    if (j < d) {
        constexpr int S = SUM_WAVES;
        int64_t r = wave;
        for (; r + 15 * S < nrows; r += 16 * S) {
            float a[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) a[u] = partial[(r + u * S) * d + j];
#pragma unroll
            for (int u = 0; u < 16; ++u) acc = __fadd_rn(acc, a[u]);
        }
        for (; r < nrows; r += S) acc = __fadd_rn(acc, partial[r * d + j]);
    }
    __shared__ float part[SUM_WAVES][64];
    part[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && j < d) {
        float s = part[0][lane];
#pragma unroll
        for (int w = 1; w < SUM_WAVES; ++w) s = __fadd_rn(s, part[w][lane]);
        out[j] = s;
    }
}

// ---- embedding backward ----------------------------------------------------------
// Workgroup u owns table row ids[u]: the gradient rows at positions
// order[start[u] .. start[u+1]) are added in that (ascending) order from zero,
// then added to the row's current value when accumulate is set.
__global__ __launch_bounds__(256) void embedding_bwd_kernel(const float *__restrict__ g,
                                                            int64_t d,
                                                            const int32_t *__restrict__ uniq,
                                                            const int32_t *__restrict__ start,
                                                            const int32_t *__restrict__ order,
                                                            float *__restrict__ table,
                                                            int accumulate) {
    const int u = blockIdx.x;
    const int64_t row = uniq[u];
    const int p0 = start[u], p1 = start[u + 1];
    for (int64_t c = (int64_t)blockIdx.y * 256 + threadIdx.x; c < d; c += (int64_t)gridDim.y * 256) {
        float acc = 0.0f;
        for (int p = p0; p < p1; ++p) acc = __fadd_rn(acc, g[(int64_t)order[p] * d + c]);
        float *dst = table + row * d + c;
        *dst = accumulate ? __fadd_rn(*dst, acc) : acc;
    }
}

__global__ __launch_bounds__(256) void fill_kernel(float *__restrict__ x, int64_t n, float v) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        x[i] = v;
}

// ---- weight-gradient unpacking ------------------------------------------------------
__global__ __launch_bounds__(256) void unpack_cols_kernel(const float *__restrict__ src,
                                                          int64_t ld_src, int64_t col_off,
                                                          int64_t rows, int64_t cols,
                                                          float *__restrict__ dst, int vec) {
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const float *s = src + r * ld_src + col_off;
        float *d = dst + r * cols;
        if (vec) {
            for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < cols / 4; q += step)
                reinterpret_cast<float4 *>(d)[q] = reinterpret_cast<const float4 *>(s)[q];
        } else {
            for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < cols; c += step)
                d[c] = s[c];
        }
    }
}

// src [rows, 2*ff_pad] interleaved (2f gate, 2f+1 up) -> wg, wu [rows, ff];
// a thread moves 4 columns f of both.
__global__ __launch_bounds__(256) void unpack_gate_up_kernel(const float *__restrict__ src,
                                                             int64_t rows, int64_t ff,
                                                             int64_t ff_pad,
                                                             float *__restrict__ wg,
                                                             float *__restrict__ wu, int vec) {
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const float *s = src + r * 2 * ff_pad;
        float *g = wg + r * ff, *u = wu + r * ff;
        for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < (ff + 3) / 4;
             q += step) {
            const int64_t f = 4 * q;
            const float4 a = reinterpret_cast<const float4 *>(s)[2 * q];
            const float4 b = reinterpret_cast<const float4 *>(s)[2 * q + 1];
            if (vec) {
                reinterpret_cast<float4 *>(g)[q] = make_float4(a.x, a.z, b.x, b.z);
                reinterpret_cast<float4 *>(u)[q] = make_float4(a.y, a.w, b.y, b.w);
            } else {
                const float gv[4] = {a.x, a.z, b.x, b.z}, uv[4] = {a.y, a.w, b.y, b.w};
                for (int j = 0; j < 4 && f + j < ff; ++j) {
                    g[f + j] = gv[j];
                    u[f + j] = uv[j];
                }
            }
        }
    }
}

// ---- global norm ---------------------------------------------------------------------
constexpr int NORM_BLOCKS = 1024;

__device__ __forceinline__ double sumsq4(float4 v) {
    const double x = v.x, y = v.y, z = v.z, w = v.w;
    return (x * x + y * y) + (z * z + w * w);
}

// Thread t of block b sums the squares of float4s b*256 + t, stepping by
// NORM_BLOCKS*256, in f64 into four accumulators (four loads in flight);
// block 0 adds the n % 4 tail; then a tree inside the block. Fixed order for
// a given n.
__global__ __launch_bounds__(256) void sumsq_partial_kernel(const float *__restrict__ g,
                                                            int64_t n,
                                                            double *__restrict__ partial) {
    __shared__ double part[256];
    const int64_t n4 = n / 4, stride = (int64_t)NORM_BLOCKS * 256;
    const float4 *__restrict__ g4 = reinterpret_cast<const float4 *>(g);
    const nt4 *__restrict__ n4p = reinterpret_cast<const nt4 *>(g);
    auto ld = [&](int64_t j) __attribute__((always_inline)) {  // streamed once: nontemporal
        const nt4 t = __builtin_nontemporal_load(n4p + j);
        return make_float4(t[0], t[1], t[2], t[3]);
    };
    double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    for (; i + 3 * stride < n4; i += 4 * stride) {
        const float4 v0 = ld(i), v1 = ld(i + stride), v2 = ld(i + 2 * stride),
                     v3 = ld(i + 3 * stride);
        a0 += sumsq4(v0);
        a1 += sumsq4(v1);
        a2 += sumsq4(v2);
        a3 += sumsq4(v3);
    }
    for (; i < n4; i += stride) a0 += sumsq4(g4[i]);
    if (blockIdx.x == 0 && (int64_t)threadIdx.x < n - 4 * n4) {
        const double v = g[4 * n4 + threadIdx.x];
        a0 += v * v;
    }
    part[threadIdx.x] = (a0 + a1) + (a2 + a3);
    __syncthreads();
    for (int stride = 128; stride > 0; stride >>= 1) {
        if ((int)threadIdx.x < stride) part[threadIdx.x] += part[threadIdx.x + stride];
        __syncthreads();
    }
    if (threadIdx.x == 0) partial[blockIdx.x] = part[0];
}

__global__ __launch_bounds__(256) void norm_final_kernel(const double *__restrict__ partial,
                                                         float *__restrict__ norm) {
    __shared__ double part[256];
    double acc = 0.0;
    for (int i = threadIdx.x; i < NORM_BLOCKS; i += 256) acc += partial[i];
    part[threadIdx.x] = acc;
    __syncthreads();
    for (int stride = 128; stride > 0; stride >>= 1) {
        if ((int)threadIdx.x < stride) part[threadIdx.x] += part[threadIdx.x + stride];
        __syncthreads();
    }
    if (threadIdx.x == 0) norm[0] = (float)sqrt(part[0]);
}

// ---- clip + AdamW ----------------------------------------------------------------------
// Workgroup chunk [c0, c1) of the flat parameter list; the rank-1 ranges
// (no weight decay) that meet the chunk are gathered into LDS first.
constexpr int ADAM_CHUNK = 8192;
constexpr int ADAM_MAX_RANGES = 64;

__global__ __launch_bounds__(256) void adamw_kernel(float *__restrict__ w,
                                                    const float *__restrict__ g,
                                                    float *__restrict__ m, float *__restrict__ v,
                                                    int64_t n, const int64_t *__restrict__ ranges,
                                                    int nranges, AdamArgs a,
                                                    const float *__restrict__ loss,
                                                    const float *__restrict__ norm, bool vec) {
    const float ln = loss[0], nv = norm[0];
    if (!(isfinite(ln) && isfinite(nv))) return;  // a failed step changes nothing
    const bool clip = nv > a.clip_norm;
    const float factor = __fdiv_rn(a.clip_norm, __fadd_rn(nv, 1e-6f));  // clip.rs:52
    const int64_t c0 = (int64_t)blockIdx.x * ADAM_CHUNK;
    const int64_t c1 = min(n, c0 + ADAM_CHUNK);
    // The undecayed ranges that meet this chunk, found by all threads at
    // once (their order in the list does not matter: membership is an OR).
    __shared__ int64_t lo[ADAM_MAX_RANGES], hi[ADAM_MAX_RANGES];
    __shared__ int cnt;
    if (threadIdx.x == 0) cnt = 0;
    __syncthreads();
    for (int r = threadIdx.x; r < nranges; r += 256) {
        const int64_t s = ranges[2 * r], e = ranges[2 * r + 1];
        if (s < c1 && e > c0) {
            const int slot = atomicAdd(&cnt, 1);
            if (slot < ADAM_MAX_RANGES) {
                lo[slot] = s;
                hi[slot] = e;
            }
        }
    }
    __syncthreads();
    const int k = min(cnt, ADAM_MAX_RANGES);
    const float one_b1 = __fsub_rn(1.0f, a.beta1), one_b2 = __fsub_rn(1.0f, a.beta2);
    const float decay = __fsub_rn(1.0f, __fmul_rn(a.lr, a.weight_decay));
    auto update = [&](int64_t i, float grad, float x, float m0, float v0, float &mi, float &vi)
        __attribute__((always_inline)) {
        bool rank1 = false;
        for (int r = 0; r < k; ++r) rank1 |= (i >= lo[r] && i < hi[r]);
        if (clip) grad = __fmul_rn(grad, factor);
        if (!rank1) x = __fmul_rn(x, decay);
        mi = __fadd_rn(__fmul_rn(a.beta1, m0), __fmul_rn(one_b1, grad));
        vi = __fadd_rn(__fmul_rn(a.beta2, v0), __fmul_rn(__fmul_rn(one_b2, grad), grad));
        const float den = __fadd_rn(__fdiv_rn(__fsqrt_rn(vi), a.bias2_sqrt), a.eps);
        return __fsub_rn(x, __fdiv_rn(__fmul_rn(a.step_size, mi), den));
    };
    int64_t i0 = c0;
    if (vec) {
        // whole float4 groups of the chunk; chunks start at multiples of 4
        const int64_t q1 = c0 + ((c1 - c0) & ~int64_t(3));
#pragma unroll 4
        // Nontemporal loads and stores: every byte is touched once per step
        // (28 GB at the large preset, far past the caches); on the same access
        // mix a probe streams 5.56 TB/s with the hint against 5.23 without.
        for (int64_t i = c0 + 4 * threadIdx.x; i < q1; i += 4 * 256) {
            const nt4 g4 = __builtin_nontemporal_load(reinterpret_cast<const nt4 *>(g + i));
            const nt4 w4 = __builtin_nontemporal_load(reinterpret_cast<const nt4 *>(w + i));
            const nt4 m4 = __builtin_nontemporal_load(reinterpret_cast<const nt4 *>(m + i));
            const nt4 v4 = __builtin_nontemporal_load(reinterpret_cast<const nt4 *>(v + i));
            nt4 wo, mo, vo;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float mi, vi;
                wo[e] = update(i + e, g4[e], w4[e], m4[e], v4[e], mi, vi);
                mo[e] = mi;
                vo[e] = vi;
            }
            __builtin_nontemporal_store(mo, reinterpret_cast<nt4 *>(m + i));
            __builtin_nontemporal_store(vo, reinterpret_cast<nt4 *>(v + i));
            __builtin_nontemporal_store(wo, reinterpret_cast<nt4 *>(w + i));
        }
        i0 = q1;
    }
    for (int64_t i = i0 + threadIdx.x; i < c1; i += 256) {
        float mi, vi;
        const float x = update(i, g[i], w[i], m[i], v[i], mi, vi);
        m[i] = mi;
        v[i] = vi;
        w[i] = x;
    }
}

unsigned grid_for(int64_t work, int per_block = 256) {
    int64_t b = (work + per_block - 1) / per_block;
    if (b < 1) b = 1;
    if (b > 65536) b = 65536;
    return (unsigned)b;
}

bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

void launch_cross_entropy_fwd_bwd(Context &ctx, float *logits, const int32_t *targets_dev,
                                  int64_t n, int64_t v, float g, float *row_loss,
                                  float *loss_dev) {
    if (n > 0x7fffffff) fail(MMH_ERR_SHAPE, "cross_entropy: too many rows");
    const int vec = (v % 4 == 0) && al16(logits);
    const float scale = g / (float)n;
    const dim3 grid((unsigned)n);
    // rows held in registers (read once) up to 32768 columns
    if (vec && v <= 32768) {
        // (the widest rows on 512 threads: 2 workgroups of 106 VGPRs share
        // a CU, where one 1024-thread workgroup would hold it alone)
        if (v <= 4096)
            hipLaunchKernelGGL((ce_fwd_bwd_regs_kernel<1024, 1>), grid, dim3(1024), 0, ctx.stream, logits, targets_dev, v, scale, row_loss);
        else if (v <= 8192)
            hipLaunchKernelGGL((ce_fwd_bwd_regs_kernel<1024, 2>), grid, dim3(1024), 0, ctx.stream, logits, targets_dev, v, scale, row_loss);
        else if (v <= 16384)
            hipLaunchKernelGGL((ce_fwd_bwd_regs_kernel<1024, 4>), grid, dim3(1024), 0, ctx.stream, logits, targets_dev, v, scale, row_loss);
        else
            hipLaunchKernelGGL((ce_fwd_bwd_regs_kernel<512, 16>), grid, dim3(512), 0, ctx.stream, logits, targets_dev, v, scale, row_loss);
    } else {
        hipLaunchKernelGGL(ce_fwd_bwd_kernel, grid, dim3(256), 0, ctx.stream, logits,
                           targets_dev, v, scale, row_loss, vec);
    }
    check_hip(hipGetLastError(), "cross_entropy backward launch");
    hipLaunchKernelGGL(mean_f64_kernel, dim3(1), dim3(256), 0, ctx.stream, row_loss, n,
                       loss_dev);
    check_hip(hipGetLastError(), "loss mean launch");
}

int64_t rms_norm_backward_scratch(int64_t rows, int64_t d) {
    // partial rows (fast path: one per workgroup of rms_wpb rows; generic: row
    // chunks of 64) plus one inv per row.
    // (rms_wpb gives 1 below 1024 rows and at least 4 from there)
    const int64_t fast = d > 4096 ? 0 : rows < 1024 ? rows : (rows + 3) / 4;
    const int64_t generic = (rows + 63) / 64;
    return std::max(fast, generic) * d + rows;
}

void launch_rms_norm_backward(Context &ctx, const float *x, const float *w, const float *dy,
                              int64_t rows, int64_t d, float eps, float *dx, bool accumulate,
                              float *dw, float *scratch) {
    // (the rows kernel clamps its column index to d/4 - 1: d >= 4)
    const int vec = (d % 4 == 0) && d >= 4 && d <= 4096 && al16(x) && al16(w) && al16(dy) &&
                    al16(dx) && al16(scratch);
    if (vec) {
        // one row per wave, rms_wpb waves per workgroup
        const int nv = rms_nv(d), wpb = rms_wpb(rows, nv);
        const int64_t blocks = (rows + wpb - 1) / wpb;
        if (blocks > 0x7fffffff) fail(MMH_ERR_SHAPE, "rms_norm backward: too many rows");
        const dim3 grid((unsigned)blocks), block(64 * wpb);
        const int dd = (int)d, acc = accumulate ? 1 : 0;
#define MMH_RMS_LAUNCH(NV, W)                                                                     \
    hipLaunchKernelGGL((rms_bwd_rows_kernel<NV, W>), grid, block, 0, ctx.stream, x, w, dy, rows, \
                       dd, eps, dx, acc, scratch)
#define MMH_RMS_WAVES(NV, TOP)       \
    if (wpb == TOP)                  \
        MMH_RMS_LAUNCH(NV, TOP);     \
    else if (wpb == 4)               \
        MMH_RMS_LAUNCH(NV, 4);       \
    else                             \
        MMH_RMS_LAUNCH(NV, 1);
        if (nv == 1) {
            MMH_RMS_WAVES(1, 16)
        } else if (nv == 2) {
            MMH_RMS_WAVES(2, 16)
        } else if (nv == 4) {
            MMH_RMS_WAVES(4, 16)
        } else if (nv == 8) {
            MMH_RMS_WAVES(8, 16)
        } else {
            MMH_RMS_WAVES(16, 8)
        }
#undef MMH_RMS_WAVES
#undef MMH_RMS_LAUNCH
        check_hip(hipGetLastError(), "rms_norm backward launch");
        hipLaunchKernelGGL(sum_rows_kernel, dim3(grid_for(d, 64)), dim3(64 * SUM_WAVES), 0,
                           ctx.stream, scratch, blocks, d, dw);
        check_hip(hipGetLastError(), "rms_norm dw launch");
        return;
    }
    const int64_t chunks = (rows + 63) / 64;
    float *inv = scratch + chunks * d;
    hipLaunchKernelGGL(rms_bwd_generic_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                       ctx.stream, x, w, dy, rows, d, eps, dx, accumulate ? 1 : 0, inv);
    check_hip(hipGetLastError(), "rms_norm backward launch");
    hipLaunchKernelGGL(rms_dw_cols_kernel, dim3(grid_for(d), (unsigned)chunks), dim3(256), 0,
                       ctx.stream, x, dy, inv, rows, d, (int64_t)64, scratch);
    check_hip(hipGetLastError(), "rms_norm dw launch");
    hipLaunchKernelGGL(sum_rows_kernel, dim3(grid_for(d, 64)), dim3(64 * SUM_WAVES), 0, ctx.stream,
                       scratch, chunks, d, dw);
    check_hip(hipGetLastError(), "rms_norm dw launch");
}

void launch_embedding_backward(Context &ctx, const float *g, int64_t d, const int32_t *uniq,
                               const int32_t *start, const int32_t *order, int64_t n_unique,
                               float *table, bool accumulate) {
    if (n_unique <= 0) return;
    if (n_unique > 0x7fffffff) fail(MMH_ERR_SHAPE, "embedding backward: too many ids");
    const unsigned ycols = (unsigned)std::min<int64_t>((d + 255) / 256, 16);
    hipLaunchKernelGGL(embedding_bwd_kernel, dim3((unsigned)n_unique, ycols), dim3(256), 0,
                       ctx.stream, g, d, uniq, start, order, table, accumulate ? 1 : 0);
    check_hip(hipGetLastError(), "embedding backward launch");
}

void launch_fill(Context &ctx, float *x, int64_t n, float v) {
    hipLaunchKernelGGL(fill_kernel, dim3(grid_for(n)), dim3(256), 0, ctx.stream, x, n, v);
    check_hip(hipGetLastError(), "fill launch");
}

void launch_unpack_cols(Context &ctx, const float *src, int64_t ld_src, int64_t col_off,
                        int64_t rows, int64_t cols, float *dst) {
    const int vec = cols % 4 == 0 && ld_src % 4 == 0 && col_off % 4 == 0 && al16(src) && al16(dst);
    const int64_t units = vec ? cols / 4 : cols;
    const dim3 grid((unsigned)std::max<int64_t>(1, std::min<int64_t>((units + 255) / 256, 64)),
                    (unsigned)std::max<int64_t>(1, std::min<int64_t>(rows, 65535)));
    hipLaunchKernelGGL(unpack_cols_kernel, grid, dim3(256), 0, ctx.stream, src, ld_src, col_off,
                       rows, cols, dst, vec);
    check_hip(hipGetLastError(), "unpack launch");
}

void launch_unpack_gate_up(Context &ctx, const float *src, int64_t rows, int64_t ff,
                           int64_t ff_pad, float *wg, float *wu) {
    if (ff_pad % 4 || ff_pad < ff || !al16(src))
        fail(MMH_ERR_ARGUMENT, "unpack: padded rows must be float4s");
    const int vec = ff % 4 == 0 && al16(wg) && al16(wu);
    const dim3 grid((unsigned)std::max<int64_t>(1, std::min<int64_t>(((ff + 3) / 4 + 255) / 256, 64)),
                    (unsigned)std::max<int64_t>(1, std::min<int64_t>(rows, 65535)));
    hipLaunchKernelGGL(unpack_gate_up_kernel, grid, dim3(256), 0, ctx.stream, src, rows, ff,
                       ff_pad, wg, wu, vec);
    check_hip(hipGetLastError(), "unpack launch");
}

int64_t global_norm_scratch_bytes() { return (int64_t)NORM_BLOCKS * 8; }

void launch_global_norm(Context &ctx, const float *g, int64_t n, double *scratch, float *norm) {
    hipLaunchKernelGGL(sumsq_partial_kernel, dim3(NORM_BLOCKS), dim3(256), 0, ctx.stream, g, n,
                       scratch);
    check_hip(hipGetLastError(), "norm launch");
    hipLaunchKernelGGL(norm_final_kernel, dim3(1), dim3(256), 0, ctx.stream, scratch, norm);
    check_hip(hipGetLastError(), "norm launch");
}

int64_t adamw_max_ranges_per_chunk(const int64_t *ranges_host, int nranges, int64_t n) {
    int64_t worst = 0;
    for (int64_t c0 = 0; c0 < n; c0 += ADAM_CHUNK) {
        const int64_t c1 = std::min<int64_t>(n, c0 + ADAM_CHUNK);
        int64_t k = 0;
        for (int r = 0; r < nranges; ++r)
            if (ranges_host[2 * r] < c1 && ranges_host[2 * r + 1] > c0) ++k;
        worst = std::max(worst, k);
    }
    return worst;
}

void launch_adamw(Context &ctx, float *w, const float *g, float *m, float *v, int64_t n,
                  const int64_t *ranges_dev, int nranges, int64_t max_per_chunk,
                  const AdamArgs &a, const float *loss_dev, const float *norm_dev) {
    if (max_per_chunk > ADAM_MAX_RANGES)
        fail(MMH_ERR_ARGUMENT, "adamw: too many undecayed parameters in one chunk");
    const int64_t blocks = (n + ADAM_CHUNK - 1) / ADAM_CHUNK;
    if (blocks > 0x7fffffff) fail(MMH_ERR_SHAPE, "adamw: too many parameters");
    const bool vec = al16(w) && al16(g) && al16(m) && al16(v);
    hipLaunchKernelGGL(adamw_kernel, dim3((unsigned)blocks), dim3(256), 0, ctx.stream, w, g, m,
                       v, n, ranges_dev, nranges, a, loss_dev, norm_dev, vec);
    check_hip(hipGetLastError(), "adamw launch");
}

}  // namespace mmh
