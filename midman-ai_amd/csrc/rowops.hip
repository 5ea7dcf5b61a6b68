// Bandwidth-bound kernels of the decoder path: embedding gather, RMSNorm,
// residual add, silu*mul, RoPE, the cross-entropy loss and weight packing.
//
// Each reads its inputs once and writes its outputs once with float4 accesses
// where the row length allows, and reduces within a wave64 with DPP/shuffles.
// Element-wise arithmetic uses the explicitly rounded intrinsics
// (__fmul_rn, __fadd_rn, ...) so that no multiply-add is contracted and each
// operation rounds exactly where the reference's does; that makes the
// embedding, RoPE and add bit-exact, and leaves RMSNorm and the loss differing
// from the reference only by summation order.
#include <algorithm>

#include "mmh_internal.h"

namespace mmh {
namespace {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// ---- embedding: ops_shape.rs:249-257 ---------------------------------------
__global__ __launch_bounds__(256) void embedding_kernel(const float *__restrict__ table,
                                                        int64_t d, const int32_t *__restrict__ ids,
                                                        int64_t n, float *__restrict__ out,
                                                        int vec) {
    const int64_t total = vec ? n * (d / 4) : n * d;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        if (vec) {
            const int64_t d4 = d / 4, row = i / d4, c = i - row * d4;
            const float4 v = reinterpret_cast<const float4 *>(table + (int64_t)ids[row] * d)[c];
            reinterpret_cast<float4 *>(out + row * d)[c] = v;
        } else {
            const int64_t row = i / d, c = i - row * d;
            out[i] = table[(int64_t)ids[row] * d + c];
        }
    }
}

// Row-major form for float4 rows of d4 = RPW-dividing or 256-multiple
// lengths: a workgroup owns RPW rows (256 / RPW threads each) and a thread
// copies U float4s of its row, all U loads issued before the stores. The
// row's id is read once (per thread group), not once per float4, and there
// is no per-element index division.
template <int RPW, int U>
__global__ __launch_bounds__(256) void embedding_rows_kernel(const float *__restrict__ table,
                                                             int64_t d, const int32_t *__restrict__ ids,
                                                             int64_t n, float *__restrict__ out) {
    constexpr int TPR = 256 / RPW;  // threads per row
    const int64_t row = (int64_t)blockIdx.x * RPW + threadIdx.x / TPR;
    if (row >= n) return;
    const int t = threadIdx.x % TPR;
    const float4 *__restrict__ src = reinterpret_cast<const float4 *>(table + (int64_t)ids[row] * d);
    float4 *__restrict__ dst = reinterpret_cast<float4 *>(out + row * d);
    float4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = src[t + u * TPR];
#pragma unroll
    for (int u = 0; u < U; ++u) dst[t + u * TPR] = v[u];
}

// ---- RMSNorm: norm.rs:36-38 -------------------------------------------------
// One wave per row: sum of squares (wave reduction), mean = sum * (1/d),
// inv = (mean + eps)^(-1/2), out = (x * inv) * w.
__global__ __launch_bounds__(256) void rms_norm_kernel(const float *__restrict__ x,
                                                       const float *__restrict__ w, int64_t rows,
                                                       int64_t d, float eps,
                                                       float *__restrict__ out, int vec) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *xr = x + row * d;
    float *o = out + row * d;
    float ss = 0.0f;
    if (vec) {
        const float4 *x4 = reinterpret_cast<const float4 *>(xr);
        for (int64_t j = lane; j < d / 4; j += 64) {
            const float4 v = x4[j];
            ss = __fadd_rn(ss, __fmul_rn(v.x, v.x));
            ss = __fadd_rn(ss, __fmul_rn(v.y, v.y));
            ss = __fadd_rn(ss, __fmul_rn(v.z, v.z));
            ss = __fadd_rn(ss, __fmul_rn(v.w, v.w));
        }
    } else {
        for (int64_t j = lane; j < d; j += 64) ss = __fadd_rn(ss, __fmul_rn(xr[j], xr[j]));
    }
    ss = wave_sum(ss);
    const float mean = __fmul_rn(ss, __fdiv_rn(1.0f, (float)d));
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, eps)));
    if (vec) {
        const float4 *x4 = reinterpret_cast<const float4 *>(xr);
        const float4 *w4 = reinterpret_cast<const float4 *>(w);
        float4 *o4 = reinterpret_cast<float4 *>(o);
        for (int64_t j = lane; j < d / 4; j += 64) {
            const float4 v = x4[j], g = w4[j];
            float4 r;
            r.x = __fmul_rn(__fmul_rn(v.x, inv), g.x);
            r.y = __fmul_rn(__fmul_rn(v.y, inv), g.y);
            r.z = __fmul_rn(__fmul_rn(v.z, inv), g.z);
            r.w = __fmul_rn(__fmul_rn(v.w, inv), g.w);
            o4[j] = r;
        }
    } else {
        for (int64_t j = lane; j < d; j += 64) o[j] = __fmul_rn(__fmul_rn(xr[j], inv), w[j]);
    }
}

// The same for rows of d <= 256*NV floats (d % 4 == 0): the wave keeps its row
// in registers, so x is read once, and all NV float4 loads per lane (and the
// matching w ones) are issued before the first is used: at clamped,
// unconditional addresses (a guarded load per float4 was compiled into its
// own branch, and each w load after the reduction into a round trip before
// its store), the columns past d then zeroed by selects.
template <int NV>
__global__ __launch_bounds__(256) void rms_norm_rows_kernel(const float *__restrict__ x,
                                                            const float *__restrict__ w,
                                                            int64_t rows, int d, float eps,
                                                            float *__restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int d4 = d >> 2;
    const float4 *x4 = reinterpret_cast<const float4 *>(x + row * d);
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    float4 v[NV], wv[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int jc = min(lane + 64 * i, d4 - 1);
        v[i] = x4[jc];
        wv[i] = w4[jc];
    }
    if (d4 < 64 * NV) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const bool in = lane + 64 * i < d4;
            v[i].x = in ? v[i].x : 0.0f;
            v[i].y = in ? v[i].y : 0.0f;
            v[i].z = in ? v[i].z : 0.0f;
            v[i].w = in ? v[i].w : 0.0f;
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        ss = __fadd_rn(ss, __fmul_rn(v[i].x, v[i].x));
        ss = __fadd_rn(ss, __fmul_rn(v[i].y, v[i].y));
        ss = __fadd_rn(ss, __fmul_rn(v[i].z, v[i].z));
        ss = __fadd_rn(ss, __fmul_rn(v[i].w, v[i].w));
    }
    ss = wave_sum(ss);
    const float mean = __fmul_rn(ss, __fdiv_rn(1.0f, (float)d));
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, eps)));
    float4 *o4 = reinterpret_cast<float4 *>(out + row * d);
    auto res = [&](int i) __attribute__((always_inline)) {
        float4 r;
        r.x = __fmul_rn(__fmul_rn(v[i].x, inv), wv[i].x);
        r.y = __fmul_rn(__fmul_rn(v[i].y, inv), wv[i].y);
        r.z = __fmul_rn(__fmul_rn(v[i].z, inv), wv[i].z);
        r.w = __fmul_rn(__fmul_rn(v[i].w, inv), wv[i].w);
        return r;
    };
    if (d4 == 64 * NV) {
        // rows that fill every lane's float4s: stores without guards, so no
        // store waits on the ones before it
#pragma unroll
        for (int i = 0; i < NV; ++i) o4[lane + 64 * i] = res(i);
    } else {
#pragma unroll
        for (int i = 0; i < NV; ++i)
            if (lane + 64 * i < d4) o4[lane + 64 * i] = res(i);
    }
}

// ---- add: ops_elementwise.rs:249-259 (same-shape path) -----------------------
__global__ __launch_bounds__(256) void add_kernel(const float *__restrict__ a,
                                                  const float *__restrict__ b,
                                                  float *__restrict__ out, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        out[i] = __fadd_rn(a[i], b[i]);
}

// ---- silu(g) * u: mlp.rs:21-23 ---------------------------------------------
__global__ __launch_bounds__(256) void silu_mul_kernel(const float *__restrict__ g,
                                                       const float *__restrict__ u,
                                                       float *__restrict__ out, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        out[i] = __fmul_rn(silu_f(g[i]), u[i]);
    }
}

// dg and du may be g and u themselves: each element is read before written.
__global__ __launch_bounds__(256) void silu_mul_backward_kernel(const float *__restrict__ dh,
                                                                const float *g, const float *u,
                                                                float *dg, float *du, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const float2 r = swiglu_bwd_f(dh[i], g[i], u[i]);
        dg[i] = r.x;
        du[i] = r.y;
    }
}

// ---- RoPE: rope.rs:28-32 (rotate-half) ---------------------------------------
__global__ __launch_bounds__(256) void rope_kernel(const float *__restrict__ x, int64_t bh,
                                                   int64_t t, int64_t hd,
                                                   const float *__restrict__ cos_t,
                                                   const float *__restrict__ sin_t,
                                                   float *__restrict__ out) {
    const int64_t half = hd / 2, total = bh * t * half;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = i / half, c = i - row * half;
        const int64_t pos = row % t;
        const float *xr = x + row * hd;
        const float x1 = xr[c], x2 = xr[c + half];
        const float cs = cos_t[pos * half + c], sn = sin_t[pos * half + c];
        out[row * hd + c] = __fsub_rn(__fmul_rn(x1, cs), __fmul_rn(x2, sn));
        out[row * hd + c + half] = __fadd_rn(__fmul_rn(x2, cs), __fmul_rn(x1, sn));
    }
}

// ---- cross-entropy: ops_reduce.rs:253-259 --------------------------------------
// One workgroup per row and one pass over the logits. Each thread loads chunks
// of 4 float4, takes the chunk max (fmaxf, which ignores NaN like f32::max),
// rescales its running sum of exp(z - max) once per chunk when the max grows,
// and adds the chunk's 16 exponentials; (max, sum) pairs then merge across the
// workgroup. The row term is formed as the reference forms it,
// (max + ln(sum)) - z[target], in f32.

__global__ __launch_bounds__(256) void ce_rows_kernel(const float *__restrict__ logits,
                                                      const int32_t *__restrict__ targets,
                                                      int64_t n, int64_t v,
                                                      float *__restrict__ row_loss, int vec) {
    constexpr int CH = 4;
    const int64_t row = blockIdx.x;
    const float *z = logits + row * v;
    const float4 *z4 = reinterpret_cast<const float4 *>(z);
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
    if (threadIdx.x == 0) {
        float M = sm[0], S = ss[0];
        for (int i = 1; i < 4; ++i) lse_merge(M, S, sm[i], ss[i]);
        const float lse = __fadd_rn(M, logf(S));
        row_loss[row] = __fsub_rn(lse, z[targets[row]]);
    }
}

// The row terms from the head GEMM's per-tile partials (EPI_CE): one wave per
// row; lane l merges tiles l, l + 64, ... in order, then the lanes merge in a
// fixed tree; the row term is (max + ln(sum)) - z[target] as in ce_rows_kernel.
__global__ __launch_bounds__(256) void ce_combine_kernel(const float *__restrict__ part,
                                                         int64_t tiles,
                                                         const float *__restrict__ zt,
                                                         int64_t n, float *__restrict__ row_loss) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;
    const float2 *pr = reinterpret_cast<const float2 *>(part) + row * tiles;
    float m = -INFINITY, s = 0.0f;
    for (int64_t j = lane; j < tiles; j += 64) {
        const float2 q = pr[j];
        lse_merge(m, s, q.x, q.y);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float m2 = __shfl_xor(m, off, 64), s2 = __shfl_xor(s, off, 64);
        lse_merge(m, s, m2, s2);
    }
    if (lane == 0) row_loss[row] = __fsub_rn(__fadd_rn(m, logf(s)), zt[row]);
}

// Mean of the row terms in f64 (ops_reduce.rs:258-259), fixed reduction order.
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

// ---- weight packing (the reference order <-> the model's device layout) -----
// A workgroup row of the grid (blockIdx.y, striding by gridDim.y) walks whole
// rows; its threads walk the row in float4s where the layout allows (vec),
// else in single floats. Bit-exact copies.
__global__ __launch_bounds__(256) void pack_cols_kernel(const float *__restrict__ src,
                                                        int64_t rows, int64_t cols,
                                                        float *__restrict__ dst, int64_t ld_dst,
                                                        int64_t col_off, int vec) {
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const float *s = src + r * cols;
        float *d = dst + r * ld_dst + col_off;
        if (vec) {
            for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < cols / 4; q += step)
                reinterpret_cast<float4 *>(d)[q] = reinterpret_cast<const float4 *>(s)[q];
        } else {
            for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < cols; c += step)
                d[c] = s[c];
        }
    }
}

// dst [rows, 2*ff_pad]: column 2f is gate column f and column 2f+1 is up
// column f; columns of f >= ff are zero. A thread moves 4 columns f of both.
__global__ __launch_bounds__(256) void pack_gate_up_kernel(const float *__restrict__ wg,
                                                           const float *__restrict__ wu,
                                                           int64_t rows, int64_t ff,
                                                           int64_t ff_pad,
                                                           float *__restrict__ dst, int vec) {
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const float *g = wg + r * ff, *u = wu + r * ff;
        float4 *d = reinterpret_cast<float4 *>(dst + r * 2 * ff_pad);
        for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < ff_pad / 4; q += step) {
            const int64_t f = 4 * q;
            float4 a, b;
            if (vec && f + 3 < ff) {
                a = reinterpret_cast<const float4 *>(g)[q];
                b = reinterpret_cast<const float4 *>(u)[q];
            } else {
                a.x = f + 0 < ff ? g[f + 0] : 0.0f;
                a.y = f + 1 < ff ? g[f + 1] : 0.0f;
                a.z = f + 2 < ff ? g[f + 2] : 0.0f;
                a.w = f + 3 < ff ? g[f + 3] : 0.0f;
                b.x = f + 0 < ff ? u[f + 0] : 0.0f;
                b.y = f + 1 < ff ? u[f + 1] : 0.0f;
                b.z = f + 2 < ff ? u[f + 2] : 0.0f;
                b.w = f + 3 < ff ? u[f + 3] : 0.0f;
            }
            d[2 * q] = make_float4(a.x, b.x, a.y, b.y);
            d[2 * q + 1] = make_float4(a.z, b.z, a.w, b.w);
        }
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

void launch_embedding(Context &ctx, const float *table, int64_t d, const int32_t *ids_dev,
                      int64_t n, float *out) {
    const int vec = (d % 4 == 0) && al16(table) && al16(out);
    const int64_t d4 = d / 4;
    auto rows = [&](auto kernel, int rpw) {
        hipLaunchKernelGGL(kernel, dim3((unsigned)((n + rpw - 1) / rpw)), dim3(256), 0, ctx.stream,
                           table, d, ids_dev, n, out);
    };
    if (vec && d4 == 512)  // the large preset's rows
        rows(embedding_rows_kernel<1, 2>, 1);
    else if (vec && d4 == 256)
        rows(embedding_rows_kernel<1, 1>, 1);
    else if (vec && d4 == 1024)
        rows(embedding_rows_kernel<1, 4>, 1);
    else if (vec && d4 == 128)
        rows(embedding_rows_kernel<2, 1>, 2);
    else if (vec && d4 == 64)
        rows(embedding_rows_kernel<4, 1>, 4);
    else if (vec && d4 == 32)
        rows(embedding_rows_kernel<8, 1>, 8);
    else
        hipLaunchKernelGGL(embedding_kernel, dim3(grid_for(vec ? n * d / 4 : n * d)), dim3(256), 0,
                           ctx.stream, table, d, ids_dev, n, out, vec);
    check_hip(hipGetLastError(), "embedding launch");
}

void launch_rms_norm(Context &ctx, const float *x, const float *w, int64_t rows, int64_t d,
                     float eps, float *out) {
    const int vec = (d % 4 == 0) && al16(x) && al16(w) && al16(out);
    if (vec && d <= 4096) {
        const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
        const int dd = (int)d;
        if (d <= 256)
            hipLaunchKernelGGL(rms_norm_rows_kernel<1>, grid, block, 0, ctx.stream, x, w, rows, dd, eps, out);
        else if (d <= 512)
            hipLaunchKernelGGL(rms_norm_rows_kernel<2>, grid, block, 0, ctx.stream, x, w, rows, dd, eps, out);
        else if (d <= 1024)
            hipLaunchKernelGGL(rms_norm_rows_kernel<4>, grid, block, 0, ctx.stream, x, w, rows, dd, eps, out);
        else if (d <= 2048)
            hipLaunchKernelGGL(rms_norm_rows_kernel<8>, grid, block, 0, ctx.stream, x, w, rows, dd, eps, out);
        else
            hipLaunchKernelGGL(rms_norm_rows_kernel<16>, grid, block, 0, ctx.stream, x, w, rows, dd, eps, out);
        check_hip(hipGetLastError(), "rms_norm launch");
        return;
    }
    hipLaunchKernelGGL(rms_norm_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                       ctx.stream, x, w, rows, d, eps, out, vec);
    check_hip(hipGetLastError(), "rms_norm launch");
}

void launch_add(Context &ctx, const float *a, const float *b, float *out, int64_t n) {
    hipLaunchKernelGGL(add_kernel, dim3(grid_for(n)), dim3(256), 0, ctx.stream, a, b, out, n);
    check_hip(hipGetLastError(), "add launch");
}

void launch_silu_mul(Context &ctx, const float *g, const float *u, float *out, int64_t n) {
    hipLaunchKernelGGL(silu_mul_kernel, dim3(grid_for(n)), dim3(256), 0, ctx.stream, g, u, out,
                       n);
    check_hip(hipGetLastError(), "silu_mul launch");
}

void launch_silu_mul_backward(Context &ctx, const float *dh, float *g, float *u, float *dg,
                              float *du, int64_t n) {
    hipLaunchKernelGGL(silu_mul_backward_kernel, dim3(grid_for(n)), dim3(256), 0, ctx.stream, dh,
                       g, u, dg, du, n);
    check_hip(hipGetLastError(), "silu_mul backward launch");
}

void launch_rope(Context &ctx, const float *x, int64_t bh, int64_t t, int64_t hd,
                 const float *cos_t, const float *sin_t, float *out) {
    hipLaunchKernelGGL(rope_kernel, dim3(grid_for(bh * t * (hd / 2))), dim3(256), 0, ctx.stream,
                       x, bh, t, hd, cos_t, sin_t, out);
    check_hip(hipGetLastError(), "rope launch");
}

void launch_cross_entropy(Context &ctx, const float *logits, const int32_t *targets_dev,
                          int64_t n, int64_t v, float *row_loss, float *loss_dev) {
    if (n > 0x7fffffff) fail(MMH_ERR_SHAPE, "cross_entropy: too many rows");
    const int vec = (v % 4 == 0) && al16(logits);
    hipLaunchKernelGGL(ce_rows_kernel, dim3((unsigned)n), dim3(256), 0, ctx.stream, logits,
                       targets_dev, n, v, row_loss, vec);
    check_hip(hipGetLastError(), "cross_entropy launch");
    hipLaunchKernelGGL(mean_f64_kernel, dim3(1), dim3(256), 0, ctx.stream, row_loss, n,
                       loss_dev);
    check_hip(hipGetLastError(), "loss mean launch");
}

void launch_ce_combine(Context &ctx, const float *part, int64_t tiles, const float *zt,
                       int64_t n, float *row_loss, float *loss_dev) {
    if (n > 0x1ffffffff) fail(MMH_ERR_SHAPE, "cross_entropy: too many rows");
    hipLaunchKernelGGL(ce_combine_kernel, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, ctx.stream,
                       part, tiles, zt, n, row_loss);
    check_hip(hipGetLastError(), "loss combine launch");
    hipLaunchKernelGGL(mean_f64_kernel, dim3(1), dim3(256), 0, ctx.stream, row_loss, n,
                       loss_dev);
    check_hip(hipGetLastError(), "loss mean launch");
}

// Grid of the row-walking copy kernels: enough threads for a row's units in
// x, rows (at most 65535 at a time) in y.
dim3 rows_grid(int64_t rows, int64_t units) {
    const int64_t x = std::max<int64_t>(1, std::min<int64_t>((units + 255) / 256, 64));
    return dim3((unsigned)x, (unsigned)std::max<int64_t>(1, std::min<int64_t>(rows, 65535)));
}

void launch_pack_cols(Context &ctx, const float *src, int64_t rows, int64_t cols, float *dst,
                      int64_t ld_dst, int64_t col_off) {
    const int vec = cols % 4 == 0 && ld_dst % 4 == 0 && col_off % 4 == 0 && al16(src) && al16(dst);
    hipLaunchKernelGGL(pack_cols_kernel, rows_grid(rows, vec ? cols / 4 : cols), dim3(256), 0,
                       ctx.stream, src, rows, cols, dst, ld_dst, col_off, vec);
    check_hip(hipGetLastError(), "pack launch");
}

void launch_pack_gate_up(Context &ctx, const float *wg, const float *wu, int64_t rows,
                         int64_t ff, int64_t ff_pad, float *dst) {
    if (ff_pad % 4 || !al16(dst)) fail(MMH_ERR_ARGUMENT, "pack: padded rows must be float4s");
    const int vec = ff % 4 == 0 && al16(wg) && al16(wu);
    hipLaunchKernelGGL(pack_gate_up_kernel, rows_grid(rows, ff_pad / 4), dim3(256), 0, ctx.stream,
                       wg, wu, rows, ff, ff_pad, dst, vec);
    check_hip(hipGetLastError(), "pack launch");
}

}  // namespace mmh
