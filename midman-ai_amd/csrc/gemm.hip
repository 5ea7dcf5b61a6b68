// fp32 GEMM on CDNA4 matrix cores (v_mfma_f32_32x32x2_f32), LDS-staged tiles.
//
// Replaces the reference's three CPU kernels (midman-tensor/src/kernels.rs:49-108,
// kernels_avx.rs:45-250): C = A.B (nn), A.B^T (nt) and A^T.B (tn). The
// transposed forms never materialize a transpose (the reference copies B^T,
// kernels.rs:68-73): the operand is read in its stored layout and written into
// LDS k-major, which is the layout the MFMA operand reads want.
//
// Tiling: a 256-thread workgroup (4 wave64s, 2x2) owns a 128x128 tile of C;
// each wave owns 64x64 = 2x2 MFMA 32x32 blocks (64 accumulators per lane).
// K advances 16 at a time through a double-buffered LDS stage: the next tile's
// global loads are issued before the current tile's 32 MFMAs per wave and
// written to the other LDS buffer after them, with one barrier per step.
//
// MFMA 32x32x2 f32 operand layout (wave64): lane l supplies A[i=l%32][k=l/32]
// and B[k=l/32][j=l%32]; accumulator register r of lane l holds
// D[i = 8*(r/4) + 4*(l/32) + r%4][j = l%32].
//
// Workgroup -> tile mapping is XCD-aware: the dispatcher hands workgroup w to
// XCD w % 8, so w is renumbered to make each XCD's share a contiguous run of
// tiles, and tiles are walked in groups of 8 tile-rows so that the tiles an
// XCD holds at once share A rows and B columns in its L2.
//
// Small-tile-count shapes (e.g. M=2048, N=256) are split along K; each split
// writes a partial tile and a second kernel sums the partials in split order,
// so the result is deterministic.
#include "mmh_internal.h"

namespace mmh {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 16;
constexpr int GROUP_M = 8;

struct KParams {
    const float *a;
    const float *b;
    float *c;
    float *partial;
    int64_t m, n, k;
    int64_t lda, ldb, ldc;
    int64_t stride_a, stride_b, stride_c;
    int64_t k_per_split;
    int64_t swiglu_ff;
    int tiles_m, tiles_n;
    int splits;
    int vec_a, vec_b;
};

__device__ __forceinline__ float silu_f(float x) {
    // ops_elementwise.rs:239-241, :355-364: x * (1 / (1 + e^-x))
    const float s = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-x)));
    return __fmul_rn(x, s);
}

// Row strides of the LDS stages, chosen so the transposing scalar stores
// spread over the banks and the float4 stores stay 16-byte aligned.
template <bool TA>
struct LdsA {
    static constexpr int S = BM + (TA ? 4 : 2);
};
template <bool TB>
struct LdsB {
    static constexpr int S = BN + (TB ? 2 : 4);
};

// The K loop of one 128x128 tile. FAST: the whole tile lies inside M, N and
// the K range is a multiple of BK with 16-byte aligned rows, so no load needs
// a predicate; otherwise every element is bounds-checked and zero-filled.
template <bool TA, bool TB, bool FAST>
__device__ __forceinline__ void gemm_mainloop(const KParams &p, const float *__restrict__ A,
                                              const float *__restrict__ B, int64_t m0, int64_t n0,
                                              int64_t kbeg, int64_t kend,
                                              float (*As)[BK][LdsA<TA>::S],
                                              float (*Bs)[BK][LdsB<TB>::S],
                                              floatx16 (&acc)[2][2]) {
    const int tid = threadIdx.x;
    const int64_t M = p.m, N = p.n;
    // One K-tile is 2 float4 of A and 2 float4 of B per thread, held in
    // named registers (an indexed array here ends up in scratch memory).
    float4 ra0, ra1, rb0, rb1;

    auto load_a = [&](int idx, int64_t k0) -> float4 {
        if (FAST) {
            if (!TA)
                return *reinterpret_cast<const float4 *>(A + (m0 + (idx >> 2)) * p.lda + k0 + (idx & 3) * 4);
            return *reinterpret_cast<const float4 *>(A + (k0 + (idx >> 5)) * p.lda + m0 + (idx & 31) * 4);
        }
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (!TA) {
            const int64_t gm = m0 + (idx >> 2), gk = k0 + (idx & 3) * 4;
            if (gm < M) {
                const float *src = A + gm * p.lda + gk;
                if (gk + 0 < kend) v.x = src[0];
                if (gk + 1 < kend) v.y = src[1];
                if (gk + 2 < kend) v.z = src[2];
                if (gk + 3 < kend) v.w = src[3];
            }
        } else {
            const int64_t gk = k0 + (idx >> 5), gm = m0 + (idx & 31) * 4;
            if (gk < kend) {
                const float *src = A + gk * p.lda + gm;
                if (gm + 0 < M) v.x = src[0];
                if (gm + 1 < M) v.y = src[1];
                if (gm + 2 < M) v.z = src[2];
                if (gm + 3 < M) v.w = src[3];
            }
        }
        return v;
    };
    auto load_b = [&](int idx, int64_t k0) -> float4 {
        if (FAST) {
            if (!TB)
                return *reinterpret_cast<const float4 *>(B + (k0 + (idx >> 5)) * p.ldb + n0 + (idx & 31) * 4);
            return *reinterpret_cast<const float4 *>(B + (n0 + (idx >> 2)) * p.ldb + k0 + (idx & 3) * 4);
        }
        float4 w = make_float4(0.f, 0.f, 0.f, 0.f);
        if (!TB) {
            const int64_t gk = k0 + (idx >> 5), gn = n0 + (idx & 31) * 4;
            if (gk < kend) {
                const float *src = B + gk * p.ldb + gn;
                if (gn + 0 < N) w.x = src[0];
                if (gn + 1 < N) w.y = src[1];
                if (gn + 2 < N) w.z = src[2];
                if (gn + 3 < N) w.w = src[3];
            }
        } else {
            const int64_t gn = n0 + (idx >> 2), gk = k0 + (idx & 3) * 4;
            if (gn < N) {
                const float *src = B + gn * p.ldb + gk;
                if (gk + 0 < kend) w.x = src[0];
                if (gk + 1 < kend) w.y = src[1];
                if (gk + 2 < kend) w.z = src[2];
                if (gk + 3 < kend) w.w = src[3];
            }
        }
        return w;
    };
    auto load = [&](int64_t k0) {
        ra0 = load_a(tid, k0);
        ra1 = load_a(tid + 256, k0);
        rb0 = load_b(tid, k0);
        rb1 = load_b(tid + 256, k0);
    };
    auto store_a = [&](int buf, int idx, const float4 &v) {
        if (!TA) {
            const int row = idx >> 2, kq = (idx & 3) * 4;
            As[buf][kq + 0][row] = v.x;
            As[buf][kq + 1][row] = v.y;
            As[buf][kq + 2][row] = v.z;
            As[buf][kq + 3][row] = v.w;
        } else {
            *reinterpret_cast<float4 *>(&As[buf][idx >> 5][(idx & 31) * 4]) = v;
        }
    };
    auto store_b = [&](int buf, int idx, const float4 &v) {
        if (!TB) {
            *reinterpret_cast<float4 *>(&Bs[buf][idx >> 5][(idx & 31) * 4]) = v;
        } else {
            const int col = idx >> 2, kq = (idx & 3) * 4;
            Bs[buf][kq + 0][col] = v.x;
            Bs[buf][kq + 1][col] = v.y;
            Bs[buf][kq + 2][col] = v.z;
            Bs[buf][kq + 3][col] = v.w;
        }
    };
    auto store = [&](int buf) {
        store_a(buf, tid, ra0);
        store_a(buf, tid + 256, ra1);
        store_b(buf, tid, rb0);
        store_b(buf, tid + 256, rb1);
    };

    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, lk = lane >> 5;

    // MFMA operands of one K-tile, read from LDS a tile ahead of their use.
    float a0[BK / 2][2], b0[BK / 2][2], a1[BK / 2][2], b1[BK / 2][2];
    auto lread = [&](int buf, float (&a)[BK / 2][2], float (&b)[BK / 2][2]) {
#pragma unroll
        for (int kk = 0; kk < BK / 2; ++kk) {
            a[kk][0] = As[buf][2 * kk + lk][wm * 64 + lr];
            a[kk][1] = As[buf][2 * kk + lk][wm * 64 + 32 + lr];
            b[kk][0] = Bs[buf][2 * kk + lk][wn * 64 + lr];
            b[kk][1] = Bs[buf][2 * kk + lk][wn * 64 + 32 + lr];
        }
    };
    auto mfma_tile = [&](float (&a)[BK / 2][2], float (&b)[BK / 2][2]) {
#pragma unroll
        for (int kk = 0; kk < BK / 2; ++kk) {
            acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[kk][0], b[kk][0], acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[kk][0], b[kk][1], acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[kk][1], b[kk][0], acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[kk][1], b[kk][1], acc[1][1], 0, 0, 0);
        }
    };

    // Pipeline: while the MFMAs of tile t run from registers, the operands of
    // tile t+1 come out of LDS and the global loads of tile t+2 are in flight;
    // tile t+2 then goes into the LDS stage tile t used. One barrier per tile.
    const int64_t nk = (kend - kbeg + BK - 1) / BK;
    if (nk > 0) {
        load(kbeg);
        store(0);
    }
    __syncthreads();
    if (nk > 0) lread(0, a0, b0);
    if (nk > 1) {
        load(kbeg + BK);
        store(1);
    }
    __syncthreads();
    auto step = [&](int64_t it, float (&ca)[BK / 2][2], float (&cb)[BK / 2][2],
                    float (&na)[BK / 2][2], float (&nb)[BK / 2][2]) {
        if (it + 2 < nk) load(kbeg + (it + 2) * BK);
        if (it + 1 < nk) lread((int)((it + 1) & 1), na, nb);
        mfma_tile(ca, cb);
        if (it + 2 < nk) store((int)(it & 1));
        __syncthreads();
    };
    for (int64_t it = 0; it < nk; it += 2) {
        step(it, a0, b0, a1, b1);
        if (it + 1 < nk) step(it + 1, a1, b1, a0, b0);
    }
}

template <bool TA, bool TB, int EPI>
__global__ __launch_bounds__(256, 2) void gemm_f32_mfma(KParams p) {
    __shared__ float As[2][BK][LdsA<TA>::S];
    __shared__ float Bs[2][BK][LdsB<TB>::S];

    const int tid = threadIdx.x;

    // XCD-aware renumbering, then grouped tile order.
    int bid = blockIdx.x;
    {
        const int nb = gridDim.x, q = nb >> 3, r = nb & 7;
        const int xcd = bid & 7, local = bid >> 3;
        bid = xcd * q + (xcd < r ? xcd : r) + local;
    }
    const int per_group = GROUP_M * p.tiles_n;
    const int group = bid / per_group;
    const int first_m = group * GROUP_M;
    const int gsize = min(p.tiles_m - first_m, GROUP_M);
    const int in_group = bid - group * per_group;
    const int tm = first_m + in_group % gsize;
    const int tn = in_group / gsize;
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

    const int64_t batch = blockIdx.y;
    const int split = blockIdx.z;
    const float *__restrict__ A = p.a + batch * p.stride_a;
    const float *__restrict__ B = p.b + batch * p.stride_b;
    const int64_t kbeg = (int64_t)split * p.k_per_split;
    const int64_t kend = min(p.k, kbeg + p.k_per_split);
    const int64_t M = p.m, N = p.n;

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const bool fast = p.vec_a && p.vec_b && m0 + BM <= M && n0 + BN <= N &&
                      (kend - kbeg) % BK == 0;
    if (fast)
        gemm_mainloop<TA, TB, true>(p, A, B, m0, n0, kbeg, kend, As, Bs, acc);
    else
        gemm_mainloop<TA, TB, false>(p, A, B, m0, n0, kbeg, kend, As, Bs, acc);

    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, lk = lane >> 5;

    // ---- epilogue ----
    if (p.splits > 1) {
        float *P = p.partial + (int64_t)split * M * N;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int64_t row = m0 + wm * 64 + i * 32 + (r >> 2) * 8 + lk * 4 + (r & 3);
                    const int64_t col = n0 + wn * 64 + j * 32 + lr;
                    if (row < M && col < N) P[row * N + col] = acc[i][j][r];
                }
        return;
    }
    float *C = p.c + batch * p.stride_c;
    if (EPI == EPI_SWIGLU) {
        // Packed columns: each 64-column group g holds 32 gate columns then the
        // 32 matching up columns, so a wave's j=0 block is gate and j=1 is up.
        const int64_t g = (n0 + wn * 64) >> 6;
        const int64_t col = g * 32 + lr;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = m0 + wm * 64 + i * 32 + (r >> 2) * 8 + lk * 4 + (r & 3);
                if (row < M && col < p.swiglu_ff)
                    C[row * p.ldc + col] = __fmul_rn(silu_f(acc[i][0][r]), acc[i][1][r]);
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = m0 + wm * 64 + i * 32 + (r >> 2) * 8 + lk * 4 + (r & 3);
                const int64_t col = n0 + wn * 64 + j * 32 + lr;
                if (row < M && col < N) {
                    float *dst = C + row * p.ldc + col;
                    if (EPI == EPI_ACCUM)
                        *dst = __fadd_rn(*dst, acc[i][j][r]);
                    else
                        *dst = acc[i][j][r];
                }
            }
}

// Sums split partials in split order, then applies the epilogue.
template <int EPI>
__global__ __launch_bounds__(256) void splitk_reduce(const float *__restrict__ partial,
                                                     float *__restrict__ c, int64_t m,
                                                     int64_t n, int64_t ldc, int splits) {
    const int64_t total = m * n;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        float acc = partial[idx];
        for (int s = 1; s < splits; ++s) acc = __fadd_rn(acc, partial[(int64_t)s * total + idx]);
        const int64_t row = idx / n, col = idx - row * n;
        float *dst = c + row * ldc + col;
        if (EPI == EPI_ACCUM)
            *dst = __fadd_rn(*dst, acc);
        else
            *dst = acc;
    }
}

template <bool TA, bool TB, int EPI>
void launch(Context &ctx, const KParams &p, dim3 grid) {
    hipLaunchKernelGGL((gemm_f32_mfma<TA, TB, EPI>), grid, dim3(256), 0, ctx.stream, p);
}

template <int EPI>
void dispatch_t(Context &ctx, bool ta, bool tb, const KParams &p, dim3 grid) {
    if (!ta && !tb) launch<false, false, EPI>(ctx, p, grid);
    else if (!ta && tb) launch<false, true, EPI>(ctx, p, grid);
    else if (ta && !tb) launch<true, false, EPI>(ctx, p, grid);
    else launch<true, true, EPI>(ctx, p, grid);
}

bool aligned16(const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

}  // namespace

void gemm(Context &ctx, const GemmDesc &d) {
    if (d.m <= 0 || d.n <= 0 || d.k <= 0 || d.batch <= 0) fail(MMH_ERR_SHAPE, "gemm: empty shape");
    KParams p{};
    p.a = d.a;
    p.b = d.b;
    p.c = d.c;
    p.m = d.m;
    p.n = d.n;
    p.k = d.k;
    p.lda = d.lda;
    p.ldb = d.ldb;
    p.ldc = d.ldc;
    p.stride_a = d.stride_a;
    p.stride_b = d.stride_b;
    p.stride_c = d.stride_c;
    p.swiglu_ff = d.swiglu_ff;
    p.tiles_m = (int)((d.m + BM - 1) / BM);
    p.tiles_n = (int)((d.n + BN - 1) / BN);
    p.vec_a = (d.lda % 4 == 0) && (d.batch == 1 || d.stride_a % 4 == 0) && aligned16(d.a);
    p.vec_b = (d.ldb % 4 == 0) && (d.batch == 1 || d.stride_b % 4 == 0) && aligned16(d.b);

    const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
    const int64_t ktiles = (d.k + BK - 1) / BK;
    int splits = 1;
    if (d.force_splits > 0) {
        splits = d.force_splits;
    } else if (d.batch == 1 && d.epi != EPI_SWIGLU) {
        // Fill the chip: at least two tiles per CU, at least 8 K-steps per split.
        const int64_t target = 2 * (int64_t)(ctx.cu_count > 0 ? ctx.cu_count : 256);
        while (tiles * splits < target && splits < 16 && ktiles / (splits * 2) >= 8) splits *= 2;
    }
    if (d.batch > 1 || d.epi == EPI_SWIGLU) splits = 1;
    const int64_t kt_per = (ktiles + splits - 1) / splits;
    p.k_per_split = kt_per * BK;
    splits = (int)((ktiles + kt_per - 1) / kt_per);
    p.splits = splits;
    if (splits > 1) p.partial = static_cast<float *>(ctx.get_scratch((size_t)splits * d.m * d.n * 4));

    if (tiles > 0x7fffffff || d.batch > 65535) fail(MMH_ERR_SHAPE, "gemm: grid too large");
    dim3 grid((unsigned)tiles, (unsigned)d.batch, (unsigned)splits);
    const int epi = splits > 1 ? EPI_STORE : d.epi;
    if (epi == EPI_SWIGLU) {
        if (d.ta || d.tb) fail(MMH_ERR_ARGUMENT, "gemm: swiglu epilogue needs the nn form");
        launch<false, false, EPI_SWIGLU>(ctx, p, grid);
    } else if (epi == EPI_ACCUM) {
        dispatch_t<EPI_ACCUM>(ctx, d.ta, d.tb, p, grid);
    } else {
        dispatch_t<EPI_STORE>(ctx, d.ta, d.tb, p, grid);
    }
    check_hip(hipGetLastError(), "gemm launch");
    if (splits > 1) {
        const int64_t total = d.m * d.n;
        const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 8192);
        if (d.epi == EPI_ACCUM)
            hipLaunchKernelGGL(splitk_reduce<EPI_ACCUM>, dim3(blocks), dim3(256), 0, ctx.stream,
                               p.partial, d.c, d.m, d.n, d.ldc, splits);
        else
            hipLaunchKernelGGL(splitk_reduce<EPI_STORE>, dim3(blocks), dim3(256), 0, ctx.stream,
                               p.partial, d.c, d.m, d.n, d.ldc, splits);
        check_hip(hipGetLastError(), "split-k reduce launch");
    }
}

}  // namespace mmh
