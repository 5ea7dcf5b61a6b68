// fp32 GEMM on CDNA4 matrix cores (v_mfma_f32_32x32x2_f32), LDS-staged tiles.
//
// Replaces the reference's three CPU kernels (midman-tensor/src/kernels.rs:49-108,
// kernels_avx.rs:45-250): C = A.B (nn), A.B^T (nt) and A^T.B (tn). The
// transposed forms never materialize a transpose (the reference copies B^T,
// kernels.rs:68-73): each operand is read in its stored layout and written into
// LDS k-major, the layout the MFMA operand reads want.
//
// Tiling: a 512-thread workgroup (8 wave64s, 4 along M x 2 along N) owns a
// 128x128 tile of C; each wave owns 32 rows x 64 columns as two MFMA 32x32
// blocks (32 accumulators per lane), whose columns are the even and the odd
// columns of its 64: one 4-byte A read and one 8-byte B read from LDS give a
// lane its operands for both blocks, and the epilogue writes column pairs.
// Eight small waves rather than four of 64x64 keep four waves on every SIMD
// when a grid has only two tiles per CU (the O and down projections of the
// large preset: 512 tiles), at under 110 registers. For the QKV product with
// RoPE in the epilogue the column blocks instead hold columns c and c + hd/2
// of a head (hd 64 or 128), so each rotation pair sits in one lane.
//
// MFMA 32x32x2 f32 operand layout (wave64): lane l supplies A[i=l%32][k=l/32]
// and B[k=l/32][j=l%32]; accumulator register r of lane l holds
// D[i = 8*(r/4) + 4*(l/32) + r%4][j = l%32].
//
// K advances 16 at a time through two LDS stages, software-pipelined: at the
// top of iteration t, tile t+1 moves from registers into the free stage and
// tile t+4's global loads are issued into the register slot it freed (a ring
// of three slots); then the 16 MFMAs per wave of tile t run while the loads
// of three tiles are in flight. One barrier per tile. Interior tiles take a
// path with no load predicates and 32-bit offsets from uniform base
// pointers; edge tiles zero-fill outside [M, N, K) and keep one slot.
//
// Workgroup -> tile mapping is XCD-aware: the dispatcher hands workgroup w to
// XCD w % 8, so w is renumbered to make each XCD's share a contiguous run of
// tiles, and tiles are walked in groups of 8 tile-rows so that the tiles an
// XCD holds at once share A rows and B columns in its L2.
//
// Small-tile-count shapes (e.g. M=2048, N=256) are split along K; the
// partials are summed in split order, so the result is deterministic: on the
// 64x64 and 32x32 tiles by the last split of each tile (the splits store
// their partial through to memory and count themselves in a per-tile
// counter), on the 128x128 tiles by a second kernel.
#include "mmh_internal.h"

#include <utility>

namespace mmh {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 16;
constexpr int NT = 512;  // threads of the 128x128 kernel: 8 waves
constexpr int GROUP_M = 8;
// Register slots of the 128x128 kernel's load ring on interior tiles: tile
// t+KSLOTS's global loads are issued while tile t's MFMAs run. Edge tiles
// (predicated loads, few per grid) keep one slot, which holds the kernel's
// registers to what the interior path needs.
constexpr int KSLOTS = 3;
// Raw buffer descriptor: byte range (interior tiles stay below 2^31 bytes from
// their base, checked on the host) and the gfx9-family dword-3 flags.
constexpr int kBufferRange = 0x7fffffff;
constexpr int kBufferFlags = 0x00020000;

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
    const float *resid;
    float *aux;
    int64_t ldaux;
    int tiles_m, tiles_n;
    int splits;
    int vec_a, vec_b, vec_c;
    // small kernel only: A-row RMSNorm in the loads, RoPE in the epilogue
    const float *norm_w;
    float norm_eps;
    const float *rope_cos, *rope_sin;
    int rope_seq, rope_hd, rope_cols;
    // EPI_CE (128x128 kernel): targets in, per-tile (max, sum) pairs and target logits out
    const int32_t *ce_targets;
    float *ce_part, *ce_zt;
    // Tail balance (128x128 kernel, one matrix): workgroups from tail_first on
    // each take one of tail_s K-pieces (tail_k long) of tiles tail_first.. in
    // the grouped order, and write their partial tile to partial (tile-local
    // [BM][BN] blocks, piece-major); tail_reduce sums them in piece order.
    int tail_first, tail_s;
    int64_t tail_k;
    // Split K on the 64x64 and 32x32 tiles (tickets set): every split stores
    // its partial tile through to memory and counts itself in tickets[tile];
    // the last split of a tile sums the tile's partials in split order and
    // applies the epilogue (split_accum: C = resid (or C) + sum, else C = sum).
    int32_t *tickets;
    int split_accum;
    // The value the sums of products start from: +0 (a product, as the
    // reference's fresh zeroed C), or -0 when the sum is added into C (the
    // seam's accumulate: C's own value starts the reference's sum, so a -0 in
    // C with all products -0 must stay -0; -0 is the identity of IEEE addition)
    float acc_init;
};

// Row strides (floats) of the k-major LDS stages: even, so the 8-byte operand
// reads stay aligned; +2 where the stores transpose (spreads consecutive k rows
// over the banks), +4 where they are float4 (keeps 16-byte alignment).
template <bool TA>
struct LdsA {
    static constexpr int S = BM + (TA ? 4 : 2);
};
template <bool TB>
struct LdsB {
    static constexpr int S = BN + (TB ? 2 : 4);
};

// Calls f(integral_constant<int, i>) for i = 0..n-1, so that i is a
// compile-time constant in each call (register-slot indices stay static).
template <class F, int... Is>
__device__ __forceinline__ void unroll_seq(F &&f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}

// Reductions over each 32-lane half of a wave with DPP moves (quad permutes,
// then rotations within a 16-lane row) and one v_permlane16_swap across the
// two rows of the half (a VALU exchange: no trip through the LDS unit). For the max every lane ends with the result; for the sum the
// lanes associate the terms differently, and lane 0 of the half (the one read)
// always the same way.
__device__ __forceinline__ float dpp_f(float v, int ctrl) {
    switch (ctrl) {
        case 0xB1: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
        case 0x4E: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
        case 0x124: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x124, 0xF, 0xF, false));
        default: return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false));
    }
}
// The pair {v[l], v[l ^ 16]} in each lane l (in some order).
__device__ __forceinline__ auto pair16_f(float v) {
    return __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
}
__device__ __forceinline__ float half_max32(float v) {
    v = fmaxf(v, dpp_f(v, 0xB1));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f(v, 0x4E));   // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_f(v, 0x124));  // row_ror:4
    v = fmaxf(v, dpp_f(v, 0x128));  // row_ror:8
    const auto q = pair16_f(v);
    return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
__device__ __forceinline__ float half_sum32(float v) {
    v += dpp_f(v, 0xB1);
    v += dpp_f(v, 0x4E);
    v += dpp_f(v, 0x124);
    v += dpp_f(v, 0x128);
    const auto q = pair16_f(v);
    return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// The K loop of one 128x128 tile; see the file comment.
// CL: the columns of a wave's two MFMA column blocks: 0 the even and odd
// columns of its 64 (one 8-byte operand read), 1 its two halves of 32, 2
// columns c and c + 64 of the tile (wave wn takes c = 32*wn .. +31), so the
// RoPE pair (c, c + hd/2) of a head of 64 (CL 1) or 128 (CL 2) columns sits
// in one lane.
template <bool TA, bool TB, bool FAST, int SLOTS, int CL, bool OPQ = false>
__device__ __forceinline__ void gemm_mainloop(const KParams &p, const float *__restrict__ A,
                                              const float *__restrict__ B, int64_t m0, int64_t n0,
                                              int64_t kbeg, int64_t kend,
                                              float (*As)[BK][LdsA<TA>::S],
                                              float (*Bs)[BK][LdsB<TB>::S],
                                              floatx16 (&acc)[2]) {
    // OPQ: the thread index through an empty asm. The register assignment
    // and schedule the compiler then picks ran the residual-epilogue forms
    // 0.8-1.4% faster on the large forward's o and down products, and the
    // SwiGLU and loss forms 2% slower, so only the former take it.
    int tid = threadIdx.x;
    if constexpr (OPQ) asm volatile("" : "+v"(tid));
    const int64_t M = p.m, N = p.n;
    // A K-tile of each operand is 128 x BK floats = 32*BK float4; thread tid
    // moves float4 idx = tid + NT*i, i < NL.
    // Row-major-in-k operands (A for nn/nt, B for nt): row idx/(BK/4), k (idx%(BK/4))*4.
    // k-major operands (A for tn, B for nn/tn): k idx/32, column (idx%32)*4.
    constexpr int NL = 32 * BK / NT;
    static_assert(NL >= 1 && 32 * BK % NT == 0, "a K-tile must split evenly over the threads");
    constexpr int RQ = BK / 4;  // float4 per row of a row-major-in-k tile
    // Uniform bases (moved by the tile's k) and loop-invariant 32-bit byte
    // offsets per thread, so each load is one SGPR base + VGPR offset
    // instruction with no per-iteration address registers.
    const float *a_base = TA ? A + m0 : A + m0 * p.lda;
    const float *b_base = TB ? B + n0 * p.ldb : B + n0;
    const uint32_t lda = (uint32_t)p.lda, ldb = (uint32_t)p.ldb;
    uint32_t ao[NL], bo[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const int idx = tid + NT * i;
        ao[i] = 4u * (TA ? (uint32_t)(idx >> 5) * lda + (idx & 31) * 4
                         : (uint32_t)(idx / RQ) * lda + (idx % RQ) * 4);
        bo[i] = 4u * (TB ? (uint32_t)(idx / RQ) * ldb + (idx % RQ) * 4
                         : (uint32_t)(idx >> 5) * ldb + (idx & 31) * 4);
    }

    constexpr int NS = FAST ? SLOTS : 1;
    float4 ra[NS][NL], rb[NS][NL];

    // Values outside [M, N, K) read as zeros; A's are -0, so a product of two
    // of them is -0, the identity of IEEE addition (a +0 would turn an exact
    // -0 sum into +0).
    auto load_a_edge = [&](int idx, int64_t k0) __attribute__((always_inline)) -> float4 {
        float4 v = make_float4(-0.f, -0.f, -0.f, -0.f);
        if (!TA) {
            const int64_t gm = m0 + idx / RQ, gk = k0 + (idx % RQ) * 4;
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
    auto load_b_edge = [&](int idx, int64_t k0) __attribute__((always_inline)) -> float4 {
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
            const int64_t gn = n0 + idx / RQ, gk = k0 + (idx % RQ) * 4;
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
    auto load = [&](int sl, int64_t k0) __attribute__((always_inline)) {
        if (FAST) {
            // Buffer loads: the tile's base in a scalar descriptor, the
            // per-thread byte offset in one loop-invariant VGPR.
            const float *ak = TA ? a_base + k0 * p.lda : a_base + k0;
            const float *bk = TB ? b_base + k0 : b_base + k0 * p.ldb;
            const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float *>(ak), (short)0, kBufferRange, kBufferFlags);
            const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float *>(bk), (short)0, kBufferRange, kBufferFlags);
#pragma unroll
            for (int i = 0; i < NL; ++i)
                ra[sl][i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rsa, ao[i], 0, 0));
#pragma unroll
            for (int i = 0; i < NL; ++i)
                rb[sl][i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rsb, bo[i], 0, 0));
        } else {
#pragma unroll
            for (int i = 0; i < NL; ++i) ra[sl][i] = load_a_edge(tid + NT * i, k0);
#pragma unroll
            for (int i = 0; i < NL; ++i) rb[sl][i] = load_b_edge(tid + NT * i, k0);
        }
    };
    auto store = [&](int sl, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int idx = tid + NT * i;
            if (!TA) {
                const int row = idx / RQ, kq = (idx % RQ) * 4;
                As[buf][kq + 0][row] = ra[sl][i].x;
                As[buf][kq + 1][row] = ra[sl][i].y;
                As[buf][kq + 2][row] = ra[sl][i].z;
                As[buf][kq + 3][row] = ra[sl][i].w;
            } else {
                float *dst = &As[buf][idx >> 5][(idx & 31) * 4];
                dst[0] = ra[sl][i].x;
                dst[1] = ra[sl][i].y;
                dst[2] = ra[sl][i].z;
                dst[3] = ra[sl][i].w;
            }
            if (!TB) {
                float *dst = &Bs[buf][idx >> 5][(idx & 31) * 4];
                dst[0] = rb[sl][i].x;
                dst[1] = rb[sl][i].y;
                dst[2] = rb[sl][i].z;
                dst[3] = rb[sl][i].w;
            } else {
                const int col = idx / RQ, kq = (idx % RQ) * 4;
                Bs[buf][kq + 0][col] = rb[sl][i].x;
                Bs[buf][kq + 1][col] = rb[sl][i].y;
                Bs[buf][kq + 2][col] = rb[sl][i].z;
                Bs[buf][kq + 3][col] = rb[sl][i].w;
            }
        }
    };

    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, lk = lane >> 5;

    // One tile's MFMAs from LDS stage `buf`: all operand reads are issued
    // first (for each k-pair kk the A value of the lane's row and the B
    // values of its two column blocks); the MFMAs consume them in order as
    // they land.
    constexpr int cstep = CL == 0 ? 1 : CL == 1 ? 32 : 64;  // block 1's column offset
    const int cbase = CL == 0 ? wn * 64 + 2 * lr : CL == 1 ? wn * 64 + lr : wn * 32 + lr;
    auto compute = [&](int buf) __attribute__((always_inline)) {
        const float *pa = &As[buf][lk][wm * 32 + lr];
        const float *pb = &Bs[buf][lk][cbase];
        float a[BK / 2];
        float2 b[BK / 2];
#pragma unroll
        for (int kk = 0; kk < BK / 2; ++kk) {
            a[kk] = pa[2 * kk * LdsA<TA>::S];
            if constexpr (CL == 0)
                b[kk] = *reinterpret_cast<const float2 *>(pb + 2 * kk * LdsB<TB>::S);
            else
                b[kk] = make_float2(pb[2 * kk * LdsB<TB>::S], pb[2 * kk * LdsB<TB>::S + cstep]);
        }
#pragma unroll
        for (int kk = 0; kk < BK / 2; ++kk) {
            acc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[kk], b[kk].x, acc[0], 0, 0, 0);
            acc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[kk], b[kk].y, acc[1], 0, 0, 0);
        }
    };

    // Pipeline: when iteration t starts, LDS stage t%2 holds tile t and
    // register slot (t+j)%NS holds tile t+j for j = 1..NS (loads in flight;
    // NS = SLOTS on interior tiles, 1 on edge tiles). Tile t+1 goes into the other stage
    // (last read in iteration t-1, before its barrier), tile t+1+NS's global
    // loads are issued into the slot that freed, and then the MFMAs of tile t
    // run: a load has NS tiles of MFMAs to land, which covers HBM latency
    // when the operands are in no cache (a layer's weights). One barrier per
    // iteration. The loop is unrolled by the period of (stage, slot) so every
    // slot index is a constant, and every step issues its loads
    // unconditionally (tiles past the end reload the last one, which nothing
    // reads): with the same loads on every path the compiler waits for
    // exactly the oldest slot instead of draining all of them.
    const int nk = (int)((kend - kbeg + BK - 1) / BK);
    if (nk <= 0) return;
    constexpr int U = NS % 2 == 0 ? NS : 2 * NS;
    auto tile_k = [&](int t) __attribute__((always_inline)) {
        return kbeg + (int64_t)min(t, nk - 1) * BK;
    };
    auto step = [&](auto uc, int it) __attribute__((always_inline)) {
        constexpr int u = decltype(uc)::value;
        store((u + 1) % NS, (u + 1) % 2);
        load((u + 1) % NS, tile_k(it + 1 + NS));
        compute(u % 2);
        __syncthreads();
    };
    load(0, kbeg);
    store(0, 0);
    unroll_seq([&](auto jc) __attribute__((always_inline)) {
        constexpr int j = decltype(jc)::value + 1;
        load(j % NS, tile_k(j));
    }, std::make_integer_sequence<int, NS>{});
    __syncthreads();
    int base = 0;
    for (; base + U <= nk; base += U)
        unroll_seq([&](auto uc) __attribute__((always_inline)) { step(uc, base + uc); },
                   std::make_integer_sequence<int, U>{});
    unroll_seq([&](auto uc) __attribute__((always_inline)) {
        if (base + uc < nk) step(uc, base + uc);
    }, std::make_integer_sequence<int, U>{});
}

// Tile t of the grouped order: GROUP_M tile rows at a time, column by column.
// Split partials for the in-kernel reduction: stored through to memory and
// read past the XCD-local L2 (device-scope relaxed atomics: sc1 stores and
// loads), so the last split of a tile, on any XCD, reads every split's values.
__device__ __forceinline__ void split_put(float *dst, float v) {
    __hip_atomic_store(dst, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float split_get(const float *src) {
    return __hip_atomic_load(const_cast<float *>(src), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// After a workgroup's split_put stores: true in the workgroup that completes
// the tile (the last of its p.splits splits to get here), which also resets
// the tile's counter for the next launch. Every thread of the workgroup calls it.
__device__ __forceinline__ bool split_last(const KParams &p, int tile) {
    __shared__ int s_last;
    __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores are complete
    __syncthreads();
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(p.tickets + tile, 1, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
        s_last = old == p.splits - 1;
        if (s_last) __hip_atomic_store(p.tickets + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    return s_last;
}
// The last split of a tile: rows [m0, m0 + tr) x columns [n0, n0 + tc) of C
// (tc a multiple of 4) as the splits' partials added in split order (the
// caller's own included, read back like the others), then the epilogue
// (split_accum: C = resid (or C) + sum). The nthreads threads walk the tile
// row-major, four columns at a time, with four splits' loads in flight;
// partial rows of N % 4 == 0 move as float4, others one value at a time.
__device__ __forceinline__ void split_reduce_tile(const KParams &p, int64_t m0, int64_t n0, int tr,
                                               int tc, int nthreads) {
    const int64_t M = p.m, N = p.n, total = M * N;
    const bool vecp = N % 4 == 0;
    const bool vecc = p.ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(p.c) & 15) == 0 &&
                      (!p.resid || (reinterpret_cast<uintptr_t>(p.resid) & 15) == 0);
    const float *R = p.resid ? p.resid : p.c;
    const int iters = tr * tc / (4 * nthreads);
    if (m0 + tr <= M && n0 + tc <= N && vecp && vecc && iters <= 4 &&
        iters * 4 * nthreads == tr * tc) {
        // The whole tile in range: every element's reads (the residual, then
        // the partials) before the first store, so no read waits for a store.
        float4 res[4];
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            if (it >= iters) break;
            const int e = 4 * (int)threadIdx.x + it * 4 * nthreads;
            const int64_t row = m0 + e / tc, col = n0 + e % tc;
            const float4 o = p.split_accum ? *reinterpret_cast<const float4 *>(R + row * p.ldc + col)
                                           : make_float4(0.f, 0.f, 0.f, 0.f);
            const float *Q = p.partial + row * N + col;
            float4 acc;
            for (int s0 = 0; s0 < p.splits; s0 += 4) {
                float4 v[4];
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (s0 + u < p.splits) {
                        const float *src = Q + (int64_t)(s0 + u) * total;
                        v[u].x = split_get(src);
                        v[u].y = split_get(src + 1);
                        v[u].z = split_get(src + 2);
                        v[u].w = split_get(src + 3);
                    }
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (s0 + u < p.splits) {
                        if (s0 + u == 0) {
                            acc = v[u];
                        } else {
                            acc.x = __fadd_rn(acc.x, v[u].x);
                            acc.y = __fadd_rn(acc.y, v[u].y);
                            acc.z = __fadd_rn(acc.z, v[u].z);
                            acc.w = __fadd_rn(acc.w, v[u].w);
                        }
                    }
            }
            res[it] = p.split_accum ? make_float4(__fadd_rn(o.x, acc.x), __fadd_rn(o.y, acc.y),
                                                  __fadd_rn(o.z, acc.z), __fadd_rn(o.w, acc.w))
                                    : acc;
        }
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            if (it >= iters) break;
            const int e = 4 * (int)threadIdx.x + it * 4 * nthreads;
            *reinterpret_cast<float4 *>(p.c + (m0 + e / tc) * p.ldc + n0 + e % tc) = res[it];
        }
        return;
    }
    for (int e = 4 * (int)threadIdx.x; e < tr * tc; e += 4 * nthreads) {
        const int64_t row = m0 + e / tc, col = n0 + e % tc;
        if (row >= M || col >= N) continue;
        const float *Q = p.partial + row * N + col;
        if (vecp && col + 3 < N) {
            float4 acc;
            for (int s0 = 0; s0 < p.splits; s0 += 4) {
                float4 v[4];
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (s0 + u < p.splits) {
                        const float *src = Q + (int64_t)(s0 + u) * total;
                        v[u].x = split_get(src);
                        v[u].y = split_get(src + 1);
                        v[u].z = split_get(src + 2);
                        v[u].w = split_get(src + 3);
                    }
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (s0 + u < p.splits) {
                        if (s0 + u == 0) {
                            acc = v[u];
                        } else {
                            acc.x = __fadd_rn(acc.x, v[u].x);
                            acc.y = __fadd_rn(acc.y, v[u].y);
                            acc.z = __fadd_rn(acc.z, v[u].z);
                            acc.w = __fadd_rn(acc.w, v[u].w);
                        }
                    }
            }
            float *dst = p.c + row * p.ldc + col;
            if (p.split_accum) {
                const float *r = R + row * p.ldc + col;
                if (vecc) {
                    const float4 o = *reinterpret_cast<const float4 *>(r);
                    acc = make_float4(__fadd_rn(o.x, acc.x), __fadd_rn(o.y, acc.y),
                                      __fadd_rn(o.z, acc.z), __fadd_rn(o.w, acc.w));
                } else {
                    acc = make_float4(__fadd_rn(r[0], acc.x), __fadd_rn(r[1], acc.y),
                                      __fadd_rn(r[2], acc.z), __fadd_rn(r[3], acc.w));
                }
            }
            if (vecc) {
                *reinterpret_cast<float4 *>(dst) = acc;
            } else {
                dst[0] = acc.x;
                dst[1] = acc.y;
                dst[2] = acc.z;
                dst[3] = acc.w;
            }
            continue;
        }
        for (int u = 0; u < 4 && col + u < N; ++u) {
            float v = split_get(Q + u);
            for (int s = 1; s < p.splits; ++s) v = __fadd_rn(v, split_get(Q + (int64_t)s * total + u));
            float *dst = p.c + row * p.ldc + col + u;
            *dst = p.split_accum ? __fadd_rn(R[row * p.ldc + col + u], v) : v;
        }
    }
}

__device__ __forceinline__ void grouped_tile(const KParams &p, int t, int &tm, int &tn) {
    const int per_group = GROUP_M * p.tiles_n;
    const int group = t / per_group;
    const int first_m = group * GROUP_M;
    const int gsize = min(p.tiles_m - first_m, GROUP_M);
    const int in_group = t - group * per_group;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}

template <bool TA, bool TB, int EPI, int CL = 0>
__global__ __launch_bounds__(NT, 2) void gemm_f32_mfma(KParams p) {
    static_assert(CL == 0 || EPI == EPI_STORE, "the RoPE column layouts store plain values");
    __shared__ __attribute__((aligned(16))) float As[2][BK][LdsA<TA>::S];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK][LdsB<TB>::S];

    const int tid = threadIdx.x;

    // XCD-aware renumbering of the whole tiles, then grouped tile order; the
    // tail pieces (if any) follow the whole tiles.
    int bid = blockIdx.x;
    int piece = -1;
    int64_t kbeg = (int64_t)blockIdx.z * p.k_per_split;
    int64_t kend = min(p.k, kbeg + p.k_per_split);
    if (p.tail_s > 1 && bid >= p.tail_first) {
        piece = bid - p.tail_first;
        bid = p.tail_first + piece / p.tail_s;
        kbeg = (int64_t)(piece % p.tail_s) * p.tail_k;
        kend = min(p.k, kbeg + p.tail_k);
    } else {
        const int nb = p.tail_s > 1 ? p.tail_first : (int)gridDim.x, q = nb >> 3, r = nb & 7;
        const int xcd = bid & 7, local = bid >> 3;
        bid = xcd * q + (xcd < r ? xcd : r) + local;
    }
    int tm, tn;
    grouped_tile(p, bid, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

    const int64_t batch = blockIdx.y;
    const int split = blockIdx.z;
    const float *__restrict__ A = p.a + batch * p.stride_a;
    const float *__restrict__ B = p.b + batch * p.stride_b;
    const int64_t M = p.m, N = p.n;

    floatx16 acc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] = p.acc_init;
    // EPI_CE: the tile's target ids go to LDS before the K loop (whose
    // barriers order them before the epilogue reads them)
    __shared__ int ce_t[EPI == EPI_CE ? BM : 1];
    if (EPI == EPI_CE && tid < BM) ce_t[tid] = m0 + tid < M ? p.ce_targets[m0 + tid] : -1;
    const bool fast = p.vec_a && p.vec_b && m0 + BM <= M && n0 + BN <= N &&
                      (kend - kbeg) % BK == 0;
    if (fast)
        gemm_mainloop<TA, TB, true, KSLOTS, CL, EPI == EPI_ACCUM>(p, A, B, m0, n0, kbeg, kend, As, Bs, acc);
    else
        gemm_mainloop<TA, TB, false, 1, CL>(p, A, B, m0, n0, kbeg, kend, As, Bs, acc);

    // ---- epilogue: block j register r of lane l is C[row][col] with
    // row = m0 + 32*wm + 8*(r/4) + 4*(l/32) + r%4 and, for CL 0,
    // col = n0 + 64*wn + 2*(l%32) + j (the other layouts below).
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, lk = lane >> 5;
    const int64_t col = n0 + wn * 64 + 2 * lr;
    auto row_local = [&](int r) __attribute__((always_inline)) {
        return wm * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
    };
    if (piece >= 0) {  // a tail piece: its partial tile, whole (edges included)
        float *P = p.partial + (int64_t)piece * (BM * BN) + wn * 64 + 2 * lr;
#pragma unroll
        for (int r = 0; r < 16; ++r)
            *reinterpret_cast<float2 *>(P + row_local(r) * BN) = make_float2(acc[0][r], acc[1][r]);
        return;
    }
    if constexpr (CL != 0) {
        // Column block j of lane lr is column c0 + j*half of C (half = 32 for
        // CL 1, 64 for CL 2), c0 the lane's column in the first half of its
        // head: RoPE (rope.rs:28-32) rotates the pair in registers, with the
        // rope kernel's arithmetic, on the q and k heads (columns below
        // rope_cols); the v heads are stored as they are.
        constexpr int half = CL == 1 ? 32 : 64;
        const int hc = CL == 1 ? lr : wn * 32 + lr;
        const int64_t c0 = CL == 1 ? n0 + wn * 64 + lr : n0 + wn * 32 + lr;
        const bool rot = p.rope_cos != nullptr && c0 < p.rope_cols;
        float *C = p.c + batch * p.stride_c;
        // The rows' table values are all read before the first store: the
        // compiler cannot tell the tables from C, so a read placed after a
        // store waits for that store's completion (one memory round trip per
        // row). Rows past M read a valid table row (row % seq) and are dropped.
        // Positions: the lane's first row modulo the sequence once; register
        // r adds 8*(r/4) + r%4 < 28 to it, at most one wrap when seq >= 28.
        float cs[16], sn[16];
        if (rot) {
            const uint32_t seq = (uint32_t)p.rope_seq;
            const uint32_t base = (uint32_t)((m0 + row_local(0)) % p.rope_seq);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                uint32_t pos = base + (uint32_t)(8 * (r >> 2) + (r & 3));
                if (seq < 28) pos %= seq;
                else if (pos >= seq) pos -= seq;
                const uint32_t t = pos * (uint32_t)half + (uint32_t)hc;
                cs[r] = p.rope_cos[t];
                sn[r] = p.rope_sin[t];
            }
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t row = m0 + row_local(r);
            if (row >= M) continue;
            float x1 = acc[0][r], x2 = acc[1][r];
            if (rot) {
                const float y1 = x1 * cs[r] - x2 * sn[r];
                const float y2 = x2 * cs[r] + x1 * sn[r];
                x1 = y1;
                x2 = y2;
            }
            if (c0 < N) C[row * p.ldc + c0] = x1;
            if (c0 + half < N) C[row * p.ldc + c0 + half] = x2;
        }
        return;
    }
    if (p.splits > 1) {
        // (summed by splitk_reduce: a tile's 2-16 partials are too much for
        // one workgroup of the launch to add up at the end)
        float *P = p.partial + (int64_t)split * M * N;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t row = m0 + row_local(r);
            if (row < M) {
                if (col < N) P[row * N + col] = acc[0][r];
                if (col + 1 < N) P[row * N + col + 1] = acc[1][r];
            }
        }
        return;
    }
    if constexpr (EPI == EPI_CE) {
        // Cross-entropy partials of this tile's columns (ops_reduce.rs:236-259
        // split by column tiles): per row, the max of the logits and the sum of
        // exp(z - max) over the lane's two columns, over the 32 lanes of its
        // half by DPP moves, then over the two waves sharing the rows through
        // LDS. The lane holding a row's target column keeps its logit.
        __shared__ float ce_m[2][BM], ce_s[2][BM];
        constexpr float kLog2e = 1.4426950408889634f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int rl = row_local(r);
            const int64_t row = m0 + rl;
            const float v0 = acc[0][r], v1 = acc[1][r];
            const float x0 = col < N ? v0 : -INFINITY, x1 = col + 1 < N ? v1 : -INFINITY;
            const float mx = half_max32(fmaxf(x0, x1));
            // exp(z - max) through the hardware's exp2 (no flush concern: the
            // terms that matter are within a few hundred of 1)
            const float e = half_sum32(
                mx == -INFINITY ? 0.0f
                                : __builtin_amdgcn_exp2f((x0 - mx) * kLog2e) +
                                      __builtin_amdgcn_exp2f((x1 - mx) * kLog2e));
            if (lr == 0) {
                ce_m[wn][rl] = mx;
                ce_s[wn][rl] = e;
            }
            const int t = ce_t[rl];
            if (t == col) p.ce_zt[row] = v0;
            if (t == col + 1) p.ce_zt[row] = v1;
        }
        __syncthreads();
        if (tid < BM && m0 + tid < M) {
            float m = ce_m[0][tid], sum = ce_s[0][tid];
            lse_merge(m, sum, ce_m[1][tid], ce_s[1][tid]);
            reinterpret_cast<float2 *>(p.ce_part)[(m0 + tid) * p.tiles_n + tn] =
                make_float2(m, sum);
        }
        return;
    }
    float *C = p.c + batch * p.stride_c;
    if (EPI == EPI_SWIGLU) {
        // Packed columns interleave gate and up: column 2f is gate f, 2f+1 up f.
        const int64_t f = col >> 1;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t row = m0 + row_local(r);
            if (row >= M) continue;
            if (p.aux && col + 1 < N)
                *reinterpret_cast<float2 *>(p.aux + row * p.ldaux + col) =
                    make_float2(acc[0][r], acc[1][r]);
            if (f < p.swiglu_ff) C[row * p.ldc + f] = __fmul_rn(silu_fast(acc[0][r]), acc[1][r]);
        }
        return;
    }
    // The epilogues that read memory (the saved gate/up pairs, the residual)
    // issue their reads ahead of their stores, 8 or 16 rows at a time: the
    // destination may be the buffer read (in-place gradients, C += ...), so
    // the compiler may not move a read past a store and would otherwise wait
    // out one memory latency per row. Each lane reads only the elements it
    // writes, so the early reads see the same values.
    if (EPI == EPI_SWIGLU_BWD) {
        // acc is dh[row][col, col+1]; their (g, u) pairs sit at aux columns
        // 2*col .. 2*col+3 and the (dg, du) pairs go to the same columns of C.
        if (m0 + BM <= M && n0 + BN <= N && p.ldc < (int64_t(1) << 20) &&
            p.ldaux < (int64_t(1) << 20)) {
            // The whole tile in range: unconditional buffer accesses from the
            // tile's first row (see the residual epilogue below), eight rows'
            // pairs read before their eight stores.
            const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float *>(p.aux + m0 * p.ldaux), (short)0, kBufferRange, kBufferFlags);
            const __amdgpu_buffer_rsrc_t rc =
                __builtin_amdgcn_make_buffer_rsrc(C + m0 * p.ldc, (short)0, kBufferRange, kBufferFlags);
            const uint32_t la = 4u * (uint32_t)p.ldaux, lc = 4u * (uint32_t)p.ldc;
            const uint32_t va = (uint32_t)row_local(0) * la + 8u * (uint32_t)col;
            const uint32_t vc = (uint32_t)row_local(0) * lc + 8u * (uint32_t)col;
#pragma unroll
            for (int r0 = 0; r0 < 16; r0 += 8) {
                float4 g[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int r = r0 + j;
                    g[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                          ra, va + (8 * (r >> 2) + (r & 3)) * la, 0, 0));
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int r = r0 + j;
                    const float2 a = swiglu_bwd_f(acc[0][r], g[j].x, g[j].y);
                    const float2 b2 = swiglu_bwd_f(acc[1][r], g[j].z, g[j].w);
                    __builtin_amdgcn_raw_buffer_store_b128(
                        __builtin_bit_cast(u32x4_t, make_float4(a.x, a.y, b2.x, b2.y)), rc,
                        vc + (8 * (r >> 2) + (r & 3)) * lc, 0, 0);
                }
            }
            return;
        }
#pragma unroll
        for (int r0 = 0; r0 < 16; r0 += 8) {
            float4 g[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int64_t row = m0 + row_local(r0 + j);
                g[j] = row < M && col + 1 < N
                           ? *reinterpret_cast<const float4 *>(p.aux + row * p.ldaux + 2 * col)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int r = r0 + j;
                const int64_t row = m0 + row_local(r);
                if (row >= M) continue;
                float *dst = C + row * p.ldc + 2 * col;
                if (col + 1 < N) {
                    const float2 a = swiglu_bwd_f(acc[0][r], g[j].x, g[j].y);
                    const float2 b2 = swiglu_bwd_f(acc[1][r], g[j].z, g[j].w);
                    *reinterpret_cast<float4 *>(dst) = make_float4(a.x, a.y, b2.x, b2.y);
                } else if (col < N) {
                    const float *gu = p.aux + row * p.ldaux + 2 * col;
                    const float2 a = swiglu_bwd_f(acc[0][r], gu[0], gu[1]);
                    dst[0] = a.x;
                    dst[1] = a.y;
                }
            }
        }
        return;
    }
    const float *R = p.resid ? p.resid + batch * p.stride_c : C;
    const bool pair = p.vec_c && col + 1 < N;
    if (EPI == EPI_ACCUM && pair) {
        float2 o[16];
        if (m0 + BM <= M && p.ldc < (int64_t(1) << 21)) {
            // Every row in range: no per-row branches, so the compiler counts
            // the reads exactly and each store waits only for its own read
            // (with the reads and stores under row tests, every store waited
            // for all earlier stores as well: one store round trip per row).
            // Buffer accesses from the tile's first row with 32-bit offsets
            // (64-bit addresses for 16 rows took the kernel past the registers
            // of four waves per SIMD). Each row's offset is added into the
            // lane offset, never passed as the scalar offset: with computed
            // scalar offsets the compiler reused an SGPR that a v_div_scale
            // had just written as its carry-out, and one row of a tile read
            // another row's values (found by the tail-pieces training test).
            const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float *>(R + m0 * p.ldc), (short)0, kBufferRange, kBufferFlags);
            const __amdgpu_buffer_rsrc_t rc =
                __builtin_amdgcn_make_buffer_rsrc(C + m0 * p.ldc, (short)0, kBufferRange, kBufferFlags);
            const uint32_t ldb4 = 4u * (uint32_t)p.ldc;
            const uint32_t vo = (uint32_t)row_local(0) * ldb4 + 4u * (uint32_t)col;
#pragma unroll
            for (int r = 0; r < 16; ++r)
                o[r] = __builtin_bit_cast(
                    float2, __builtin_amdgcn_raw_buffer_load_b64(rr, vo + (8 * (r >> 2) + (r & 3)) * ldb4, 0, 0));
#pragma unroll
            for (int r = 0; r < 16; ++r)
                __builtin_amdgcn_raw_buffer_store_b64(
                    __builtin_bit_cast(u32x2_t, make_float2(__fadd_rn(o[r].x, acc[0][r]),
                                                            __fadd_rn(o[r].y, acc[1][r]))),
                    rc, vo + (8 * (r >> 2) + (r & 3)) * ldb4, 0, 0);
            return;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t row = m0 + row_local(r);
            o[r] = row < M ? *reinterpret_cast<const float2 *>(R + row * p.ldc + col)
                           : make_float2(0.f, 0.f);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t row = m0 + row_local(r);
            if (row >= M) continue;
            *reinterpret_cast<float2 *>(C + row * p.ldc + col) =
                make_float2(__fadd_rn(o[r].x, acc[0][r]), __fadd_rn(o[r].y, acc[1][r]));
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + row_local(r);
        if (row >= M) continue;
        float *dst = C + row * p.ldc + col;
        const float *src = R + row * p.ldc + col;
        float v0 = acc[0][r], v1 = acc[1][r];
        if (pair) {
            if (EPI == EPI_ACCUM) {
                const float2 o = *reinterpret_cast<const float2 *>(src);
                v0 = __fadd_rn(o.x, v0);
                v1 = __fadd_rn(o.y, v1);
            }
            *reinterpret_cast<float2 *>(dst) = make_float2(v0, v1);
        } else {
            if (col < N) dst[0] = EPI == EPI_ACCUM ? __fadd_rn(src[0], v0) : v0;
            if (col + 1 < N) dst[1] = EPI == EPI_ACCUM ? __fadd_rn(src[1], v1) : v1;
        }
    }
}

// ---- small-tile GEMM ---------------------------------------------------------
// For shapes with fewer 128x128 tiles than CUs (the tiny preset's projections,
// M = 2048 with N and K of a few hundred) the big tile leaves most of the chip
// idle and every workgroup walks the whole K alone. Here a 256-thread
// workgroup owns a 64x64 tile, each wave one 32x32 MFMA block (16
// accumulators), K advancing 32 at a time, so the grid holds 4x the
// workgroups. With so few steps per tile, latency rules: three steps of global
// loads are kept in flight (a ring of register slots) ahead of the two LDS
// stages, and each lane reads its operands of a step as four 16-byte LDS
// reads. The epilogues match the big kernel's; in the SwiGLU epilogue the gate
// and up columns of a pair sit in neighbouring lanes and meet through one lane
// exchange.
constexpr int SBM = 64, SBN = 64, SBK = 32;
// LDS rows hold one output row (A) or column (B) with its 32 k values
// contiguous, padded to 36 floats: a lane reads its 16 k values of a step as
// four 16-byte reads, and eight consecutive rows fall in distinct 16-byte bank
// groups. An operand stored k-major in memory (A when TA, B when !TB) reaches
// LDS as single values at (row, k), 16 rows 4 apart per 16 lanes: its rows
// keep their eight float4 groups of k in the order g ^ ((row >> 3) & 7), so
// those stores spread over the banks (2 lanes per bank instead of 8) while the
// float4 reads stay aligned and conflict-free.
constexpr int SKS = SBK + 4;
__device__ __forceinline__ int sk_swz(int row) { return (row >> 3) & 7; }

// The K loop of one 64x64 tile. MFMA kk of a step takes k = kk from lanes
// 0-31 and k = 16 + kk from lanes 32-63 (any split of the step's k values
// between the two lane halves gives the same sum; A and B agree on it).
// FAST: every step is a full interior step (no predicates anywhere, so the
// compiler can count the loads in flight exactly).
template <bool TA, bool TB, bool FAST, bool NORM>
__device__ __forceinline__ void small_mainloop(const KParams &p, const float *__restrict__ A,
                                               const float *__restrict__ B, int64_t m0,
                                               int64_t n0, int64_t kbeg, int nk, int64_t kend,
                                               float (*As)[SBM][SKS], float (*Bs)[SBN][SKS],
                                               floatx16 &acc, float (&ss)[2]) {
    const int tid = threadIdx.x;
    const int64_t M = p.m, N = p.n;
    // A tile of each operand is 64 x 32 floats = 512 float4: thread tid moves
    // float4 idx = tid + 256*i, i < 2. Operands stored row-major in k (A for
    // nn/nt, B for nt): row idx/8, k (idx%8)*4. Operands stored k-major: k
    // idx/16, row (idx%16)*4.
    constexpr int PF = 3;  // k-steps of loads in flight
    float4 ra[PF][2], rb[PF][2], rw[PF];  // rw: the norm weights of A's k values
    auto load = [&](int64_t k0, int slot) __attribute__((always_inline)) {
        if (NORM) {
            // both of a thread's A float4 cover k = k0 + (tid%8)*4 .. +3
            const int64_t gk = k0 + (tid & 7) * 4;
            const float *wk = p.norm_w + gk;
            float4 w4 = make_float4(0.f, 0.f, 0.f, 0.f);
            if (FAST) {
                w4 = *reinterpret_cast<const float4 *>(wk);
            } else {
                if (gk + 0 < kend) w4.x = wk[0];
                if (gk + 1 < kend) w4.y = wk[1];
                if (gk + 2 < kend) w4.z = wk[2];
                if (gk + 3 < kend) w4.w = wk[3];
            }
            rw[slot] = w4;
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 256 * i;
            // padding: A -0, B +0, so a padded product is -0 (see load_a_edge)
            float4 v = make_float4(-0.f, -0.f, -0.f, -0.f), w = make_float4(0.f, 0.f, 0.f, 0.f);
            if (!TA) {
                const int64_t gm = m0 + (idx >> 3), gk = k0 + (idx & 7) * 4;
                const float *src = A + gm * p.lda + gk;
                if (FAST) {
                    v = *reinterpret_cast<const float4 *>(src);
                } else if (gm < M) {
                    if (gk + 0 < kend) v.x = src[0];
                    if (gk + 1 < kend) v.y = src[1];
                    if (gk + 2 < kend) v.z = src[2];
                    if (gk + 3 < kend) v.w = src[3];
                }
            } else {
                const int64_t gk = k0 + (idx >> 4), gm = m0 + (idx & 15) * 4;
                const float *src = A + gk * p.lda + gm;
                if (FAST) {
                    v = *reinterpret_cast<const float4 *>(src);
                } else if (gk < kend) {
                    if (gm + 0 < M) v.x = src[0];
                    if (gm + 1 < M) v.y = src[1];
                    if (gm + 2 < M) v.z = src[2];
                    if (gm + 3 < M) v.w = src[3];
                }
            }
            if (!TB) {
                const int64_t gk = k0 + (idx >> 4), gn = n0 + (idx & 15) * 4;
                const float *src = B + gk * p.ldb + gn;
                if (FAST) {
                    w = *reinterpret_cast<const float4 *>(src);
                } else if (gk < kend) {
                    if (gn + 0 < N) w.x = src[0];
                    if (gn + 1 < N) w.y = src[1];
                    if (gn + 2 < N) w.z = src[2];
                    if (gn + 3 < N) w.w = src[3];
                }
            } else {
                const int64_t gn = n0 + (idx >> 3), gk = k0 + (idx & 7) * 4;
                const float *src = B + gn * p.ldb + gk;
                if (FAST) {
                    w = *reinterpret_cast<const float4 *>(src);
                } else if (gn < N) {
                    if (gk + 0 < kend) w.x = src[0];
                    if (gk + 1 < kend) w.y = src[1];
                    if (gk + 2 < kend) w.z = src[2];
                    if (gk + 3 < kend) w.w = src[3];
                }
            }
            ra[slot][i] = v;
            rb[slot][i] = w;
        }
    };
    // real: the slot holds a k-step not yet summed (the ring's last stores
    // repeat the final step into the idle stage; those must not count)
    auto store = [&](int buf, int slot, bool real) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 256 * i;
            float4 va = ra[slot][i];
            const float4 vb = rb[slot][i];
            if (NORM) {
                // the row's sum of squares as its values pass, and x * w; the
                // row's 1/rms scales the products in the epilogue
                const float4 w4 = rw[slot];
                float t = __fadd_rn(ss[i], __fmul_rn(va.x, va.x));
                t = __fadd_rn(t, __fmul_rn(va.y, va.y));
                t = __fadd_rn(t, __fmul_rn(va.z, va.z));
                t = __fadd_rn(t, __fmul_rn(va.w, va.w));
                ss[i] = real ? t : ss[i];
                va.x = __fmul_rn(va.x, w4.x);
                va.y = __fmul_rn(va.y, w4.y);
                va.z = __fmul_rn(va.z, w4.z);
                va.w = __fmul_rn(va.w, w4.w);
            }
            if (!TA) {
                *reinterpret_cast<float4 *>(&As[buf][idx >> 3][(idx & 7) * 4]) = va;
            } else {
                const int k = idx >> 4, row = (idx & 15) * 4;
                As[buf][row + 0][k ^ (4 * sk_swz(row + 0))] = va.x;
                As[buf][row + 1][k ^ (4 * sk_swz(row + 1))] = va.y;
                As[buf][row + 2][k ^ (4 * sk_swz(row + 2))] = va.z;
                As[buf][row + 3][k ^ (4 * sk_swz(row + 3))] = va.w;
            }
            if (!TB) {
                const int k = idx >> 4, col = (idx & 15) * 4;
                Bs[buf][col + 0][k ^ (4 * sk_swz(col + 0))] = vb.x;
                Bs[buf][col + 1][k ^ (4 * sk_swz(col + 1))] = vb.y;
                Bs[buf][col + 2][k ^ (4 * sk_swz(col + 2))] = vb.z;
                Bs[buf][col + 3][k ^ (4 * sk_swz(col + 3))] = vb.w;
            } else {
                *reinterpret_cast<float4 *>(&Bs[buf][idx >> 3][(idx & 7) * 4]) = vb;
            }
        }
    };

    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, lk = lane >> 5;
    const int ga = TA ? sk_swz(wm * 32 + lr) : 0, gb = TB ? 0 : sk_swz(wn * 32 + lr);
    auto compute = [&](int buf) __attribute__((always_inline)) {
        const float4 *pa = reinterpret_cast<const float4 *>(&As[buf][wm * 32 + lr][0]);
        const float4 *pb = reinterpret_cast<const float4 *>(&Bs[buf][wn * 32 + lr][0]);
        float4 a[4], b[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            a[q] = pa[(4 * lk + q) ^ ga];
            b[q] = pb[(4 * lk + q) ^ gb];
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[q].x, b[q].x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[q].y, b[q].y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[q].z, b[q].z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[q].w, b[q].w, acc, 0, 0, 0);
        }
    };

    // Steps that do not fill a group of PF run first, one at a time. Then,
    // per group, sub-iteration j (global step t) stores step t+1 from slot
    // (j+1)%PF into the LDS stage not in use, loads step t+PF into slot j
    // (whose step t went to LDS one sub-iteration earlier), runs the MFMAs of
    // step t and ends with the one barrier. Slot indices are constants of the
    // unrolled group and every load is issued unconditionally (past the last
    // step they re-read it, from cache), so the wait before each store counts
    // exactly the PF-2 younger steps and lets them stay in flight.
    auto step_k = [&](int t) __attribute__((always_inline)) {
        return kbeg + (int64_t)min(t, nk - 1) * SBK;
    };
    int t = 0;
    for (; t < nk % PF; ++t) {
        load(step_k(t), 0);
        store(0, 0, true);
        __syncthreads();
        compute(0);
        __syncthreads();
    }
    if (t == nk) return;
#pragma unroll
    for (int j = 0; j < PF; ++j) load(step_k(t + j), j);
    store(0, 0, true);
    __syncthreads();
    for (int g = 0; t < nk; ++g, t += PF) {
#pragma unroll
        for (int j = 0; j < PF; ++j) {
            const int cur = (g * PF + j) & 1;
            store(cur ^ 1, (j + 1) % PF, t + j + 1 < nk);
            load(step_k(t + j + PF), j);
            compute(cur);
            __syncthreads();
        }
    }
}

// One accumulator value v of C[row][col] of a 32-column MFMA block (lane lr
// holds column col) through the epilogues of the small kernels. Every lane of
// the wave calls it: the SwiGLU gate/up pair and the RoPE pair meet through
// lane exchanges. SwiGLU: gate f at column 2f (even lane), up f at 2f+1 (the
// next lane). RoPE (rope.rs:28-32) on heads of rope_hd (<= 32, dividing 32)
// columns: the pair (c, c + hd/2) of a head sits in lanes lr and lr ^ hd/2.
template <int EPI>
__device__ __forceinline__ void block32_epilogue(const KParams &p, float *C, const float *R,
                                                 int64_t row, int64_t col, int lr, float v) {
    if (EPI == EPI_SWIGLU) {
        const float up = __shfl_xor(v, 1, 64);
        if ((lr & 1) || row >= p.m) return;
        const int64_t f = col >> 1;
        if (p.aux && col + 1 < p.n)
            *reinterpret_cast<float2 *>(p.aux + row * p.ldaux + col) = make_float2(v, up);
        if (f < p.swiglu_ff) C[row * p.ldc + f] = __fmul_rn(silu_f(v), up);
        return;
    }
    if (EPI == EPI_STORE && p.rope_cos) {
        const int hd = p.rope_hd, half = hd >> 1;
        const float other = __shfl_xor(v, half, 64);
        if (row >= p.m || col >= p.n) return;
        if (col < p.rope_cols) {
            const int pc = (int)(col % hd);
            const int64_t pos = row % p.rope_seq;
            const int c = pc < half ? pc : pc - half;
            const float cs = p.rope_cos[pos * half + c], sn = p.rope_sin[pos * half + c];
            v = pc < half ? v * cs - other * sn : v * cs + other * sn;
        }
        C[row * p.ldc + col] = v;
        return;
    }
    if (row >= p.m || col >= p.n) return;
    C[row * p.ldc + col] = EPI == EPI_ACCUM ? __fadd_rn(R[row * p.ldc + col], v) : v;
}

template <bool TA, bool TB, int EPI, bool NORM>
__global__ __launch_bounds__(256) void gemm_f32_mfma_small(KParams p) {
    __shared__ __attribute__((aligned(16))) float As[2][SBM][SKS];
    __shared__ __attribute__((aligned(16))) float Bs[2][SBN][SKS];
    __shared__ float sm_inv[SBM];  // NORM: 1/rms of the tile's rows

    const int tid = threadIdx.x;
    const int bid = blockIdx.x;
    const int tm = bid / p.tiles_n, tn = bid - (bid / p.tiles_n) * p.tiles_n;
    const int64_t m0 = (int64_t)tm * SBM, n0 = (int64_t)tn * SBN;
    const int64_t batch = blockIdx.y;
    const int split = blockIdx.z;
    const float *__restrict__ A = p.a + batch * p.stride_a;
    const float *__restrict__ B = p.b + batch * p.stride_b;
    const int64_t kbeg = (int64_t)split * p.k_per_split;
    const int64_t kend = min(p.k, kbeg + p.k_per_split);
    const int64_t M = p.m, N = p.n;

    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = p.acc_init;
    // NORM: sums of squares of this thread's two A rows (the loads give
    // thread tid rows tid/8 and 32 + tid/8 at every K-step), gathered as the
    // values pass through the LDS stores.
    float ss[2] = {0.0f, 0.0f};
    const int nk = (int)((kend - kbeg + SBK - 1) / SBK);
    if (p.vec_a && p.vec_b && m0 + SBM <= M && n0 + SBN <= N) {
        // interior: the full steps branch-free, then a K tail (if any) on the
        // predicated path, after the last barrier of the full steps
        const int nfull = (int)((kend - kbeg) / SBK);
        small_mainloop<TA, TB, true, NORM>(p, A, B, m0, n0, kbeg, nfull, kend, As, Bs, acc,
                                           ss);
        if (nfull < nk)
            small_mainloop<TA, TB, false, NORM>(p, A, B, m0, n0, kbeg + (int64_t)nfull * SBK, 1,
                                                kend, As, Bs, acc, ss);
    } else {
        small_mainloop<TA, TB, false, NORM>(p, A, B, m0, n0, kbeg, nk, kend, As, Bs, acc, ss);
    }
    // NORM: each row's 1/rms = (sum/K + eps)^-1/2 (norm.rs:21-39) combined
    // over the row's 8 threads, through LDS to the lanes holding its results,
    // which scale their accumulators by it before any epilogue
    if (NORM) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            float t = ss[i];
            t = __fadd_rn(t, __shfl_xor(t, 1, 64));
            t = __fadd_rn(t, __shfl_xor(t, 2, 64));
            t = __fadd_rn(t, __shfl_xor(t, 4, 64));
            const float mean = __fmul_rn(t, __fdiv_rn(1.0f, (float)p.k));
            if ((tid & 7) == 0)
                sm_inv[((tid + 256 * i) >> 3)] =
                    __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, p.norm_eps)));
        }
        __syncthreads();
        const int lw = tid >> 6, ll = tid & 63;
#pragma unroll
        for (int r = 0; r < 16; ++r)
            acc[r] = __fmul_rn(acc[r], sm_inv[(lw >> 1) * 32 + 8 * (r >> 2) + 4 * (ll >> 5) + (r & 3)]);
    }

    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int lr = lane & 31, lk = lane >> 5;
    // Register r of lane l is C[row][col], row = m0 + wm*32 + 8*(r/4) +
    // 4*(l/32) + r%4, col = n0 + wn*32 + l%32.
    const int64_t col = n0 + wn * 32 + lr;
    auto row_of = [&](int r) { return m0 + wm * 32 + 8 * (r >> 2) + 4 * lk + (r & 3); };

    if (p.splits > 1) {
        float *P = p.partial + (int64_t)split * M * N;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t row = row_of(r);
            if (row < M && col < N) split_put(P + row * N + col, acc[r]);
        }
        if (split_last(p, tm * p.tiles_n + tn)) split_reduce_tile(p, m0, n0, SBM, SBN, 256);
        return;
    }
    float *C = p.c + batch * p.stride_c;
    // A tile inside [M, N): the epilogue's reads all go out before its first
    // store, with no per-row branches (under row tests each read waited for
    // the stores before it: one memory round trip per row). Buffer accesses
    // from the tile's first row, each row's offset in the lane offset (as in
    // the 128x128 kernel's epilogues).
    const bool inside = m0 + SBM <= M && n0 + SBN <= N && p.ldc < (int64_t(1) << 21) &&
                        (EPI != EPI_SWIGLU_BWD || p.ldaux < (int64_t(1) << 21));
    const uint32_t lc = 4u * (uint32_t)p.ldc;
    const uint32_t vrow = (uint32_t)(wm * 32 + 4 * lk);  // row_of(r) - m0 - (8*(r/4) + r%4)
    if (EPI == EPI_SWIGLU_BWD && inside) {
        const uint32_t la = 4u * (uint32_t)p.ldaux;
        const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float *>(p.aux + m0 * p.ldaux), (short)0, kBufferRange, kBufferFlags);
        const __amdgpu_buffer_rsrc_t rc =
            __builtin_amdgcn_make_buffer_rsrc(C + m0 * p.ldc, (short)0, kBufferRange, kBufferFlags);
        float2 gu[16];
#pragma unroll
        for (int r = 0; r < 16; ++r)
            gu[r] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(
                                                   ra, (vrow + 8 * (r >> 2) + (r & 3)) * la + 8u * (uint32_t)col,
                                                   0, 0));
#pragma unroll
        for (int r = 0; r < 16; ++r)
            __builtin_amdgcn_raw_buffer_store_b64(
                __builtin_bit_cast(u32x2_t, swiglu_bwd_f(acc[r], gu[r].x, gu[r].y)), rc,
                (vrow + 8 * (r >> 2) + (r & 3)) * lc + 8u * (uint32_t)col, 0, 0);
        return;
    }
    if (EPI == EPI_SWIGLU_BWD) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t row = row_of(r);
            if (row >= M || col >= N) continue;
            const float2 gu = *reinterpret_cast<const float2 *>(p.aux + row * p.ldaux + 2 * col);
            const float2 o = swiglu_bwd_f(acc[r], gu.x, gu.y);
            *reinterpret_cast<float2 *>(C + row * p.ldc + 2 * col) = o;
        }
        return;
    }
    const float *R = p.resid ? p.resid + batch * p.stride_c : C;
    if (EPI == EPI_ACCUM && inside) {
        const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float *>(R + m0 * p.ldc), (short)0, kBufferRange, kBufferFlags);
        const __amdgpu_buffer_rsrc_t rc =
            __builtin_amdgcn_make_buffer_rsrc(C + m0 * p.ldc, (short)0, kBufferRange, kBufferFlags);
        const uint32_t vo = vrow * lc + 4u * (uint32_t)col;
        float o[16];
#pragma unroll
        for (int r = 0; r < 16; ++r)
            o[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                 rr, vo + (8 * (r >> 2) + (r & 3)) * lc, 0, 0));
#pragma unroll
        for (int r = 0; r < 16; ++r)
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, __fadd_rn(o[r], acc[r])), rc,
                                                  vo + (8 * (r >> 2) + (r & 3)) * lc, 0, 0);
        return;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) block32_epilogue<EPI>(p, C, R, row_of(r), col, lr, acc[r]);
}

// ---- K-split 32x32 GEMM -------------------------------------------------------
// For nn shapes that leave most of the chip idle with a K of a few steps (the
// tiny preset's projections: M = 2048, N = 128-704, K = 128-352) the cost is
// latency, not the MFMA rate: a 64x64 tile walks its K steps one after
// another on one workgroup. Here a workgroup owns a 32x32 tile of C and its
// NW waves take the 32-wide K steps round-robin (wave w: steps w, w + NW,
// ...), so a tile's steps run side by side and the grid holds 4x the
// workgroups. Operands go straight from memory into the MFMA layout, no LDS
// staging: lane l takes row (A) or column (B) l%32 and k 16*(l/32) .. +15 of
// a step, A as four float4 reads of its row and B as sixteen reads that are
// coalesced across the lanes. The NW partial tiles meet in LDS and are summed
// in wave order; then wave w applies the epilogue to accumulator registers
// w, w + NW, ... of the sum.
// NORM: the A rows are RMS-normalised on the way in, as in the small kernel:
// x * w feeds the MFMAs, the sums of squares of x are gathered per lane and
// combined over the lane halves and then the waves, and each row's 1/rms
// scales the summed results.
// The epilogue's own reads (the residual of EPI_ACCUM, the cos/sin of the
// rotation) are issued before the operand loads, so their latency hides
// behind the main loop instead of following it.
// MODE: 2 when the K range of every split is a multiple of 32 and the
// k-contiguous operands (A rows when !TA, B rows when TB, the norm weights)
// are 16-byte aligned: float4 reads, no predicates; 1 when only the rows are
// aligned: a lane whose 16 k values all lie in range reads them as float4,
// the lanes of the partial last step one predicated value at a time; 0
// otherwise: every read predicated. (Keeping the predicated path out of mode
// 2 keeps its registers low; a separate tail step measured slower than the
// per-lane test of mode 1.) Operands stored k-major (A when TA, B when !TB)
// are read one value per k, coalesced across the 32 lanes of a half.
// Split K (grid z > 1): each split covers k_per_split values and writes its
// partial tile; the last split of the tile sums the splits in order and
// applies the epilogue.
template <bool TA, bool TB, int EPI, bool NORM, int NW, int MODE>
__global__ __launch_bounds__(64 * NW) void gemm_f32_mfma_ksplit(KParams p) {
    __shared__ float part[NW][16][64];
    __shared__ float sm_ss[NW][32];
    __shared__ float sm_inv[32];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lr = lane & 31, lk = lane >> 5;
    const int tm = (int)blockIdx.x / p.tiles_n, tn = (int)blockIdx.x - tm * p.tiles_n;
    const int64_t m0 = (int64_t)tm * 32, n0 = (int64_t)tn * 32;
    const int64_t M = p.m, N = p.n;
    const int split = blockIdx.z;
    const int64_t kbeg = (int64_t)split * p.k_per_split;
    const int64_t kend = min(p.k, kbeg + p.k_per_split);
    const int nsteps = (int)((kend - kbeg + 31) / 32);
    // rows and columns past the edge read the last one; their results are not stored
    const int64_t am = min(m0 + lr, M - 1), bn = min(n0 + lr, N - 1);
    const float *arow = TA ? p.a + am : p.a + am * p.lda;    // then + k * (TA ? lda : 1)
    const float *bcol = TB ? p.b + bn * p.ldb : p.b + bn;    // then + k * (TB ? 1 : ldb)

    // Register r of lane l is C[m0 + 8*(r/4) + 4*(l/32) + r%4][n0 + l%32]; wave
    // w applies the epilogue to registers w + i*NW, i < NR.
    constexpr int NR = (16 + NW - 1) / NW;
    const int64_t col = n0 + lr;
    float *C = p.c;
    const float *R = p.resid ? p.resid : C;
    const bool fin = p.splits == 1;
    float pre_r[NR], pre_c[NR], pre_s[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        pre_r[i] = 0.0f;
        pre_c[i] = 1.0f;
        pre_s[i] = 0.0f;
        const int r = wave + i * NW;
        const int64_t row = m0 + 8 * (r >> 2) + 4 * lk + (r & 3);
        if (r >= 16 || !fin || row >= M || col >= N) continue;
        if (EPI == EPI_ACCUM) pre_r[i] = R[row * p.ldc + col];
        if (EPI == EPI_STORE && p.rope_cos && col < p.rope_cols) {
            const int hd = p.rope_hd, half = hd >> 1;
            const int pc = (int)col % hd;  // rows and columns below 2^31 (checked at launch)
            const int64_t t = (int64_t)((int)row % p.rope_seq) * half + (pc < half ? pc : pc - half);
            pre_c[i] = p.rope_cos[t];
            pre_s[i] = p.rope_sin[t];
        }
    }

    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = p.acc_init;
    float ss = 0.0f;
    for (int st = wave; st < nsteps; st += NW) {
        const int64_t kb = kbeg + (int64_t)st * 32 + 16 * lk;  // this lane's first k of the step
        const bool whole = MODE == 2 || (MODE == 1 && kb + 16 <= kend);
        float a[16], b[16];
        if (!TA && whole) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 v = reinterpret_cast<const float4 *>(arow + kb)[i];
                a[4 * i + 0] = v.x;
                a[4 * i + 1] = v.y;
                a[4 * i + 2] = v.z;
                a[4 * i + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j)
                a[j] = (whole || kb + j < kend) ? arow[(kb + j) * (TA ? p.lda : 1)] : -0.0f;
        }
        if (TB && whole) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 v = reinterpret_cast<const float4 *>(bcol + kb)[i];
                b[4 * i + 0] = v.x;
                b[4 * i + 1] = v.y;
                b[4 * i + 2] = v.z;
                b[4 * i + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j)
                b[j] = (whole || kb + j < kend) ? bcol[(kb + j) * (TB ? 1 : p.ldb)] : 0.0f;
        }
        if (NORM) {
            float w[16];
            if (whole) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float4 v = reinterpret_cast<const float4 *>(p.norm_w + kb)[i];
                    w[4 * i + 0] = v.x;
                    w[4 * i + 1] = v.y;
                    w[4 * i + 2] = v.z;
                    w[4 * i + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int j = 0; j < 16; ++j) w[j] = kb + j < kend ? p.norm_w[kb + j] : 0.0f;
            }
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                ss = __fadd_rn(ss, __fmul_rn(a[j], a[j]));
                a[j] = __fmul_rn(a[j], w[j]);
            }
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[j], b[j], acc, 0, 0, 0);
    }

    if (NORM) {
        // this wave's share of row lr: k 0-15 of its steps in lane lr, 16-31 in lane lr+32
        ss = __fadd_rn(ss, __shfl_xor(ss, 32, 64));
        if (lk == 0) sm_ss[wave][lr] = ss;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) part[wave][r][lane] = acc[r];
    __syncthreads();
    if (NORM) {
        if (tid < 32) {
            float t = sm_ss[0][tid];
#pragma unroll
            for (int w = 1; w < NW; ++w) t = __fadd_rn(t, sm_ss[w][tid]);
            const float mean = __fmul_rn(t, __fdiv_rn(1.0f, (float)p.k));  // norm.rs:21-39
            sm_inv[tid] = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, p.norm_eps)));
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int r = wave + i * NW;
        if (r >= 16) break;
        float v = part[0][r][lane];
#pragma unroll
        for (int w = 1; w < NW; ++w) v = __fadd_rn(v, part[w][r][lane]);
        const int rl = 8 * (r >> 2) + 4 * lk + (r & 3);
        const int64_t row = m0 + rl;
        if (NORM) v = __fmul_rn(v, sm_inv[rl]);
        if (!fin) {
            if (row < M && col < N) split_put(p.partial + ((int64_t)split * M + row) * N + col, v);
        } else if (EPI == EPI_ACCUM) {
            if (row < M && col < N) C[row * p.ldc + col] = __fadd_rn(pre_r[i], v);
        } else if (EPI == EPI_STORE && p.rope_cos) {
            // RoPE as in block32_epilogue, with the cos/sin read up front
            const int hd = p.rope_hd, half = hd >> 1;
            const float other = __shfl_xor(v, half, 64);
            if (row >= M || col >= N) continue;
            if (col < p.rope_cols) {
                const int pc = (int)col % hd;
                v = pc < half ? v * pre_c[i] - other * pre_s[i] : v * pre_c[i] + other * pre_s[i];
            }
            C[row * p.ldc + col] = v;
        } else {
            block32_epilogue<EPI>(p, C, R, row, col, lr, v);
        }
    }
    if (fin) return;
    if (split_last(p, tm * p.tiles_n + tn)) split_reduce_tile(p, m0, n0, 32, 32, 64 * NW);
}

template <bool TA, bool TB, int EPI, bool NORM, int MODE>
void launch_ksplit_mode(Context &ctx, const KParams &p, dim3 grid, int nw) {
    if (nw == 4)
        hipLaunchKernelGGL((gemm_f32_mfma_ksplit<TA, TB, EPI, NORM, 4, MODE>), grid, dim3(256), 0,
                           ctx.stream, p);
    else if (nw == 8)
        hipLaunchKernelGGL((gemm_f32_mfma_ksplit<TA, TB, EPI, NORM, 8, MODE>), grid, dim3(512), 0,
                           ctx.stream, p);
    else if (nw == 12)
        hipLaunchKernelGGL((gemm_f32_mfma_ksplit<TA, TB, EPI, NORM, 12, MODE>), grid, dim3(768),
                           0, ctx.stream, p);
    else
        hipLaunchKernelGGL((gemm_f32_mfma_ksplit<TA, TB, EPI, NORM, 16, MODE>), grid, dim3(1024),
                           0, ctx.stream, p);
}

template <bool TA, bool TB, int EPI, bool NORM>
void launch_ksplit_nw(Context &ctx, const KParams &p, dim3 grid, int mode, int nw) {
    if (mode == 2)
        launch_ksplit_mode<TA, TB, EPI, NORM, 2>(ctx, p, grid, nw);
    else if (mode == 1)
        launch_ksplit_mode<TA, TB, EPI, NORM, 1>(ctx, p, grid, nw);
    else
        launch_ksplit_mode<TA, TB, EPI, NORM, 0>(ctx, p, grid, nw);
}

// One wave per K step of a split, in multiples of four waves (one per SIMD)
// up to sixteen: a wave that walked two steps would wait on its second
// step's loads after its first step's MFMAs, and the others on it.
template <bool TA, bool TB, int EPI>
void launch_ksplit(Context &ctx, const KParams &p, dim3 grid, int mode) {
    const int64_t steps = (p.k_per_split + 31) / 32;
    const int nw = steps <= 4 ? 4 : steps <= 8 ? 8 : steps <= 12 ? 12 : 16;
    if constexpr (!TA && !TB && (EPI == EPI_STORE || EPI == EPI_SWIGLU)) {
        if (p.norm_w) {
            launch_ksplit_nw<false, false, EPI, true>(ctx, p, grid, mode, nw);
            return;
        }
    }
    launch_ksplit_nw<TA, TB, EPI, false>(ctx, p, grid, mode, nw);
}

// ---- fp32 MFMA issue-rate probe ---------------------------------------------------
// Every wave runs n MFMAs in 4 independent accumulator chains on register
// operands, with no memory traffic but one store per lane at the end. As in a
// GEMM, the operands change from one MFMA to the next: each lane cycles
// through 8 values with pseudo-random mantissas in [-1, 1) (the matrix
// cores' power, and so the clock they hold, depends on how many operand bits
// toggle; fixed operands run near the peak clock). The result is the rate
// the matrix cores sustain under full MFMA load on GEMM-like data: the
// practical ceiling under the published peak for the GEMM kernels.
__global__ __launch_bounds__(512) void mfma_peak_kernel(float *out, int n, uint32_t seed) {
    floatx16 acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[c][r] = 0.0f;
    float v[8];
    uint32_t h = seed ^ (blockIdx.x * 0x9e3779b9u) ^ (threadIdx.x * 0x85ebca6bu);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        h ^= h << 13;
        h ^= h >> 17;
        h ^= h << 5;
        v[i] = (float)(int32_t)h * (1.0f / 2147483648.0f);
    }
    for (int i = 0; i < n; i += 8) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
            acc[j & 3] = __builtin_amdgcn_mfma_f32_32x32x2f32(v[j], v[(j + 3) & 7], acc[j & 3], 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[c][r];
    out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// Sums the 128x128 kernel's split partials in split order, then applies the
// epilogue. VEC: four consecutive columns per thread (n, ldc multiples of 4,
// 16-byte aligned C, residual and partials), four splits' loads in flight.
template <int EPI, bool VEC>
__global__ __launch_bounds__(256) void splitk_reduce(const float *__restrict__ partial,
                                                     float *c, const float *resid, int64_t m,
                                                     int64_t n, int64_t ldc, int splits) {
    const int64_t total = m * n;
    if (VEC) {
        for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; 4 * q < total;
             q += (int64_t)gridDim.x * blockDim.x) {
            const int64_t idx = 4 * q;
            float4 acc = *reinterpret_cast<const float4 *>(partial + idx);
            for (int s0 = 1; s0 < splits; s0 += 4) {
                float4 v[4];
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (s0 + u < splits)
                        v[u] = *reinterpret_cast<const float4 *>(partial + (int64_t)(s0 + u) * total + idx);
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (s0 + u < splits) {
                        acc.x = __fadd_rn(acc.x, v[u].x);
                        acc.y = __fadd_rn(acc.y, v[u].y);
                        acc.z = __fadd_rn(acc.z, v[u].z);
                        acc.w = __fadd_rn(acc.w, v[u].w);
                    }
            }
            const int64_t row = idx / n, col = idx - row * n;
            float4 *dst = reinterpret_cast<float4 *>(c + row * ldc + col);
            if (EPI == EPI_ACCUM) {
                const float4 r = *reinterpret_cast<const float4 *>((resid ? resid : c) + row * ldc + col);
                acc.x = __fadd_rn(r.x, acc.x);
                acc.y = __fadd_rn(r.y, acc.y);
                acc.z = __fadd_rn(r.z, acc.z);
                acc.w = __fadd_rn(r.w, acc.w);
            }
            *dst = acc;
        }
        return;
    }
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        float acc = partial[idx];
        for (int s = 1; s < splits; ++s) acc = __fadd_rn(acc, partial[(int64_t)s * total + idx]);
        const int64_t row = idx / n, col = idx - row * n;
        float *dst = c + row * ldc + col;
        if (EPI == EPI_ACCUM)
            *dst = __fadd_rn((resid ? resid : c)[row * ldc + col], acc);
        else
            *dst = acc;
    }
}

// The tail tiles of a balanced 128x128 launch: each element sums its tile's
// tail_s pieces in piece order, then takes the epilogue (store, accumulate, or
// the SwiGLU backward into the (dg, du) pairs). TAIL_PARTS workgroups per
// tile (grid y), each thread four consecutive columns at a time with every
// piece's load issued before the adds. VEC: 16-byte aligned C (and residual /
// gate-up pairs) with ldc (ldaux) a multiple of 4, so interior columns move as
// float4; otherwise, and past the matrix's last column, one at a time.
constexpr int TAIL_PARTS = 8;

template <int EPI, bool VEC>
__global__ __launch_bounds__(256) void tail_reduce(KParams p) {
    const int t = p.tail_first + (int)blockIdx.x;
    int tm, tn;
    grouped_tile(p, t, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const float *part = p.partial + (int64_t)blockIdx.x * p.tail_s * (BM * BN);
    const float *R = p.resid ? p.resid : p.c;
    constexpr int PER = BM * BN / TAIL_PARTS;
    for (int e = (int)blockIdx.y * PER + 4 * (int)threadIdx.x; e < ((int)blockIdx.y + 1) * PER;
         e += 4 * 256) {
        const int64_t row = m0 + e / BN, col = n0 + e % BN;
        if (row >= p.m || col >= p.n) continue;
        float4 v = *reinterpret_cast<const float4 *>(part + e);
        for (int i0 = 1; i0 < p.tail_s; i0 += 4) {
            float4 w[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (i0 + u < p.tail_s)
                    w[u] = *reinterpret_cast<const float4 *>(part + (int64_t)(i0 + u) * (BM * BN) + e);
#pragma unroll
            for (int u = 0; u < 4; ++u)
                if (i0 + u < p.tail_s) {
                    v.x = __fadd_rn(v.x, w[u].x);
                    v.y = __fadd_rn(v.y, w[u].y);
                    v.z = __fadd_rn(v.z, w[u].z);
                    v.w = __fadd_rn(v.w, w[u].w);
                }
        }
        const float vv[4] = {v.x, v.y, v.z, v.w};
        if (VEC && col + 3 < p.n) {
            if (EPI == EPI_SWIGLU_BWD) {
                const float *gu = p.aux + row * p.ldaux + 2 * col;
                const float4 a = *reinterpret_cast<const float4 *>(gu);
                const float4 b = *reinterpret_cast<const float4 *>(gu + 4);
                const float2 o0 = swiglu_bwd_f(vv[0], a.x, a.y), o1 = swiglu_bwd_f(vv[1], a.z, a.w);
                const float2 o2 = swiglu_bwd_f(vv[2], b.x, b.y), o3 = swiglu_bwd_f(vv[3], b.z, b.w);
                float4 *dst = reinterpret_cast<float4 *>(p.c + row * p.ldc + 2 * col);
                dst[0] = make_float4(o0.x, o0.y, o1.x, o1.y);
                dst[1] = make_float4(o2.x, o2.y, o3.x, o3.y);
            } else if (EPI == EPI_ACCUM) {
                const float4 r = *reinterpret_cast<const float4 *>(R + row * p.ldc + col);
                *reinterpret_cast<float4 *>(p.c + row * p.ldc + col) =
                    make_float4(__fadd_rn(r.x, vv[0]), __fadd_rn(r.y, vv[1]),
                                __fadd_rn(r.z, vv[2]), __fadd_rn(r.w, vv[3]));
            } else {
                *reinterpret_cast<float4 *>(p.c + row * p.ldc + col) = v;
            }
            continue;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t cu = col + u;
            if (cu >= p.n) break;
            if (EPI == EPI_SWIGLU_BWD) {
                const float *gu = p.aux + row * p.ldaux + 2 * cu;
                const float2 o = swiglu_bwd_f(vv[u], gu[0], gu[1]);
                float *dst = p.c + row * p.ldc + 2 * cu;
                dst[0] = o.x;
                dst[1] = o.y;
            } else if (EPI == EPI_ACCUM) {
                p.c[row * p.ldc + cu] = __fadd_rn(R[row * p.ldc + cu], vv[u]);
            } else {
                p.c[row * p.ldc + cu] = vv[u];
            }
        }
    }
}

template <bool TA, bool TB, int EPI>
void launch(Context &ctx, const KParams &p, dim3 grid, bool small) {
    if constexpr (!TA && !TB && (EPI == EPI_STORE || EPI == EPI_SWIGLU)) {
        if (small && p.norm_w) {
            hipLaunchKernelGGL((gemm_f32_mfma_small<false, false, EPI, true>), grid, dim3(256), 0,
                               ctx.stream, p);
            return;
        }
    }
    if constexpr (!TA && !TB && EPI == EPI_STORE) {
        // RoPE in the 128x128 kernel's epilogue (heads of 64 or 128 columns)
        if (!small && p.rope_cos) {
            if (p.rope_hd == 64)
                hipLaunchKernelGGL((gemm_f32_mfma<TA, TB, EPI, 1>), grid, dim3(NT), 0,
                                   ctx.stream, p);
            else
                hipLaunchKernelGGL((gemm_f32_mfma<TA, TB, EPI, 2>), grid, dim3(NT), 0,
                                   ctx.stream, p);
            return;
        }
    }
    if (small)
        hipLaunchKernelGGL((gemm_f32_mfma_small<TA, TB, EPI, false>), grid, dim3(256), 0,
                           ctx.stream, p);
    else
        hipLaunchKernelGGL((gemm_f32_mfma<TA, TB, EPI>), grid, dim3(NT), 0, ctx.stream, p);
}

template <int EPI>
void dispatch_t(Context &ctx, bool ta, bool tb, const KParams &p, dim3 grid, bool small) {
    if (!ta && !tb) launch<false, false, EPI>(ctx, p, grid, small);
    else if (!ta && tb) launch<false, true, EPI>(ctx, p, grid, small);
    else if (ta && !tb) launch<true, false, EPI>(ctx, p, grid, small);
    else launch<true, true, EPI>(ctx, p, grid, small);
}

bool aligned16(const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

}  // namespace

namespace {

int cus_of(const Context &ctx) { return ctx.cu_count > 0 ? ctx.cu_count : 256; }

// Small tiles when the big ones cannot fill the chip and K is short enough
// that one workgroup walking it alone stays cheap.
bool use_small(const Context &ctx, const GemmDesc &d) {
    const int64_t big_tiles = ((d.m + BM - 1) / BM) * ((d.n + BN - 1) / BN) * d.batch;
    // (K up to 2048 for products of at most 2^29 multiply-adds: the 64x64
    // tiles' splits sum in one launch, where the 128x128 splits need the
    // reduce kernel; larger products keep the 128x128 tiles' operand reuse)
    return d.force_splits == 0 && big_tiles < cus_of(ctx) &&
           (d.k <= 1024 || (d.k <= 2048 && d.m * d.n * d.k <= (int64_t(1) << 29)));
}

// When the K-split kernel runs: 1 for the small nn shapes of one matrix whose
// K is at most 15 steps of 32 (one split; the store, accumulate and SwiGLU
// epilogues, with the RMSNorm and RoPE folds) while the 64x64 tiles number
// under two per CU (beyond that the small kernel's grid is deep enough and its
// tiles share their operands through LDS); 2 for the other products of one
// matrix whose 128x128 tiles would not give every CU one and of at most 2^28
// multiply-adds (any form but tt, store or accumulate), split along K across
// workgroups: on the benchmark sweep it wins at 0.27 GFLOP (dA, dB at K = N =
// 256: 27 -> 37 and 13 -> 23 TFLOP/s) and loses from 1 GFLOP up, where the
// other kernels' operand reuse through LDS pays; 0 otherwise.
int ksplit_kind(const Context &ctx, const GemmDesc &d) {
    const int cus = cus_of(ctx);
    const bool plain = d.epi == EPI_STORE || d.epi == EPI_ACCUM;
    const int64_t small_tiles = ((d.m + SBM - 1) / SBM) * ((d.n + SBN - 1) / SBN);
    if (use_small(ctx, d) && !d.ta && !d.tb && d.batch == 1 && d.k <= 480 &&
        small_tiles < 2 * cus && (plain || d.epi == EPI_SWIGLU))
        return 1;
    const int64_t big_tiles = ((d.m + BM - 1) / BM) * ((d.n + BN - 1) / BN);
    if (d.batch == 1 && d.force_splits == 0 && !(d.ta && d.tb) && plain && !d.norm_w &&
        !d.rope_cos && big_tiles < cus && d.m * d.n * d.k <= (int64_t(1) << 28))
        return 2;
    return 0;
}

bool vec_a_of(const GemmDesc &d, const float *a, int64_t lda) {
    const int64_t off_limit = int64_t(1) << 29;  // interior byte offsets stay below 2^31
    return (lda % 4 == 0) && (d.batch == 1 || d.stride_a % 4 == 0) && aligned16(a) &&
           lda * BM < off_limit;
}

}  // namespace

GemmFusion gemm_fusion(const Context &ctx, const GemmDesc &d) {
    GemmFusion f;
    const bool small = use_small(ctx, d);
    const bool nn = !d.ta && !d.tb && d.batch == 1 && d.k % 4 == 0 &&
                    vec_a_of(d, d.a, d.lda) && aligned16(d.norm_w) &&
                    (d.epi == EPI_STORE || d.epi == EPI_SWIGLU);
    if (small) {
        f.norm = nn && d.k <= 256;
        f.rope = d.batch == 1 && d.epi == EPI_STORE && d.rope_hd > 0 && d.rope_hd <= 32 &&
                 32 % d.rope_hd == 0;
    } else {
        // the 128x128 kernel rotates heads of 64 or 128 columns in registers;
        // the norm stays a kernel of its own (in this kernel's loads it costs
        // the registers of a ring slot, and the GEMM loses more than the norm
        // kernel takes)
        f.rope = !d.ta && !d.tb && d.batch == 1 && d.epi == EPI_STORE &&
                 (d.rope_hd == 64 || d.rope_hd == 128);
    }
    return f;
}

int64_t gemm_ce_tiles(const Context &ctx, const GemmDesc &d) {
    if (use_small(ctx, d) || d.batch != 1 || d.force_splits || d.ta || d.norm_w || d.rope_cos)
        return 0;
    return (d.n + BN - 1) / BN;
}

void gemm(Context &ctx, const GemmDesc &d) {
    if (d.m <= 0 || d.n <= 0 || d.k <= 0 || d.batch <= 0) fail(MMH_ERR_SHAPE, "gemm: empty shape");
    if (d.epi == EPI_CE && (gemm_ce_tiles(ctx, d) == 0 || !d.ce_targets || !d.ce_part || !d.ce_zt))
        fail(MMH_ERR_ARGUMENT, "gemm: the loss folds only into the 128x128 kernel of one matrix");
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
    p.resid = d.resid;
    p.aux = d.aux;
    p.ldaux = d.ldaux;
    p.ce_targets = d.ce_targets;
    p.ce_part = d.ce_part;
    p.ce_zt = d.ce_zt;
    if (d.accumulate_into_c && (d.epi != EPI_ACCUM || d.resid))
        fail(MMH_ERR_ARGUMENT, "gemm: accumulate_into_c takes EPI_ACCUM into C itself");
    p.acc_init = d.accumulate_into_c ? -0.0f : 0.0f;
    if (d.epi == EPI_SWIGLU_BWD || (d.epi == EPI_SWIGLU && d.aux)) {
        if (!d.aux || d.ldaux < (d.epi == EPI_SWIGLU ? d.n : 2 * d.n) || d.ldaux % 4 ||
            !aligned16(d.aux) ||
            (d.epi == EPI_SWIGLU_BWD && (d.ldc % 4 || !aligned16(d.c))))
            fail(MMH_ERR_ARGUMENT, "gemm: swiglu pairs need 16-byte aligned rows of >= 2n");
        if (d.batch != 1) fail(MMH_ERR_ARGUMENT, "gemm: swiglu epilogues take one matrix");
    }
    const int cus = cus_of(ctx);
    const bool small = use_small(ctx, d);
    const int kind = ksplit_kind(ctx, d);
    const bool ksplit = kind != 0;
    const GemmFusion fuse = gemm_fusion(ctx, d);
    p.tiles_m = (int)(ksplit ? (d.m + 31) / 32 : small ? (d.m + SBM - 1) / SBM : (d.m + BM - 1) / BM);
    p.tiles_n = (int)(ksplit ? (d.n + 31) / 32 : small ? (d.n + SBN - 1) / SBN : (d.n + BN - 1) / BN);
    // The interior path addresses a tile with byte offsets below 2^31 (128 rows of ld).
    const int64_t off_limit = int64_t(1) << 29;
    p.vec_a = vec_a_of(d, d.a, d.lda);
    p.vec_b = (d.ldb % 4 == 0) && (d.batch == 1 || d.stride_b % 4 == 0) && aligned16(d.b) &&
              d.ldb * BN < off_limit;
    p.vec_c = (d.ldc % 2 == 0) && (d.batch == 1 || d.stride_c % 2 == 0) &&
              (reinterpret_cast<uintptr_t>(d.c) & 7) == 0;

    // RMSNorm of A: in the small kernel's loads, or first as its own kernel.
    if (d.norm_w) {
        if (d.ta || d.batch != 1 || d.force_splits > 0)
            fail(MMH_ERR_ARGUMENT, "gemm: the A-row norm takes one row-major A");
        if (fuse.norm) {
            p.norm_w = d.norm_w;
            p.norm_eps = d.norm_eps;
        } else {
            if (!d.norm_tmp) fail(MMH_ERR_ARGUMENT, "gemm: the A-row norm needs norm_tmp");
            launch_rms_norm(ctx, d.a, d.norm_w, d.m, d.k, d.norm_eps, d.norm_tmp);
            p.a = d.norm_tmp;
            p.lda = d.k;
            p.vec_a = vec_a_of(d, d.norm_tmp, d.k);
        }
    }

    const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
    const int64_t kstep = ksplit ? 32 : small ? SBK : BK;
    const int64_t ktiles = (d.k + kstep - 1) / kstep;
    int splits = 1;
    if (d.force_splits > 0) {
        splits = d.force_splits;
    } else if (kind == 2) {
        // Up to two workgroups per CU, each split keeping >= 4 steps of 32
        // (a step per wave at least).
        while (tiles * splits < 2 * (int64_t)cus && splits < 64 && ktiles / (splits * 2) >= 4)
            splits *= 2;
    } else if (!ksplit && d.batch == 1 && d.epi != EPI_SWIGLU && d.epi != EPI_SWIGLU_BWD) {
        if (small) {
            // Split only while a split keeps >= 8 steps of 32 (the reduce
            // launch costs about what 8 steps do) and the grid is below a
            // workgroup per CU.
            while (tiles * splits < cus && splits < 16 && ktiles / (splits * 2) >= 8)
                splits *= 2;
        } else {
            // Fill the chip: a tile per CU (two, with twice the split partials
            // written and summed, measured 7-10% slower from 1 GFLOP up: the
            // sweep's dB forms, the training's 2048 x 2048 weight gradient), at
            // least 8 K-steps per split.
            const int64_t target = (int64_t)cus;
            while (tiles * splits < target && splits < 16 && ktiles / (splits * 2) >= 8)
                splits *= 2;
        }
    }
    if (d.batch > 1 || d.epi == EPI_SWIGLU || d.epi == EPI_SWIGLU_BWD || d.epi == EPI_CE ||
        p.norm_w || kind == 1)
        splits = 1;
    const int64_t kt_per = (ktiles + splits - 1) / splits;
    p.k_per_split = kt_per * kstep;
    splits = (int)((ktiles + kt_per - 1) / kt_per);
    p.splits = splits;
    if (splits > 1) {
        // 64x64 and 32x32 tiles: the last split of each tile sums the
        // partials in split order and applies the epilogue (one launch;
        // every such grid has fewer tiles than two per CU, far below the
        // counters); 128x128 tiles: splitk_reduce after the launch
        if (small || ksplit) {
            p.tickets = d.scratch ? d.scratch_tickets : ctx.tickets;
            if (!p.tickets || tiles > Context::kTickets)
                fail(MMH_ERR_OTHER, "gemm: no split counters for " + std::to_string(tiles) + " tiles");
            p.split_accum = d.epi == EPI_ACCUM ? 1 : 0;
        }
        const size_t need_bytes = (size_t)splits * d.m * d.n * 4;
        if (d.scratch) {
            if (need_bytes > d.scratch_bytes)
                fail(MMH_ERR_SHAPE, "gemm: the split-K partials of a " + std::to_string(d.m) +
                                        " x " + std::to_string(d.n) + " product (" +
                                        std::to_string(splits) + " splits) need " +
                                        std::to_string(need_bytes) + " bytes; the scratch holds " +
                                        std::to_string(d.scratch_bytes));
            p.partial = d.scratch;
        } else {
            p.partial = static_cast<float *>(ctx.get_scratch(need_bytes));
        }
    }

    // RoPE in the small kernel's epilogue when a head fits 32 columns.
    const bool rope = d.rope_cos != nullptr;
    if (rope) {
        if (d.batch != 1 || d.rope_hd <= 0 || d.rope_hd % 2 || d.rope_seq <= 0 ||
            d.m % d.rope_seq || d.rope_cols % d.rope_hd || d.rope_cols > d.n || !d.rope_sin ||
            d.m > INT32_MAX || d.n > INT32_MAX)
            fail(MMH_ERR_ARGUMENT, "gemm: bad rope arguments");
        if (fuse.rope && splits == 1) {
            p.rope_cos = d.rope_cos;
            p.rope_sin = d.rope_sin;
            p.rope_seq = (int)d.rope_seq;
            p.rope_hd = (int)d.rope_hd;
            p.rope_cols = (int)d.rope_cols;
        }
    }

    // Tail balance for the 128x128 kernel: with tiles = q * CUs + R (q >= 1,
    // R > 0) the CUs that draw q + 1 tiles set the launch's length. The last R
    // tiles instead split K into s pieces (each a workgroup of its own, at
    // least 16 K-steps long), so every CU takes about q + R/CUs tiles' work;
    // tail_reduce sums each tile's pieces in order. Chosen when it shortens
    // the longest CU's share by at least 5%.
    const int epi = splits > 1 ? EPI_STORE : d.epi;
    if (!ksplit && !small && splits == 1 && d.batch == 1 && !p.rope_cos && d.force_splits == 0 &&
        (epi == EPI_STORE || epi == EPI_ACCUM || epi == EPI_SWIGLU_BWD)) {
        const int64_t cus = cus_of(ctx), q = tiles / cus, R = tiles % cus;
        int best_s = 1;
        double best = (double)(q + (R > 0));
        for (int s : {2, 3, 4, 6, 8}) {
            if (q < 1 || R == 0 || ktiles / s < 16) break;
            const double span = (double)q + (double)((R * s + cus - 1) / cus) / s;
            if (span < best - 1e-9) {
                best = span;
                best_s = s;
            }
        }
        const size_t need = (size_t)R * best_s * BM * BN * 4;
        if (best_s > 1 && best <= 0.95 * (double)(q + 1)) {
            // the choice never depends on the caller's scratch, so a fixed
            // scratch gives the same summation order (and bits) as the
            // workspace, or the call is refused
            if (d.scratch && need > d.scratch_bytes)
                fail(MMH_ERR_SHAPE, "gemm: the tail pieces of a " + std::to_string(d.m) + " x " +
                                        std::to_string(d.n) + " product (" + std::to_string(R) +
                                        " tiles x " + std::to_string(best_s) + " pieces) need " +
                                        std::to_string(need) + " bytes; the scratch holds " +
                                        std::to_string(d.scratch_bytes));
            p.tail_first = (int)(tiles - R);
            p.tail_s = best_s;
            p.tail_k = (ktiles + best_s - 1) / best_s * BK;
            p.partial = d.scratch ? d.scratch : static_cast<float *>(ctx.get_scratch(need));
        }
    }
    const int64_t tail_pieces = p.tail_s > 1 ? (tiles - p.tail_first) * p.tail_s : 0;
    const int64_t grid_x = p.tail_s > 1 ? p.tail_first + tail_pieces : tiles;
    if (grid_x > 0x7fffffff || d.batch > 65535) fail(MMH_ERR_SHAPE, "gemm: grid too large");
    dim3 grid((unsigned)grid_x, (unsigned)d.batch, (unsigned)splits);
    if (ksplit) {
        // The k-contiguous operands (A when !ta, B when tb, the norm weights)
        // decide between vector and predicated reads (vec_a / vec_b hold
        // ld % 4 == 0 and a 16-byte aligned base).
        const bool vec = (d.ta || p.vec_a) && (!d.tb || p.vec_b) &&
                         (!p.norm_w || aligned16(p.norm_w));
        const int mode = !vec ? 0 : d.k % 32 == 0 ? 2 : 1;
        if (epi == EPI_SWIGLU)
            launch_ksplit<false, false, EPI_SWIGLU>(ctx, p, grid, mode);
        else if (!d.ta && !d.tb)
            (epi == EPI_ACCUM ? launch_ksplit<false, false, EPI_ACCUM>
                              : launch_ksplit<false, false, EPI_STORE>)(ctx, p, grid, mode);
        else if (!d.ta)
            (epi == EPI_ACCUM ? launch_ksplit<false, true, EPI_ACCUM>
                              : launch_ksplit<false, true, EPI_STORE>)(ctx, p, grid, mode);
        else
            (epi == EPI_ACCUM ? launch_ksplit<true, false, EPI_ACCUM>
                              : launch_ksplit<true, false, EPI_STORE>)(ctx, p, grid, mode);
    } else if (epi == EPI_CE) {
        if (d.tb)
            hipLaunchKernelGGL((gemm_f32_mfma<false, true, EPI_CE>), grid, dim3(NT), 0,
                               ctx.stream, p);
        else
            hipLaunchKernelGGL((gemm_f32_mfma<false, false, EPI_CE>), grid, dim3(NT), 0,
                               ctx.stream, p);
    } else if (epi == EPI_SWIGLU) {
        if (d.ta || d.tb) fail(MMH_ERR_ARGUMENT, "gemm: swiglu epilogue needs the nn form");
        launch<false, false, EPI_SWIGLU>(ctx, p, grid, small);
    } else if (epi == EPI_SWIGLU_BWD) {
        if (d.ta || !d.tb) fail(MMH_ERR_ARGUMENT, "gemm: swiglu backward epilogue needs the nt form");
        launch<false, true, EPI_SWIGLU_BWD>(ctx, p, grid, small);
    } else if (epi == EPI_ACCUM) {
        dispatch_t<EPI_ACCUM>(ctx, d.ta, d.tb, p, grid, small);
    } else {
        dispatch_t<EPI_STORE>(ctx, d.ta, d.tb, p, grid, small);
    }
    check_hip(hipGetLastError(), "gemm launch");
    if (splits > 1 && !p.tickets) {
        const int64_t total = d.m * d.n;
        const bool vec = d.n % 4 == 0 && d.ldc % 4 == 0 && aligned16(d.c) &&
                         aligned16(p.partial) && (!d.resid || aligned16(d.resid));
        const int64_t items = vec ? total / 4 : total;
        const unsigned blocks = (unsigned)std::min<int64_t>((items + 255) / 256, 8192);
#define MMH_SPLITK(E, V)                                                                   \
    hipLaunchKernelGGL((splitk_reduce<E, V>), dim3(blocks), dim3(256), 0, ctx.stream, p.partial, \
                       d.c, E == EPI_ACCUM ? d.resid : nullptr, d.m, d.n, d.ldc, splits)
        if (d.epi == EPI_ACCUM) {
            if (vec) MMH_SPLITK(EPI_ACCUM, true); else MMH_SPLITK(EPI_ACCUM, false);
        } else {
            if (vec) MMH_SPLITK(EPI_STORE, true); else MMH_SPLITK(EPI_STORE, false);
        }
#undef MMH_SPLITK
        check_hip(hipGetLastError(), "split-k reduce launch");
    }
    if (p.tail_s > 1) {
        const dim3 rg((unsigned)(tiles - p.tail_first), TAIL_PARTS);
        const bool vec = d.ldc % 4 == 0 && aligned16(d.c) && (!d.resid || aligned16(d.resid)) &&
                         (epi != EPI_SWIGLU_BWD || (d.ldaux % 4 == 0 && aligned16(d.aux)));
#define MMH_TAIL(E)                                                                        \
    do {                                                                                   \
        if (vec)                                                                           \
            hipLaunchKernelGGL((tail_reduce<E, true>), rg, dim3(256), 0, ctx.stream, p);   \
        else                                                                               \
            hipLaunchKernelGGL((tail_reduce<E, false>), rg, dim3(256), 0, ctx.stream, p);  \
    } while (0)
        if (epi == EPI_SWIGLU_BWD)
            MMH_TAIL(EPI_SWIGLU_BWD);
        else if (epi == EPI_ACCUM)
            MMH_TAIL(EPI_ACCUM);
        else
            MMH_TAIL(EPI_STORE);
#undef MMH_TAIL
        check_hip(hipGetLastError(), "tail reduce launch");
    }
    if (rope && !p.rope_cos)
        launch_rope_strided(ctx, d.c, d.rope_seq * d.ldc, d.rope_hd, d.ldc, d.m / d.rope_seq,
                            d.rope_cols / d.rope_hd, d.rope_seq, d.rope_hd, d.rope_cos,
                            d.rope_sin);
}

double mfma_peak_tflops(Context &ctx) {
    // two 512-thread workgroups per CU (4 waves per SIMD), 8192 MFMAs per wave
    // (about 0.5 ms a launch); 20 launches first bring the clock to its
    // steady state under this load, then 40 are timed
    const int blocks = 2 * cus_of(ctx), threads = 512, n = 8192;
    float *out = static_cast<float *>(ctx.get_scratch((size_t)blocks * threads * 4));
    for (int i = 0; i < 20; ++i)
        hipLaunchKernelGGL(mfma_peak_kernel, dim3(blocks), dim3(threads), 0, ctx.stream, out, n,
                           1u + (uint32_t)i);
    check_hip(hipGetLastError(), "mfma probe launch");
    const int reps = 40;
    check_hip(hipEventRecord(ctx.t0, ctx.stream), "event record");
    for (int i = 0; i < reps; ++i)
        hipLaunchKernelGGL(mfma_peak_kernel, dim3(blocks), dim3(threads), 0, ctx.stream, out, n,
                           100u + (uint32_t)i);
    check_hip(hipGetLastError(), "mfma probe launch");
    check_hip(hipEventRecord(ctx.t1, ctx.stream), "event record");
    check_hip(hipEventSynchronize(ctx.t1), "event sync");
    float ms = 0.0f;
    check_hip(hipEventElapsedTime(&ms, ctx.t0, ctx.t1), "elapsed time");
    const double flops = 2.0 * 32 * 32 * 2 * (double)n * (blocks * threads / 64) * reps;
    return flops / (ms * 1e-3) / 1e12;
}

}  // namespace mmh
