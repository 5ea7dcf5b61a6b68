// The whole loss-only forward of a small model (model.rs:127-183: embedding,
// the blocks of block.rs:77-81, final norm, head, cross-entropy mean) as ONE
// persistent launch, for the presets whose per-operation kernels are all
// latency-bound (the tiny preset: 25 kernels of 4-25 us, each boundary paying
// an L2 write-back and invalidate on every XCD).
//
// MI355X layout: 8 XCDs of 32 CUs, each XCD with its own L2. A workgroup
// reads the XCD it runs on from the XCC_ID hardware register and takes the
// next slot of that XCD's team (the launch is 8 x 32 workgroups, dealt
// round-robin over the XCDs). The team of XCD x owns the sequences s with s % 8 == x,
// so every intermediate a team produces is consumed inside the same XCD:
//   * results leave with plain stores; after s_waitcnt vmcnt(0) they sit in
//     the XCD's L2, where device-scope (sc1) loads of other CUs of the same
//     XCD find them (sc1 loads miss the per-CU L1 and take dirty L2 lines);
//   * a finished task bumps a device-scope atomic counter; a waiting task
//     polls it with device-scope atomic loads and then reads the data with
//     sc1 loads;
//   * no cross-XCD fence is needed (agent-scope release/acquire fences write
//     back and invalidate the whole L2: ~18 us per round measured on the box,
//     against ~1.3 us for a 32-workgroup round of the scheme above).
// The only cross-XCD data are the per-row-block f64 loss sums, written with
// sc1 stores (write-through) and read with sc1 loads by the last workgroup to
// finish, which forms the mean and resets the counters for the next launch.
//
// Work: a fixed list of tasks in dependency order, dealt round-robin to the
// team's workgroups (task t to slot t % 32), each waiting only on tasks
// earlier in the list, so with every workgroup resident the list drains.
// Every wait is bounded: past the limit the workgroup sets an error bit and
// stops, the others see the error word and stop, and the host raises.
// Per layer l and 32-row block q of a sequence:
//   Q(l,q,c)   x rows (layer 0: the embedding rows of the ids, also stored as
//              x) RMS-normalised in the loads, times Wqkv, RoPE on q and k
//              (128-column blocks; every layer has its own qkv buffer, so no
//              later layer overwrites keys an attention task still reads)
//   A(l,h,q)   causal attention of query block q for head h over key tiles
//              0..q (the online softmax of attention.hip's key-split kernel),
//              then that head's share of the O projection: ctx_h . Wo[rows of
//              head h], stored as a 32 x d partial
//   G(l,q,c)   the block's x plus the heads' partials in head order (the
//              attention residual of block.rs:79; column block 0 stores it as
//              x2), RMS-normalised, times Wgu, h = silu(gate) * up (256 packed
//              gate/up columns: 128 columns of h per task)
//   D(l,q,c)   x = x2 + h . Wd (32-column blocks, K split over the 8 waves)
// then HEAD(q,c): logits of 256 vocabulary rows (final norm folded), per row
// the (max, sum of exp) pair and the target logit; COMB(q): the rows' losses
// (ops_reduce.rs:236-259) and their f64 sum.
//
// Every global access goes through a buffer descriptor sized to its buffer,
// so an index outside it reads zero / writes nothing instead of faulting.
#include <vector>

#include "mmh_internal.h"

#include <type_traits>

namespace mmh {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((vector_size(16)));
typedef unsigned int u32x2 __attribute__((vector_size(8)));
typedef __amdgpu_buffer_rsrc_t Rsrc;

constexpr int kNT = 512;               // 8 waves per workgroup
constexpr int kDev = 16;               // sc1: device-coherent load / write-through store
constexpr uint32_t kOOB = 0x80000000u;  // an offset past every descriptor: reads 0
constexpr int kSpinLimit = 1 << 18;
constexpr int kLdsFloats = 8 * 32 * 33 + 2 * 8 * 32;
constexpr int kRowStage = 32 * (256 + 4);  // the normalised rows of a task (floats)
constexpr int kLossSlots = kRowStage / 2;  // f64 row-block sums the last workgroup parks there

// task stages within a layer (stage 2, the O projection, rides on the
// attention tasks and the gate/up tasks' loads; its counter slot is unused),
// then the head (5)
enum : int { ST_Q = 0, ST_A = 1, ST_G = 3, ST_D = 4 };

__device__ __forceinline__ Rsrc rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, (int)bytes, 0x00020000);
}
template <int AUX>
__device__ __forceinline__ float4 ld4(Rsrc r, uint32_t off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX));
}
template <int AUX>
__device__ __forceinline__ float ld1(Rsrc r, uint32_t off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, AUX));
}
template <int AUX>
__device__ __forceinline__ int ldi(Rsrc r, uint32_t off) {
    return (int)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, AUX);
}
template <int AUX>
__device__ __forceinline__ float2 ld2(Rsrc r, uint32_t off) {
    return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, AUX));
}
template <int AUX>
__device__ __forceinline__ float4 ld4s(Rsrc r, uint32_t voff, int soff) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, AUX));
}
template <int AUX>
__device__ __forceinline__ float ld1s(Rsrc r, uint32_t voff, int soff) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, AUX));
}
__device__ __forceinline__ void st4s(Rsrc r, uint32_t voff, int soff, float4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, voff, soff, 0);
}
template <int AUX = 0>
__device__ __forceinline__ void st1(Rsrc r, uint32_t off, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, AUX);
}
template <int AUX = 0>
__device__ __forceinline__ void st2(Rsrc r, uint32_t off, float2 v) {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, off, 0, AUX);
}

__device__ __forceinline__ int xcc_id() {
    // HW_REG_XCC_ID (20), bits [3:0]
    return __builtin_amdgcn_s_getreg(20 | (0 << 6) | ((16 - 1) << 11)) & 0xf;
}

}  // namespace

struct FusedP {
    const float *w;       // the device weight layout
    float *f;             // the fused arena (every region below, in floats)
    const int32_t *ids;   // staged ids; the targets at ids + tgt_off
    float *loss;
    int32_t *err;         // error bits (a word of the arena, also addressed here)
    uint64_t *stamps;     // diagnostic clock stamps (start, end) per workgroup, or null
    int32_t rr;           // team slots from the dispatch order (blockIdx / 8), see the kernel
    uint32_t w_bytes, f_bytes, i_bytes, tgt_off;
    // arena regions (float offsets)
    uint32_t o_x, o_h, o_qkv, o_part, o_zt, o_rl, o_p64, o_ctl, o_err, o_cos, o_sin, o_op, o_x2;
    uint32_t ctl_ints;
    int B, T, d, H, Hkv, ff, ff_pad, V, L, tie, qc, kvw, n;
    float eps, scale;
    // weights (floats): layer l's block at blk0 + l * blk, then its parts
    int blk0, blk, o_wqkv, o_wo, o_mn, o_wgu, o_wd, o_fn, o_head;
    int nrb, smax, nsi, nq_c, ng_c, nd_c, nh_c;
    int hb, nh_t;  // head: 256-row vocabulary blocks per task, tasks per row block
};

namespace {

// Counter of stage instance si, sequence slot j, row block q on XCD x.
__device__ __forceinline__ int cnt_index(const FusedP &p, int x, int si, int j, int q) {
    return 64 + ((x * p.nsi + si) * p.smax + j) * p.nrb + q;
}

// Wave-wide bounded wait until the n counters ctl[first ..] all reach target
// (device-scope atomic loads: polled afresh every round). False on time-out
// (error bit 1 set) or when another workgroup has reported an error.
__device__ bool wave_wait(int32_t *ctl, int first, int n, int target, int32_t *err,
                          uint32_t ctl_ints, int lane) {
    for (int it = 0;; ++it) {
        bool done = true;
        for (int i = lane; i < n; i += 64) {
            const uint32_t ci = (uint32_t)(first + i);
            done &= ci < ctl_ints &&
                    __hip_atomic_load(ctl + ci, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= target;
        }
        if (__all(done)) return true;
        if ((it & 31) == 31 &&
            __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0)
            return false;
        if (it >= kSpinLimit) {
            if (lane == 0) __hip_atomic_fetch_or(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// The three descriptors: weights (read-only, cached loads), the arena
// (activations written in the launch: sc1 loads), the staged ids / targets.
struct Res {
    Rsrc w, f, i;
};

// Register r of lane l of a 32x32 MFMA block holds row 8*(r/4) + 4*(l/32) + r%4.
__device__ __forceinline__ int row_local(int r, int lk) { return 8 * (r >> 2) + 4 * lk + (r & 3); }

// Lane exchanges without the LDS unit: v of lane l ^ 1 (DPP quad_perm
// [1,0,3,2]), of lane l ^ 8 (DPP row_ror:8 within a 16-lane row), of lane
// l ^ 16 (v_permlane16_swap: lanes 0-15 of each half receive lanes 16-31 in
// the second result, lanes 16-31 the first ones in the first).
__device__ __forceinline__ float lane_xor1(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_xor8(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_xor16(float v, int lane) {
    const auto pr = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((lane & 16) ? pr[0] : pr[1]);
}
// The two values of lanes l and l ^ 32 combined (max or sum: order-free).
__device__ __forceinline__ float pair32_max(float v) {
    const auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(pr[0]), __uint_as_float(pr[1]));
}
__device__ __forceinline__ float pair32_sum(float v) {
    const auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(pr[0]) + __uint_as_float(pr[1]);
}

// A task's weight operands, loaded before its dependency wait. GEMM tasks:
// the B values of the wave's first two K steps (v[16 s + j]: column
// n0 + 32*ct + l%32, k = 32*(kg + s*KG) + 16*(l/32) + j); the head: the
// vocabulary rows' values of its first two K steps.
struct GemmPre {
    float v[32];
};

// Issues the B loads of GemmPre for a block of CT 32-column tiles of W
// (row-major [K][ldb] at float offset wo in the weights). Wave w takes
// column tile w % CT and the K steps w / CT, w / CT + KG, ... (KG = 8 / CT).
template <int CT>
__device__ __forceinline__ void gemm_fetch_b(int tid, const Res &R, int wo, int ldb, int n0, int N,
                                             int K, GemmPre &g) {
    constexpr int KG = 8 / CT;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, lr = lane & 31, lk = lane >> 5;
    const int ct = wave % CT, kg = wave / CT;
    const int ns = (K + 31) >> 5;
    const int col = min(n0 + 32 * ct + lr, N - 1);
    const uint32_t vb = 4u * ((uint32_t)(wo + col) + 16u * lk * (uint32_t)ldb);
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
        const int st = kg + s2 * KG;
        if (st < ns) {
#pragma unroll
            for (int j = 0; j < 16; ++j) g.v[16 * s2 + j] = ld1s<0>(R.w, vb, 4 * (32 * st + j) * ldb);
        }
    }
}

// The product of a 32-row block of A with the block of gemm_fetch_b, into
// the wave's accumulator. A rows: AS 0 reads row row_a of an activation
// region (float offset a_base, stride lda; sc1 loads); AS 1 reads the
// embedding row of the row's id (weights) and, when xcopy, column tile 0
// stores it as the row of x. NORM: the A values are multiplied by the norm
// weights staged in LDS (nw) and their squares summed into ss. K is a
// multiple of 4; k >= K contributes zero. Steps past the first two per wave
// (K > 64 * KG) stream both operands.
template <int CT, int AS, bool NORM>
__device__ __forceinline__ void gemm_run(int tid, const FusedP &p, const Res &R, uint32_t a_base,
                                         int lda, int row_a, bool xcopy_ok, const GemmPre &g,
                                         int wo, int ldb, int n0, int N, int K, const float *nw,
                                         floatx16 &acc, float &ss) {
    constexpr int KG = 8 / CT;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, lr = lane & 31, lk = lane >> 5;
    const int ct = wave % CT, kg = wave / CT;
    const int ns = (K + 31) >> 5;
    uint32_t va;
    if (AS == 1) {
        const int id = ldi<0>(R.i, 4u * row_a);
        va = 4u * (uint32_t)id * (uint32_t)p.d + 64u * lk;
    } else {
        va = 4u * (a_base + (uint32_t)row_a * (uint32_t)lda) + 64u * lk;
    }
    const uint32_t vx = 4u * (p.o_x + (uint32_t)row_a * (uint32_t)p.d) + 64u * lk;
    const bool xcopy = AS == 1 && ct == 0 && xcopy_ok;
    auto load_a = [&](int st, float (&a)[16]) __attribute__((always_inline)) {
        const int sa = 128 * st;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = AS == 1 ? ld4s<0>(R.w, va + 16u * i, sa) : ld4s<kDev>(R.f, va + 16u * i, sa);
            a[4 * i + 0] = v.x;
            a[4 * i + 1] = v.y;
            a[4 * i + 2] = v.z;
            a[4 * i + 3] = v.w;
        }
    };
    auto compute = [&](int st, float (&a)[16], const float *b) __attribute__((always_inline)) {
        const int kb = 32 * st + 16 * lk;  // this lane's first k
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (kb + 4 * i >= K) a[4 * i] = a[4 * i + 1] = a[4 * i + 2] = a[4 * i + 3] = 0.0f;
        if (xcopy) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (kb + 4 * i < K)
                    st4s(R.f, vx + 16u * i, 128 * st,
                         make_float4(a[4 * i], a[4 * i + 1], a[4 * i + 2], a[4 * i + 3]));
        }
        if (NORM) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 wv = kb + 4 * i < K ? *reinterpret_cast<const float4 *>(nw + kb + 4 * i)
                                                 : make_float4(0.f, 0.f, 0.f, 0.f);
                const float wn[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    ss = __fadd_rn(ss, __fmul_rn(a[4 * i + e], a[4 * i + e]));
                    a[4 * i + e] = __fmul_rn(a[4 * i + e], wn[e]);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 16; ++j)
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[j], kb + j < K ? b[j] : 0.0f, acc, 0, 0, 0);
    };
    const int st0 = kg, st1 = kg + KG;
    float a0[16], a1[16];
    if (st0 < ns) load_a(st0, a0);
    if (st1 < ns) load_a(st1, a1);
    if (st0 < ns) compute(st0, a0, g.v);
    if (st1 < ns) compute(st1, a1, g.v + 16);
    if (kg + 2 * KG < ns) {
        const int col = min(n0 + 32 * ct + lr, N - 1);
        const uint32_t vb = 4u * ((uint32_t)(wo + col) + 16u * lk * (uint32_t)ldb);
        for (int st = kg + 2 * KG; st < ns; st += KG) {
            float a[16], b[16];
            load_a(st, a);
#pragma unroll
            for (int j = 0; j < 16; ++j) b[j] = ld1s<0>(R.w, vb, 4 * (32 * st + j) * ldb);
            compute(st, a, b);
        }
    }
}

// Stages the block's rows into xs (row stride d + 4 floats), RMS-normalised
// as norm.rs:21-39 rounds them: y = (x * inv) * w with inv = (mean(x^2) +
// eps)^-1/2 and w the norm weights staged in nw. 16 threads per row (the
// 512 threads cover the 32 rows), each with d / 64 float4s; the row's sum of
// squares meets over the 16 lanes by XOR exchanges, so every lane holds the
// same sum. AS 0: rows of x (sc1 loads); AS 1: the embedding rows of the ids
// (weights), also stored as the rows of x when xcopy; AS 2: the rows of x
// plus the heads' O-projection partials (x + ((p_0 + p_1) + ...), block.rs:79),
// stored as the rows of x2 when xcopy (the down projection's residual; x
// itself stays as it is while the row block's other gate/up tasks read it).
// Rows past `rows` repeat the last one.
template <int AS>
__device__ __forceinline__ void stage_norm_rows(int tid, const FusedP &p, const Res &R, int row0,
                                                int rows, const float *nw, float *xs, bool xcopy) {
    const int r = tid >> 4, tl = tid & 15;
    const int d = p.d, xst = d + 4;
    const int row = row0 + min(r, rows - 1);
    uint32_t base;
    if (AS == 1) {
        const int id = ldi<0>(R.i, 4u * row);
        base = 4u * (uint32_t)id * (uint32_t)d;
    } else {
        base = 4u * (p.o_x + (uint32_t)row * (uint32_t)d);
    }
    float4 v[4];
    float ss = 0.0f;
    if (AS == 2) {
        const uint32_t pb = 4u * (p.o_op + (uint32_t)row * (uint32_t)p.H * (uint32_t)d);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int k = 4 * (tl + 16 * i);
            if (k < d) {
                float4 sm = ld4<kDev>(R.f, pb + 4u * k);
                for (int h2 = 1; h2 < p.H; ++h2) {
                    const float4 pv = ld4<kDev>(R.f, pb + 4u * (h2 * d + k));
                    sm = make_float4(__fadd_rn(sm.x, pv.x), __fadd_rn(sm.y, pv.y), __fadd_rn(sm.z, pv.z),
                                     __fadd_rn(sm.w, pv.w));
                }
                const float4 xv = ld4<kDev>(R.f, base + 4u * k);
                v[i] = make_float4(__fadd_rn(xv.x, sm.x), __fadd_rn(xv.y, sm.y), __fadd_rn(xv.z, sm.z),
                                   __fadd_rn(xv.w, sm.w));
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int k = 4 * (tl + 16 * i);
        if (k < d) {
            if (AS != 2) v[i] = AS == 1 ? ld4<0>(R.w, base + 4u * k) : ld4<kDev>(R.f, base + 4u * k);
            ss = __fadd_rn(ss, __fmul_rn(v[i].x, v[i].x));
            ss = __fadd_rn(ss, __fmul_rn(v[i].y, v[i].y));
            ss = __fadd_rn(ss, __fmul_rn(v[i].z, v[i].z));
            ss = __fadd_rn(ss, __fmul_rn(v[i].w, v[i].w));
        }
    }
    ss = __fadd_rn(ss, lane_xor1(ss));
    ss = __fadd_rn(ss, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, ss), 0x4E, 0xF, 0xF, false)));
    ss = __fadd_rn(ss, __shfl_xor(ss, 4, 16));
    ss = __fadd_rn(ss, __shfl_xor(ss, 8, 16));
    const float mean = __fmul_rn(ss, __fdiv_rn(1.0f, (float)d));
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(mean, p.eps)));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int k = 4 * (tl + 16 * i);
        if (k < d) {
            if (AS != 0 && xcopy && r < rows)
                __builtin_amdgcn_raw_buffer_store_b128(
                    __builtin_bit_cast(u32x4, v[i]), R.f,
                    4u * ((AS == 2 ? p.o_x2 : p.o_x) + (uint32_t)row * (uint32_t)d + k), 0, 0);
            const float4 w = *reinterpret_cast<const float4 *>(nw + k);
            *reinterpret_cast<float4 *>(xs + r * xst + k) =
                make_float4(__fmul_rn(__fmul_rn(v[i].x, inv), w.x), __fmul_rn(__fmul_rn(v[i].y, inv), w.y),
                            __fmul_rn(__fmul_rn(v[i].z, inv), w.z), __fmul_rn(__fmul_rn(v[i].w, inv), w.w));
        }
    }
}

// The product of the staged rows xs (32 x K, stride K + 4) with the block of
// gemm_fetch_b into the wave's accumulator (K a multiple of 32 here: d).
template <int CT>
__device__ __forceinline__ void gemm_run_lds(int tid, const Res &R, const float *xs,
                                             const GemmPre &g, int wo, int ldb, int n0, int N,
                                             int K, floatx16 &acc) {
    constexpr int KG = 8 / CT;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, lr = lane & 31, lk = lane >> 5;
    const int ct = wave % CT, kg = wave / CT;
    const int ns = K >> 5;
    const float *xr = xs + lr * (K + 4) + 16 * lk;
    auto step = [&](int st, const float *b) __attribute__((always_inline)) {
        float a[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = *reinterpret_cast<const float4 *>(xr + 32 * st + 4 * i);
            a[4 * i + 0] = v.x;
            a[4 * i + 1] = v.y;
            a[4 * i + 2] = v.z;
            a[4 * i + 3] = v.w;
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[j], b[j], acc, 0, 0, 0);
    };
    if (kg < ns) step(kg, g.v);
    if (kg + KG < ns) step(kg + KG, g.v + 16);
    if (kg + 2 * KG < ns) {
        const int col = min(n0 + 32 * ct + lr, N - 1);
        const uint32_t vb = 4u * ((uint32_t)(wo + col) + 16u * lk * (uint32_t)ldb);
        for (int st = kg + 2 * KG; st < ns; st += KG) {
            float b[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) b[j] = ld1s<0>(R.w, vb, 4 * (32 * st + j) * ldb);
            step(st, b);
        }
    }
}

// The KG partial tiles of each column tile meet through LDS: wave (ct, kg)
// then owns registers kg, kg + KG, ... (16 / KG of them) of its column tile
// and holds their sums, taken in K-group order, in acc[0 .. 16 / KG). With
// KG = 1 acc is already whole.
template <int CT>
__device__ __forceinline__ void share_block(int tid, float *lds, floatx16 &acc) {
    constexpr int KG = 8 / CT, NR = 16 / KG;
    if (KG == 1) return;
    const int wave = tid >> 6, lane = tid & 63;
    const int ct = wave % CT, kg = wave / CT;
#pragma unroll
    for (int r = 0; r < 16; ++r) lds[(wave * 16 + r) * 64 + lane] = acc[r];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int r = kg + i * KG;
        float v = lds[(ct * 16 + r) * 64 + lane];
#pragma unroll
        for (int g = 1; g < KG; ++g) v = __fadd_rn(v, lds[((ct + g * CT) * 16 + r) * 64 + lane]);
        acc[i] = v;
    }
}

// The causal attention of query block qb, head hh of sequence s (layer
// buffer qkv_off floats into the arena): attention.hip's key-split scheme
// with 8 waves taking the key tiles round-robin.
template <int HD>
__device__ __forceinline__ void attention_task(int tid, const FusedP &p, const Res &R, float *lds,
                                               uint32_t qkv_off, int s, int hh, int qb,
                                               float *ctx) {
    constexpr int NS = HD / 2;
    constexpr int OS = HD + 1;
    float *sm_o = lds;                   // [8][32 * OS]
    float *sm_m = lds + 8 * 32 * OS;     // [8][32]
    float *sm_l = sm_m + 8 * 32;         // [8][32]
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int lq = lane & 31, lh = lane >> 5;
    const int T = p.T, qc = p.qc;
    const int kvh = hh / (p.H / p.Hkv);
    const int q0 = qb * 32, qi = q0 + lq;
    const int ntiles = min(q0 + 31, T - 1) / 32 + 1;
    const uint32_t rbase = (uint32_t)s * (uint32_t)T;  // first row of the sequence
    const uint32_t qo = qkv_off + hh * HD, ko = qkv_off + p.d + kvh * HD,
                   vo = qkv_off + p.d + p.kvw + kvh * HD;
    auto at = [&](uint32_t colbase, int t) -> uint32_t {
        return 4u * (colbase + (rbase + (uint32_t)t) * (uint32_t)qc);
    };
    // Lane parts of the K and V offsets; a tile's rows add kt * 32 * qc floats
    // (uniform). Keys past T read whatever follows (finite or zero: the
    // descriptor stops at the arena's end) and are masked; V rows past T are
    // clamped to row T-1 (a partial last tile), since P = 0 must not meet NaN.
    const uint32_t vk_lane = at(ko, lq) + 4u * (lh * NS);
    const uint32_t vv_lane = at(vo, 4 * lh) + 4u * (HD >= 32 ? lq : min(lq, HD - 1));
    float qr[NS], kr[NS], vr[16];
    const bool has = wave < ntiles;
    // the wave's first tile is loaded together with the queries
    auto load_kv = [&](int kt) __attribute__((always_inline)) {
        const int sk = 4 * kt * 32 * qc;
#pragma unroll
        for (int i = 0; i < NS / 4; ++i) {
            const float4 v = ld4s<kDev>(R.f, vk_lane + 16u * i, sk);
            kr[4 * i + 0] = v.x;
            kr[4 * i + 1] = v.y;
            kr[4 * i + 2] = v.z;
            kr[4 * i + 3] = v.w;
        }
        if (kt * 32 + 32 <= T) {
#pragma unroll
            for (int i = 0; i < 16; ++i)
                vr[i] = ld1s<kDev>(R.f, vv_lane, sk + 4 * (8 * (i >> 2) + (i & 3)) * qc);
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int vk = min(kt * 32 + 8 * (i >> 2) + 4 * lh + (i & 3), T - 1);
                vr[i] = ld1<kDev>(R.f, at(vo, vk) + 4u * (HD >= 32 ? lq : min(lq, HD - 1)));
            }
        }
    };
    if (has) {
#pragma unroll
        for (int i = 0; i < NS / 4; ++i) {
            const float4 v = ld4<kDev>(R.f, at(qo, min(qi, T - 1)) + 4u * (lh * NS + 4 * i));
            qr[4 * i + 0] = v.x;
            qr[4 * i + 1] = v.y;
            qr[4 * i + 2] = v.z;
            qr[4 * i + 3] = v.w;
        }
        load_kv(wave);
    }
    floatx16 o;
#pragma unroll
    for (int r = 0; r < 16; ++r) o[r] = 0.0f;
    const float sc = p.scale * 1.4426950408889634f;
    float m_run = -INFINITY, l_run = 0.0f;
    for (int kt = wave; kt < ntiles; kt += 8) {
        if (kt != wave) load_kv(kt);
        floatx16 sacc, sacc1;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            sacc[r] = 0.0f;
            sacc1[r] = 0.0f;
        }
#pragma unroll
        for (int i = 0; i < NS; i += 2) {
            sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(kr[i], qr[i], sacc, 0, 0, 0);
            if (i + 1 < NS)
                sacc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(kr[i + 1], qr[i + 1], sacc1, 0, 0, 0);
        }
        // (the matrix core and the VALU take turns on a SIMD, so the VALU work
        // between the products is kept short: the mask only on the tiles that
        // need it, no rescale of the zero sums on a wave's first tile, the
        // hardware exp2 (probabilities below 2^-126 flush to zero))
        const int k0 = kt * 32;
        float pv[16];
        float mloc = -INFINITY;
        if (k0 + 31 > q0 || k0 + 32 > T) {
            // the diagonal tile or the sequence's partial last one
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = k0 + 8 * (r >> 2) + 4 * lh + (r & 3);
                const float sv = (sacc[r] + sacc1[r]) * sc;
                pv[r] = (key <= qi && key < T) ? sv : -INFINITY;
                mloc = fmaxf(mloc, pv[r]);
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                pv[r] = (sacc[r] + sacc1[r]) * sc;
                mloc = fmaxf(mloc, pv[r]);
            }
        }
        mloc = pair32_max(mloc);
        if (kt == wave) {
            m_run = mloc;  // o and l are still zero
        } else {
            const bool need = mloc > m_run + 8.0f;
            if (__any(need)) {
                const float m_new = need ? mloc : m_run;
                const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
                l_run *= alpha;
#pragma unroll
                for (int r = 0; r < 16; ++r) o[r] *= alpha;
                m_run = m_new;
            }
        }
        float lsum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            pv[r] = __builtin_amdgcn_exp2f(pv[r] - m_run);
            lsum += pv[r];
        }
        l_run += pair32_sum(lsum);
#pragma unroll
        for (int i = 0; i < 16; ++i) o = __builtin_amdgcn_mfma_f32_32x32x2f32(vr[i], pv[i], o, 0, 0, 0);
    }
    if (lh == 0) {
        sm_m[wave * 32 + lq] = m_run;
        sm_l[wave * 32 + lq] = l_run;
    }
    __syncthreads();
    float mx = sm_m[lq];
#pragma unroll
    for (int w = 1; w < 8; ++w) mx = fmaxf(mx, sm_m[w * 32 + lq]);
    float Ls = 0.0f;
#pragma unroll
    for (int w = 0; w < 8; ++w) Ls += sm_l[w * 32 + lq] * __builtin_amdgcn_exp2f(sm_m[w * 32 + lq] - mx);
    const float f = __builtin_amdgcn_exp2f(m_run - mx) / Ls;  // 0 for a wave that saw no key
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int dd = 8 * (r >> 2) + 4 * lh + (r & 3);
        if (dd < HD) sm_o[wave * 32 * OS + lq * OS + dd] = o[r] * f;
    }
    __syncthreads();
    for (int idx = tid; idx < 32 * HD; idx += kNT) {
        const int jr = idx / HD, c = idx - jr * HD;
        float v = sm_o[jr * OS + c];
#pragma unroll
        for (int w = 1; w < 8; ++w) v += sm_o[w * 32 * OS + jr * OS + c];
        ctx[jr * (HD + 4) + c] = v;
    }
}

// The head's A operand for vocabulary block b (256 rows), K step stp: the
// wave's 32 vocabulary rows 256 b + 32 w + l % 32 (clamped to V - 1), k =
// 32 stp + 16 (l / 32) + j, from the tied embedding [V, d] (TIE) or lm_head [d, V].
// oob: the loads read past the descriptor (zeros, no memory access): the
// loop's last refill, whose values are never used, costs no round trip that
// the task's final wait would sit out.
template <bool TIE>
__device__ __forceinline__ void head_load_a(int tid, const FusedP &p, const Res &R, int b, int stp,
                                            int wave, float *a, bool oob = false) {
    const int lane = tid & 63, lr = lane & 31, lk = lane >> 5;
    const int v = min(256 * b + 32 * wave + lr, p.V - 1);
    if constexpr (TIE) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 ev = ld4s<0>(R.w, oob ? kOOB : 4u * (uint32_t)v * (uint32_t)p.d + 64u * lk + 16u * i, 128 * stp);
            a[4 * i + 0] = ev.x;
            a[4 * i + 1] = ev.y;
            a[4 * i + 2] = ev.z;
            a[4 * i + 3] = ev.w;
        }
    } else {
        const uint32_t vh = oob ? kOOB : 4u * ((uint32_t)(p.o_head + v) + 16u * lk * (uint32_t)p.V);
#pragma unroll
        for (int jj = 0; jj < 16; ++jj) a[jj] = ld1s<0>(R.w, vh, 4 * (32 * stp + jj) * p.V);
    }
}

template <int HD>
__global__ __launch_bounds__(kNT, 1) void forward_team_kernel(FusedP p) {
    __shared__ __attribute__((aligned(16))) float lds[kLdsFloats];
    __shared__ __attribute__((aligned(16))) float s_nw[256];        // norm weights of the task
    __shared__ __attribute__((aligned(16))) float s_xs[kRowStage];  // normalised rows
    __shared__ float s_cs[32 * 16], s_sn[32 * 16];                 // RoPE rows of the block
    __shared__ float s_inv[32];
    __shared__ int s_ok, s_last, s_x, s_slot;
    const int tid0 = threadIdx.x;
    const int team = gridDim.x >> 3;
    int32_t *ctl = reinterpret_cast<int32_t *>(p.f + p.o_ctl);
    if (p.stamps && tid0 == 0) p.stamps[2 * blockIdx.x] = __builtin_amdgcn_s_memrealtime();

    Res R;
    R.w = rsrc(p.w, p.w_bytes);
    R.f = rsrc(p.f, p.f_bytes);
    R.i = rsrc(p.ids, p.i_bytes);

    // The XCD this workgroup runs on and its slot in that XCD's team (the
    // dispatcher deals workgroups round-robin over the XCDs, but not always
    // from XCD 0: as a graph node the first one lands elsewhere).
    // rr: the context's probe found the dispatch round-robin over the XCDs
    // with one offset per launch (workgroup b on XCD (b + o) % 8), so the
    // workgroups of an XCD are b = c, c + 8, ... and b / 8 is a slot of its
    // own, with no atomic (32 returning atomics on one counter per XCD put
    // 1.5-4.5 us before the first task). Each workgroup records its offset
    // (xcc - b) % 8 in a mask; the last one out flags (error bit 2) a launch
    // whose workgroups saw more than one. Otherwise: a returning atomic per XCD.
    if (tid0 == 0) {
        const int xr = xcc_id();
        int sl = team;
        if (xr < 8) {
            if (p.rr) {
                sl = (int)(blockIdx.x >> 3);
                __hip_atomic_fetch_or(ctl + 1, 1 << ((xr - (int)blockIdx.x) & 7), __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
            } else {
                sl = __hip_atomic_fetch_add(ctl + 1 + xr, 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        s_x = xr & 7;
        s_slot = sl;
        if (sl >= team) __hip_atomic_fetch_or(p.err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    const int x = s_x, slot = s_slot;
    const bool on_xcd = slot < team;

    // this XCD's sequences: s = x + 8 j
    const int S = x < p.B ? (p.B - x + 7) >> 3 : 0;
    const int nrb = p.nrb;
    const int nQ = S * nrb * p.nq_c, nA = S * p.H * nrb, nG = S * nrb * p.ng_c,
              nD = S * nrb * p.nd_c;
    const int LT = nQ + nA + nG + nD;
    const int nH = S * nrb * p.nh_t;
    const int total = on_xcd ? p.L * LT + nH : 0;
    const int d = p.d, T = p.T;
    constexpr float kLog2e = 1.4426950408889634f;

    for (int t = slot; t < total; t += team) {
        // The thread index through an empty asm: lane-dependent addresses are
        // then formed inside each task instead of being hoisted out of the
        // loop and held in registers for the whole kernel.
        int tid = threadIdx.x;
        asm volatile("" : "+v"(tid));
        const int lane = tid & 63, lr = lane & 31, lk = lane >> 5;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        // decode: stage instance si (layer l, stage st), sequence slot j, row block q, column block c
        int l = 0, st, j = 0, q = 0, c = 0, hh = 0;
        int r = t;
        if (r < p.L * LT) {
            l = r / LT;
            r -= l * LT;
            if (r < nQ) {
                st = ST_Q;
                c = r % p.nq_c;
                r /= p.nq_c;
                j = r % S;
                q = r / S;
            } else if ((r -= nQ) < nA) {
                st = ST_A;  // longest query blocks first
                hh = r % p.H;
                r /= p.H;
                j = r % S;
                q = nrb - 1 - r / S;
            } else if ((r -= nA) < nG) {
                st = ST_G;
                c = r % p.ng_c;
                r /= p.ng_c;
                j = r % S;
                q = r / S;
            } else {
                r -= nG;
                st = ST_D;
                c = r % p.nd_c;
                r /= p.nd_c;
                j = r % S;
                q = r / S;
            }
        } else {
            r -= p.L * LT;
            st = 5;  // head (and, by the last of a row block's, the combine)
            c = r % p.nh_t;
            r /= p.nh_t;
            j = r % S;
            q = r / S;
        }
        const int si = st < 5 ? l * 5 + st : p.L * 5 + (st - 5);
        const int s = x + 8 * j;                       // the sequence
        const int rows = min(32, T - 32 * q);          // valid rows of the block
        const int row0 = s * T + 32 * q;               // its first row
        const int ra = row0 + min(lr, rows - 1);       // this lane's (clamped) row
        const bool row_ok = lr < rows;
        const int wb = p.blk0 + l * p.blk;             // this layer's weights
        const uint32_t qkv_off = p.o_qkv + (uint32_t)l * (uint32_t)p.n * (uint32_t)p.qc;
        const bool isq = st == ST_Q;
        const int ncol = isq ? p.qc : 2 * p.ff_pad;    // Q / G output columns
        const int qg_wo = isq ? wb + p.o_wqkv : wb + p.o_wgu;
        const int od_wo = wb + p.o_wd, od_k = p.ff;  // down
        const int hns = (d + 31) >> 5;                 // head: K steps per vocabulary block
        const int hb0 = c * p.hb, hb1 = min(p.nh_c, hb0 + p.hb);  // its 256-row blocks
        int tg = 0;                                    // head: the lane's row's target

        // ---- what does not depend on earlier tasks, issued before the wait
        GemmPre gp;  // GEMM tasks: B operands; the head: its vocabulary rows (2 steps)
        if (st == ST_Q || st == ST_G) {
            if (isq)
                gemm_fetch_b<4>(tid, R, qg_wo, ncol, 128 * c, ncol, d, gp);
            else
                gemm_fetch_b<8>(tid, R, qg_wo, ncol, 256 * c, ncol, d, gp);
            const int nwo = isq ? wb : wb + p.o_mn;
            for (int i = tid; i < d; i += kNT) s_nw[i] = ld1<0>(R.w, 4u * (uint32_t)(nwo + i));
            if (isq) {
                constexpr int half = HD / 2;
                for (int i = tid; i < 32 * half; i += kNT) {
                    const int rr = i / half, cc = i - rr * half;
                    const uint32_t ti = 4u * (uint32_t)((32 * q + rr) * half + cc);
                    s_cs[i] = ld1<0>(R.f, 4u * p.o_cos + ti);
                    s_sn[i] = ld1<0>(R.f, 4u * p.o_sin + ti);
                }
            }
        } else if (st == ST_A) {
            // the head's HD rows of Wo for this wave's 32 output columns (waves
            // below d / 32): gp.v[j] = Wo[HD hh + 16 (l/32) + j][32 w + l%32]
            if (32 * wave < d) {
                const uint32_t vb = 4u * ((uint32_t)(wb + p.o_wo) + (uint32_t)(hh * HD + 16 * lk) * (uint32_t)d +
                                          32u * wave + lr);
#pragma unroll
                for (int jj = 0; jj < 16; ++jj) gp.v[jj] = ld1s<0>(R.w, vb, 4 * jj * d);
            }
        } else if (st == ST_D) {
            gemm_fetch_b<1>(tid, R, od_wo, d, 32 * c, d, od_k, gp);
        } else if (st == 5) {
            for (int i = tid; i < d; i += kNT) s_nw[i] = ld1<0>(R.w, 4u * (uint32_t)(p.o_fn + i));
            tg = ldi<0>(R.i, 4u * (p.tgt_off + (uint32_t)ra));
            // the first two K steps of the first block
#pragma unroll
            for (int f = 0; f < 2; ++f)
                if (f < hns) {
                    if (p.tie)
                        head_load_a<true>(tid, p, R, hb0, f, wave, gp.v + 16 * f);
                    else
                        head_load_a<false>(tid, p, R, hb0, f, wave, gp.v + 16 * f);
                }
        }

        // ---- dependencies
        if (wave == 0) {
            bool ok = true;
            auto wait = [&](int dsi, int q_first, int count, int target) {
                ok = ok && wave_wait(ctl, cnt_index(p, x, dsi, j, q_first), count, target, p.err,
                                     p.ctl_ints, lane);
            };
            if (st == ST_Q && l > 0) wait((l - 1) * 5 + ST_D, q, 1, p.nd_c);
            if (st == ST_A) wait(l * 5 + ST_Q, 0, q + 1, p.nq_c);
            if (st == ST_G) wait(l * 5 + ST_A, q, 1, p.H);  // every head's O partial
            if (st == ST_D) wait(l * 5 + ST_G, q, 1, p.ng_c);
            if (st == 5) wait((p.L - 1) * 5 + ST_D, q, 1, p.nd_c);
            if (lane == 0) s_ok = ok;
        }
        __syncthreads();
        if (!s_ok) break;

        if (st == ST_Q || st == ST_G) {
            // the rows normalised into LDS; Q: RoPE epilogue into this layer's qkv
            // (128-column blocks, two K groups); G: SwiGLU into h (256 columns)
            if (isq && l == 0)  // the embedding rows; column block 0 also stores them as x
                stage_norm_rows<1>(tid, p, R, row0, rows, s_nw, s_xs, c == 0);
            else if (isq)
                stage_norm_rows<0>(tid, p, R, row0, rows, s_nw, s_xs, false);
            else  // x after the O projection; column block 0 stores it as x2
                stage_norm_rows<2>(tid, p, R, row0, rows, s_nw, s_xs, c == 0);
            __syncthreads();
            floatx16 acc;
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
            if (isq) {
                const int n0 = 128 * c;
                gemm_run_lds<4>(tid, R, s_xs, gp, qg_wo, ncol, n0, ncol, d, acc);
                share_block<4>(tid, lds, acc);
                constexpr int half = HD / 2;
                const int ct = wave & 3, kg = wave >> 2;
                const int col = n0 + 32 * ct + lr;
                // the tile's 32 columns hold whole heads (HD divides 32); the
                // rotation applies to q and k, which fill whole tiles
                const bool rot = n0 + 32 * ct < d + p.kvw;
                const int pc = col % HD, pcm = pc < half ? pc : pc - half;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int rl = row_local(kg + 2 * i, lk);
                    float v = acc[i];
                    const float other = HD == 32 ? lane_xor16(v, lane) : lane_xor8(v);
                    if (rot) {
                        const float cs = s_cs[rl * half + pcm], sn = s_sn[rl * half + pcm];
                        v = pc < half ? v * cs - other * sn : v * cs + other * sn;
                    }
                    if (rl < rows && col < ncol)
                        st1(R.f, 4u * (qkv_off + (uint32_t)(row0 + rl) * (uint32_t)p.qc + col), v);
                }
            } else {
                const int n0 = 256 * c;
                gemm_run_lds<8>(tid, R, s_xs, gp, qg_wo, ncol, n0, ncol, d, acc);
                // the pair (gate, up) of output f sits in lanes 2f, 2f + 1: even
                // lanes finish registers 0-7, odd lanes registers 8-15
                const int col = n0 + 32 * wave + lr, f = col >> 1;
                const bool odd = lr & 1;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float lo = acc[e], hi = acc[e + 8];
                    const float lo_x = lane_xor1(lo), hi_x = lane_xor1(hi);
                    const float g = odd ? hi_x : lo, u = odd ? hi : lo_x;
                    const int rl = row_local(odd ? e + 8 : e, lk);
                    if (rl < rows && f < p.ff)
                        st1(R.f, 4u * (p.o_h + (uint32_t)(row0 + rl) * (uint32_t)p.ff + f),
                            __fmul_rn(silu_f(g), u));
                }
            }
        } else if (st == ST_D) {
            // x = x2 + h . Wd over one 32-column block, K split over the 8 waves;
            // wave w adds the residual to registers w and w + 8
            const int col = 32 * c + lr;
            float res[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int rl = row_local(wave + 8 * i, lk);
                res[i] = ld1<kDev>(R.f, rl < rows && col < d
                                            ? 4u * (p.o_x2 + (uint32_t)(row0 + rl) * (uint32_t)d + col)
                                            : kOOB);
            }
            floatx16 acc;
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
            float ss = 0.0f;
            gemm_run<1, 0, false>(tid, p, R, p.o_h, p.ff, ra, false, gp, od_wo, d, 32 * c, d, p.ff,
                                  nullptr, acc, ss);
            share_block<1>(tid, lds, acc);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int rl = row_local(wave + 8 * i, lk);
                if (rl < rows && col < d)
                    st1(R.f, 4u * (p.o_x + (uint32_t)(row0 + rl) * (uint32_t)d + col),
                        __fadd_rn(res[i], acc[i]));
            }
        } else if (st == ST_A) {
            // attention, then this head's share of the O projection, ctx_h .
            // Wo[head rows] (32 x d, K = HD), as a partial; the gate/up tasks of
            // the row block add the partials in head order to the residual
            float *ctx = s_xs;  // [32][HD + 4]
            attention_task<HD>(tid, p, R, lds, qkv_off, s, hh, q, ctx);
            __syncthreads();
            if (32 * wave < d) {
                floatx16 acc;
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
#pragma unroll
                for (int jj = 0; jj < 16; ++jj) {
                    const int k = 16 * lk + jj;
                    const float a = k < HD ? ctx[lr * (HD + 4) + k] : 0.0f;
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, k < HD ? gp.v[jj] : 0.0f, acc, 0, 0, 0);
                }
                const int col = 32 * wave + lr;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int rl = row_local(e, lk);
                    if (rl < rows)
                        st1(R.f, 4u * (p.o_op + ((uint32_t)(row0 + rl) * (uint32_t)p.H + hh) * (uint32_t)d + col),
                            acc[e]);
                }
            }
        } else {
            // logits^T of 32 vocabulary rows per wave and 256-row block against the
            // block's normalised rows (staged in LDS): lane l holds row l % 32,
            // register e vocabulary row 256 b + 32 w + row_local(e). Per lane a
            // running (max, sum of exp) over the task's blocks, then merged over
            // the waves into one pair per row and task.
            stage_norm_rows<0>(tid, p, R, row0, rows, s_nw, s_xs, false);
            __syncthreads();
            const float *xr = s_xs + lr * (d + 4) + 16 * lk;
            floatx16 acc;
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
            float m_run = -INFINITY, s_run = 0.0f;
            // K step stp: 16 MFMAs in four groups of 4, each group's four x
            // values one LDS read, issued a group ahead (x0 holds the step's
            // first group on entry and step nstp's first group on return), so
            // no group waits for its read
            auto head_step = [&](int stp, int nstp, const float *a, float4 &x0) __attribute__((always_inline)) {
                float4 cur = x0;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 nxt = *reinterpret_cast<const float4 *>(xr + (q < 3 ? 32 * stp + 4 * (q + 1) : 32 * nstp));
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[4 * q + 0], cur.x, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[4 * q + 1], cur.y, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[4 * q + 2], cur.z, acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[4 * q + 3], cur.w, acc, 0, 0, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
                    cur = nxt;
                }
                x0 = cur;
            };
            float4 x0 = *reinterpret_cast<const float4 *>(xr);
            // block b's logits complete: the target logit out, the block's (max,
            // sum of exp) over the wave's 32 rows into the running pair
            // (the matrix core and the VALU take turns on a SIMD: every VALU
            // instruction here adds its cycles to the loop's)
            auto head_block = [&](int b) __attribute__((always_inline)) {
                const int v0 = 256 * b + 32 * wave;
                // register e holds vocabulary row v0 + 4 (l / 32) + re(e)
                auto re = [](int e) { return 8 * (e >> 2) + (e & 3); };
                // (both tests below are wave-uniform: most blocks skip them)
                // the target logit, where some lane's target is in these 32 rows
                if (__any((unsigned)(tg - v0) < 32u)) {
                    const int dt = tg - v0 - 4 * lk;
                    float zt = 0.0f;
                    bool hit = false;
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        zt = dt == re(e) ? acc[e] : zt;
                        hit = hit || dt == re(e);
                    }
                    if (hit && row_ok) st1(R.f, 4u * (p.o_zt + (uint32_t)ra), zt);
                }
                // rows past the vocabulary, where it ends inside these 32
                if (v0 + 32 > p.V) {
                    const int lim = p.V - v0 - 4 * lk;
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        if (re(e) >= lim) acc[e] = -INFINITY;
                }
                float mx = -INFINITY;
#pragma unroll
                for (int e = 0; e < 16; ++e) mx = fmaxf(mx, acc[e]);
                mx = pair32_max(mx);
                float sum = 0.0f;
                if (mx != -INFINITY) {
                    // exp2((z - max) log2 e) as one FMA per logit
                    const float nml = -mx * kLog2e;
#pragma unroll
                    for (int e = 0; e < 16; ++e) sum += __builtin_amdgcn_exp2f(__builtin_fmaf(acc[e], kLog2e, nml));
                }
                lse_merge(m_run, s_run, mx, pair32_sum(sum));
            };
            // one loop per head layout: with the layout chosen inside the
            // loop, the compiler's wait for a register set covered the other
            // set's newer loads as well (each set then waited out its loads)
            auto head_loop = [&](auto tie_c) __attribute__((always_inline)) {
            constexpr bool TIE = decltype(tie_c)::value;
            if ((hns & 1) == 0) {
                // steps in pairs: register set 0 holds the even step, set 1 the odd
                // one; each set is refilled two steps ahead (across blocks)
#pragma unroll 1
                for (int b = hb0; b < hb1; ++b) {
                    // (the pair as a lambda: the register assignment the
                    // compiler then chooses runs the head task 1.5-2 us faster
                    // than the same loop written inline, same box, 3 rounds)
                    auto pair = [&](int stp) __attribute__((always_inline)) {
                        head_step(stp, stp + 1, gp.v, x0);
                        // every pair issues both sets' loads: the task's last
                        // pair reloads its own rows (in range, never used), so
                        // each path through the loop has the same loads in
                        // flight and the compiler waits for a set only where
                        // that set is used, two steps after its loads
                        const bool wrap = stp + 2 >= hns, last = wrap && b + 1 >= hb1;
                        const int nb = wrap && !last ? b + 1 : b;
                        const int ns = wrap ? (last ? stp : 0) : stp + 2;
                        // (scheduling barriers keep the loads where they are
                        // written: the scheduler would sink them to the end)
                        __builtin_amdgcn_sched_barrier(0);
                        head_load_a<TIE>(tid, p, R, nb, ns, wave, gp.v, last);
                        __builtin_amdgcn_sched_barrier(0);
                        head_step(stp + 1, stp + 2 < hns ? stp + 2 : 0, gp.v + 16, x0);
                        __builtin_amdgcn_sched_barrier(0);
                        head_load_a<TIE>(tid, p, R, nb, ns + 1, wave, gp.v + 16, last);
                        __builtin_amdgcn_sched_barrier(0);
                    };
#pragma unroll 1
                    for (int stp = 0; stp < hns; stp += 2) pair(stp);
                    head_block(b);
#pragma unroll
                    for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
                }
            } else {
#pragma unroll 1
                for (int b = hb0; b < hb1; ++b) {
                    auto one = [&](int stp) __attribute__((always_inline)) {
                        if (b != hb0 || stp >= 2) head_load_a<TIE>(tid, p, R, b, stp, wave, gp.v);
                        head_step(stp, stp + 1 < hns ? stp + 1 : 0, gp.v + (b == hb0 && stp == 1 ? 16 : 0), x0);
                    };
#pragma unroll 1
                    for (int stp = 0; stp < hns; ++stp) one(stp);
                    head_block(b);
#pragma unroll
                    for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
                }
            }
            };
            if (p.tie)
                head_loop(std::true_type{});
            else
                head_loop(std::false_type{});
            float *sm_m = lds, *sm_s = lds + 8 * 32;
            if (lk == 0) {
                sm_m[wave * 32 + lr] = m_run;
                sm_s[wave * 32 + lr] = s_run;
            }
            __syncthreads();
            if (tid < 32 && tid < rows) {
                float m = sm_m[tid], sm = sm_s[tid];
#pragma unroll
                for (int w = 1; w < 8; ++w) lse_merge(m, sm, sm_m[w * 32 + tid], sm_s[w * 32 + tid]);
                st2(R.f, 4u * p.o_part + 8u * ((uint32_t)(row0 + tid) * (uint32_t)p.nh_t + c), make_float2(m, sm));
            }
            // the last head task of the row block forms its rows' losses
            // (max + ln(sum) - z[target], ops_reduce.rs:236-259) and their f64 sum
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (tid == 0)
                s_last = __hip_atomic_fetch_add(ctl + cnt_index(p, x, si, j, q), 1, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT) == p.nh_t - 1;
            __syncthreads();
            if (s_last && wave == 0) {
                double dsum = 0.0;
                if (lane < rows) {
                    const uint32_t row = (uint32_t)(row0 + lane);
                    const float zt = ld1<kDev>(R.f, 4u * (p.o_zt + row));
                    float m = -INFINITY, sm = 0.0f;
                    for (int c0 = 0; c0 < p.nh_t; c0 += 4) {
                        float2 pr[4];
#pragma unroll
                        for (int u = 0; u < 4; ++u)
                            pr[u] = c0 + u < p.nh_t
                                        ? ld2<kDev>(R.f, 4u * p.o_part + 8u * (row * (uint32_t)p.nh_t + c0 + u))
                                        : make_float2(-INFINITY, 0.0f);
#pragma unroll
                        for (int u = 0; u < 4; ++u) lse_merge(m, sm, pr[u].x, pr[u].y);
                    }
                    const float loss = __fsub_rn(__fadd_rn(m, logf(sm)), zt);
                    st1(R.f, 4u * (p.o_rl + row), loss);
                    dsum = (double)loss;
                }
#pragma unroll
                for (int off = 32; off > 0; off >>= 1) dsum += __shfl_xor(dsum, off, 64);
                if (lane == 0) {
                    __builtin_amdgcn_raw_buffer_store_b64(
                        __builtin_bit_cast(u32x2, dsum), R.f,
                        4u * p.o_p64 + 8u * ((uint32_t)s * (uint32_t)nrb + q), 0, kDev);
                    __builtin_amdgcn_s_waitcnt(0);
                    __hip_atomic_fetch_add(ctl + cnt_index(p, x, p.L * 5 + 1, j, q), 1,
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            __syncthreads();
            continue;  // published above
        }
        // publish: the task's stores are complete in L2, then its counter moves
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            const int ci = cnt_index(p, x, si, j, q);
            if ((uint32_t)ci < p.ctl_ints)
                __hip_atomic_fetch_add(ctl + ci, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }

    // The last workgroup out forms the mean and resets the counters.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid0 == 0)
        s_last = __hip_atomic_fetch_add(ctl, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 (int)gridDim.x - 1;
    __syncthreads();
    if (!s_last) {
        if (p.stamps && tid0 == 0) p.stamps[2 * blockIdx.x + 1] = __builtin_amdgcn_s_memrealtime();
        return;
    }
    // every row block of every sequence combined? Each thread checks row
    // blocks i = tid, tid + 512, ... and parks their f64 sums in LDS; wave 0
    // then adds them in a fixed order.
    double *sm_p = reinterpret_cast<double *>(s_xs);  // B * nrb <= kLossSlots (host-checked)
    const int nblk = p.B * nrb;
    // rr: every workgroup's offset recorded before it counted itself out
    // (the word read first, so its round trip overlaps the loads below)
    const int rr_mask = p.rr && tid0 == 0 ? __hip_atomic_load(ctl + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 1;
    int missing = 0;
    for (int i = tid0; i < nblk; i += kNT) {
        const int ss_ = i / nrb, qq = i - ss_ * nrb;
        missing += __hip_atomic_load(ctl + cnt_index(p, ss_ & 7, p.L * 5 + 1, ss_ >> 3, qq),
                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 1;
        sm_p[i] = __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(R.f, 4u * p.o_p64 + 8u * i, 0, kDev));
    }
    if (__any(missing != 0) && (tid0 & 63) == 0)
        __hip_atomic_fetch_or(p.err, 4, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (__builtin_popcount(rr_mask) != 1)
        __hip_atomic_fetch_or(p.err, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (tid0 < 64) {
        // fixed order: lane l adds blocks l, l + 64, ... in turn, then the 64
        // lane sums meet in a fixed tree
        double sum = 0.0;
        for (int i = tid0; i < nblk; i += 64) sum += sm_p[i];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
        if (tid0 == 0) *p.loss = (float)(sum / (double)p.n);
    }
    __syncthreads();
    for (int i = tid0; i < (int)p.ctl_ints; i += kNT) st1<kDev>(R.f, 4u * (p.o_ctl + i), 0.0f);
    if (p.stamps) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid0 == 0) p.stamps[2 * blockIdx.x + 1] = __builtin_amdgcn_s_memrealtime();
    }
}

// One single-wave workgroup per CU, counted per XCD; each workgroup's XCD
// recorded by its index.
__global__ __launch_bounds__(64) void xcd_probe_kernel(int *counts, int *order) {
    if (threadIdx.x == 0) {
        const int x = xcc_id();
        __hip_atomic_fetch_add(counts + (x & 15), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        order[blockIdx.x] = x;
    }
}

}  // namespace

// ---- host side -------------------------------------------------------------

bool probe_xcd_teams(Context &ctx) {
    ctx.xcd_rr = false;
    if (ctx.cu_count < 8 || ctx.cu_count % 8 != 0) return false;
    const int g = ctx.cu_count;
    int *counts = nullptr;
    std::vector<int> order((size_t)g);
    int h[16] = {};
    bool ok = hipMalloc(&counts, sizeof(h) + (size_t)g * 4) == hipSuccess;
    // three launches: equal XCD shares in each; the round-robin order (block b
    // on XCD (b + o) % 8, o fixed within a launch) in every one of them
    bool rr = true;
    for (int run = 0; run < 3 && ok; ++run) {
        ok = hipMemset(counts, 0, sizeof(h) + (size_t)g * 4) == hipSuccess;
        if (!ok) break;
        hipLaunchKernelGGL(xcd_probe_kernel, dim3((unsigned)g), dim3(64), 0, nullptr, counts,
                           counts + 16);
        ok = hipGetLastError() == hipSuccess && hipDeviceSynchronize() == hipSuccess &&
             hipMemcpy(h, counts, sizeof(h), hipMemcpyDeviceToHost) == hipSuccess &&
             hipMemcpy(order.data(), counts + 16, (size_t)g * 4, hipMemcpyDeviceToHost) == hipSuccess;
        for (int x = 0; x < 16 && ok; ++x) ok = h[x] == (x < 8 ? g / 8 : 0);
        const int o = (order[0] & 7);
        for (int b = 0; b < g && ok; ++b) rr = rr && order[b] < 8 && order[b] == ((b + o) & 7);
    }
    if (counts) (void)hipFree(counts);
    ctx.xcd_rr = ok && rr;
    return ok;
}

bool fused_forward_fits(const Context &ctx, const FusedShape &s) {
    if (!ctx.xcd_teams || ctx.cu_count < 8 || ctx.cu_count % 8 != 0) return false;
    if (s.heads <= 0 || s.kv_heads <= 0 || s.heads % s.kv_heads != 0) return false;
    const int64_t hd = s.d / s.heads;
    if (hd * s.heads != s.d || (hd != 16 && hd != 32)) return false;
    if (s.d % 32 != 0 || s.d > 256 || s.ff % 4 != 0 || s.ff <= 0) return false;
    if (s.batch < 1 || s.seq < 1 || s.layers < 1 || s.vocab < 1) return false;
    const int64_t n = s.batch * s.seq;
    const int64_t qc = s.d + 2 * s.kv_heads * hd;
    // every buffer addressable with 32-bit byte offsets
    const int64_t lim = (int64_t)1 << 30;
    if (s.weight_floats * 4 >= lim || fused_layout(s).floats * 4 >= lim || n * qc >= lim)
        return false;
    // small work only: one launch with a few hundred tasks per XCD
    if (n > 16384) return false;
    // the last workgroup parks one f64 sum per (sequence, 32-row block) in
    // its LDS row stage (32 x 260 floats) before adding them in order
    if (s.batch * ((s.seq + 31) / 32) > kLossSlots) return false;
    return true;
}

FusedLayout fused_layout(const FusedShape &s) {
    FusedLayout f;
    const int64_t hd = s.d / s.heads, n = s.batch * s.seq;
    auto al = [](int64_t v) { return (v + 63) / 64 * 64; };
    f.qc = s.d + 2 * s.kv_heads * hd;
    f.nrb = (s.seq + 31) / 32;
    f.smax = (s.batch + 7) / 8;
    f.nsi = 5 * s.layers + 2;
    f.ctl_ints = 64 + 8 * f.nsi * f.smax * f.nrb;
    f.tab_floats = s.max_seq * (hd / 2);
    // every region is fenced by a guard band of kBand floats on each side
    int64_t o = FusedLayout::kBand;
    f.bands[f.nbands++] = 0;
    auto take = [&](int64_t floats) {
        const int64_t at = o;
        o += al(floats);
        f.bands[f.nbands++] = o;
        o += FusedLayout::kBand;
        return at;
    };
    f.o_x = take(n * s.d);
    f.o_op = take(n * s.heads * s.d);
    f.o_x2 = take(n * s.d);
    f.o_h = take(n * s.ff);
    f.o_qkv = take(s.layers * n * f.qc);
    f.o_part = take(n * ((s.vocab + 255) / 256) * 2);
    f.o_zt = take(n);
    f.o_rl = take(n);
    f.o_p64 = take(2 * s.batch * f.nrb);
    f.o_ctl = take(f.ctl_ints);
    f.o_err = take(1);
    f.o_cos = take(f.tab_floats);
    f.o_sin = take(f.tab_floats);
    f.floats = o;
    return f;
}

void launch_fused_forward(Context &ctx, const FusedArgs &a) {
    const FusedShape &s = a.shape;
    const FusedLayout f = fused_layout(s);
    const int64_t n = s.batch * s.seq, hd = s.d / s.heads;
    if (a.tgt < a.ids || a.tgt - a.ids > (int64_t)1 << 28)
        fail(MMH_ERR_ARGUMENT, "fused forward: the targets must follow the ids");
    FusedP p{};
    p.w = a.w;
    p.f = a.arena;
    p.ids = a.ids;
    p.loss = a.loss;
    p.err = reinterpret_cast<int32_t *>(a.arena + f.o_err);
    p.stamps = a.stamps;
    p.rr = ctx.xcd_rr ? 1 : 0;
    p.w_bytes = (uint32_t)(s.weight_floats * 4);
    p.f_bytes = (uint32_t)(f.floats * 4);
    p.tgt_off = (uint32_t)(a.tgt - a.ids);
    p.i_bytes = (uint32_t)((p.tgt_off + n) * 4);
    p.o_x = (uint32_t)f.o_x;
    p.o_op = (uint32_t)f.o_op;
    p.o_x2 = (uint32_t)f.o_x2;
    p.o_h = (uint32_t)f.o_h;
    p.o_qkv = (uint32_t)f.o_qkv;
    p.o_part = (uint32_t)f.o_part;
    p.o_zt = (uint32_t)f.o_zt;
    p.o_rl = (uint32_t)f.o_rl;
    p.o_p64 = (uint32_t)f.o_p64;
    p.o_ctl = (uint32_t)f.o_ctl;
    p.o_err = (uint32_t)f.o_err;
    p.o_cos = (uint32_t)f.o_cos;
    p.o_sin = (uint32_t)f.o_sin;
    p.ctl_ints = (uint32_t)f.ctl_ints;
    p.B = (int)s.batch;
    p.T = (int)s.seq;
    p.d = (int)s.d;
    p.H = (int)s.heads;
    p.Hkv = (int)s.kv_heads;
    p.ff = (int)s.ff;
    p.ff_pad = (int)s.ff_pad;
    p.V = (int)s.vocab;
    p.L = (int)s.layers;
    p.tie = s.tie ? 1 : 0;
    p.qc = (int)f.qc;
    p.kvw = (int)(s.kv_heads * hd);
    p.n = (int)n;
    p.eps = s.eps;
    p.scale = 1.0f / sqrtf((float)hd);  // attention.rs:82
    p.blk0 = (int)a.off_block0;
    p.blk = (int)a.block_floats;
    p.o_wqkv = (int)s.d;
    p.o_wo = (int)(s.d + s.d * f.qc);
    p.o_mn = (int)(s.d + s.d * f.qc + s.d * s.d);
    p.o_wgu = p.o_mn + (int)s.d;
    p.o_wd = p.o_wgu + (int)(2 * s.d * s.ff_pad);
    p.o_fn = (int)a.off_final_norm;
    p.o_head = (int)(a.off_final_norm + s.d);
    p.nrb = (int)f.nrb;
    p.smax = (int)f.smax;
    p.nsi = (int)f.nsi;
    p.nq_c = (int)((f.qc + 127) / 128);

    p.ng_c = (int)((2 * s.ff_pad + 255) / 256);
    p.nd_c = (int)((s.d + 31) / 32);
    p.nh_c = (int)((s.vocab + 255) / 256);
    // head tasks: about one per team workgroup over the row blocks of an XCD
    const int team = ctx.cu_count / 8;
    p.hb = (int)std::max<int64_t>(1, (p.nh_c * f.nrb * f.smax + team - 1) / team);
    p.nh_t = (p.nh_c + p.hb - 1) / p.hb;
    const dim3 grid((unsigned)ctx.cu_count);
    if (hd == 32)
        hipLaunchKernelGGL((forward_team_kernel<32>), grid, dim3(kNT), 0, ctx.stream, p);
    else
        hipLaunchKernelGGL((forward_team_kernel<16>), grid, dim3(kNT), 0, ctx.stream, p);
    check_hip(hipGetLastError(), "fused forward launch");
}

}  // namespace mmh
