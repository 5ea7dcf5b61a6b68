// Fused causal attention on CDNA4 matrix cores (fp32 MFMA 32x32x2), replacing
// the reference's materialised path (midman-nn/src/attention.rs:79-101,146-170):
// repeat_interleave of K/V, Q.K^T, scale, additive -1e9 mask, softmax, P.V.
//
// A 512-thread workgroup (8 wave64s) owns two 128-row query blocks of one
// (batch, head), paired so that every workgroup carries the same causal work:
// block nqb-1-z (the longest rows) on waves 0-3 and block z on waves 4-7, each
// wave owning 32 rows. The workgroup walks 32-key tiles of K and V up to the
// long block's last diagonal; the short block's keys are a prefix of those,
// so every tile is loaded once with float4 loads into registers, written to a
// double-buffered LDS stage, and shared by all eight waves; the next tile's
// loads are in flight while the current one is used. A SIMD then runs one wave
// of each block, nqb+1 blocks' worth of tiles in every workgroup, where
// unpaired blocks would leave the CUs that drew two long blocks working while
// the rest idle. (attn_fwd16_kernel below takes heads of 64 and 128 with 16
// rows per wave; attn_fwd_split_kernel covers small grids.)
// Each wave keeps an online softmax for its rows, so no [T,T] tensor exists.
//
// The products are computed transposed so that every per-query quantity lives
// in the lane that owns the query:
//   S^T[key][q] = K_tile . Q^T   (A = K from LDS, B = Q from registers)
//   O^T[d][q]  += V^T . P^T      (A = V from LDS, B = P straight from the S^T
//                                 accumulators, no LDS round trip)
// With the MFMA layout (lane l: column l%32; register r: row
// 8*(r/4) + 4*(l/32) + r%4), query q = l%32 is fixed per lane in both
// products, so a row's max and sum need one exchange between lanes l and l^32
// and the rescale of O is a per-lane scalar. In S^T the lanes 0-31 feed head
// dims [0, hd/2) and lanes 32-63 feed [hd/2, hd), so each lane reads its Q
// operands as one contiguous run.
//
// RoPE (rope.rs:28-32) is applied once, in place, to the q and k rows before
// the attention kernel (rope_strided below), with separately rounded
// multiplies and adds, so rotated values equal the reference's bit for bit.
// The score scale is applied after the dot product as attention.rs:83 does.
// Keys above the diagonal are skipped: the reference's -1e9 mask gives them
// exp(.) == 0 exactly. Query head j reads kv head j / (H/Hkv)
// (repeat_interleave, ops_shape.rs:192-200).
#include "mmh_internal.h"

namespace mmh {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

struct AttnP {
    const float *q, *k, *v;
    float *out;
    float *lse;
    int64_t sqb, sqh, sqt, skb, skh, skt, svb, svh, svt, sob, soh, sot;
    int h, hkv, t, nqb;
    float scale;
};

template <int HD>
__global__ __launch_bounds__(512) void attn_fwd_kernel(AttnP p) {
    constexpr int NT = 512;                  // threads
    constexpr int QB = 128;                  // query rows per block (4 waves)
    constexpr int NS = HD / 2;               // S^T k-steps (lanes 32-63 take dims NS..HD-1)
    constexpr int NDB = (HD + 31) / 32;      // O^T row blocks; block db row i is dim NDB*i+db
    constexpr int KS = HD + 4;               // K row stride: 16-byte aligned rows
    constexpr int OS = HD + 1;               // output staging stride: odd, conflict-free
    constexpr int F4 = 32 * HD / 4;          // float4s per K or V tile
    constexpr int PER = (F4 + NT - 1) / NT;  // float4s per thread per tile
    // Two K stages [32][KS] and two V stages [32][HD]; at the end the same
    // memory holds one block's outputs as [QB][OS], one block after the other.
    constexpr int STAGES = 2 * 32 * KS + 2 * 32 * HD;
    constexpr int OUT = QB * OS;
    __shared__ __attribute__((aligned(16))) float smem[STAGES > OUT ? STAGES : OUT];
    auto Ks = [&](int buf) { return smem + buf * 32 * KS; };
    auto Vs = [&](int buf) { return smem + 64 * KS + buf * 32 * HD; };

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int half = wave >> 2, w4 = wave & 3;     // block of the pair, wave in it
    const int lq = lane & 31, lh = lane >> 5;
    const int head = blockIdx.x, b = blockIdx.y;
    const int long_blk = p.nqb - 1 - (int)blockIdx.z;
    const int qblk = half ? (int)blockIdx.z : long_blk;
    // with nqb odd the middle block pairs with itself: waves 4-7 sit it out
    const bool active = half == 0 || qblk < long_blk;
    const int kvh = head / (p.h / p.hkv);
    const int T = p.t;
    const int ntiles = min(long_blk * QB + QB - 1, T - 1) / 32 + 1;  // key tiles to walk
    const int q0 = qblk * QB + w4 * 32;            // this wave's first query
    const int my_tiles = active && q0 < T ? q0 / 32 + 1 : 0;  // tiles this wave needs

    const float *Q = p.q + b * p.sqb + head * p.sqh;
    const float *K = p.k + b * p.skb + kvh * p.skh;
    const float *V = p.v + b * p.svb + kvh * p.svh;

    // Q operand: lane holds Q[q0 + lq][lh * NS + s] * scale * log2(e), s < NS
    // (the scores come out of the MFMAs already in log2 units).
    const float sc = p.scale * 1.4426950408889634f;
    float qr[NS];
    {
        const int qi = min(q0 + lq, T - 1);
        const float *src = Q + (int64_t)qi * p.sqt + lh * NS;
        if (NS % 4 == 0) {
#pragma unroll
            for (int s = 0; s < NS / 4; ++s) {
                const float4 v = reinterpret_cast<const float4 *>(src)[s];
                qr[4 * s + 0] = v.x * sc;
                qr[4 * s + 1] = v.y * sc;
                qr[4 * s + 2] = v.z * sc;
                qr[4 * s + 3] = v.w * sc;
            }
        } else {
#pragma unroll
            for (int s = 0; s < NS; ++s) qr[s] = src[s] * sc;
        }
    }

    // Keys past T read row T-1 instead (real, finite values: their scores
    // are masked and their P is 0), so every load is unconditional.
    float4 kreg[PER], vreg[PER];
    auto load_tile = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int f = tid + i * NT;
            if (F4 % NT == 0 || f < F4) {
                const int j = (4 * f) / HD, c = (4 * f) % HD;
                const int key = min(kt * 32 + j, T - 1);
                kreg[i] = *reinterpret_cast<const float4 *>(K + (int64_t)key * p.skt + c);
                vreg[i] = *reinterpret_cast<const float4 *>(V + (int64_t)key * p.svt + c);
            }
        }
    };
    auto store_tile = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int f = tid + i * NT;
            if (f < F4) {
                const int j = (4 * f) / HD, c = (4 * f) % HD;
                float *kd = Ks(buf) + j * KS + c;
                kd[0] = kreg[i].x;
                kd[1] = kreg[i].y;
                kd[2] = kreg[i].z;
                kd[3] = kreg[i].w;
                float *vd = Vs(buf) + j * HD + c;
                vd[0] = vreg[i].x;
                vd[1] = vreg[i].y;
                vd[2] = vreg[i].z;
                vd[3] = vreg[i].w;
            }
        }
    };

    floatx16 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;
    // Softmax state in log2 units: scores are scaled by scale * log2(e) and
    // exponentials are exp2 (the hardware's, which flushes results below
    // 2^-126 to 0). m_run is raised only when some lane's max grows by more
    // than 8 (then every exponential stays <= 2^8); O and l share the same
    // stale max, so O / l is unchanged.
    float m_run = -INFINITY, l_run = 0.0f;
    const int qi = q0 + lq;

    load_tile(0);
    store_tile(0);
    __syncthreads();
    for (int kt = 0; kt < ntiles; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < ntiles) load_tile(kt + 1);
        if (kt < my_tiles) {
            const float *Kb = Ks(cur);
            const float *Vb = Vs(cur);
            // S^T = K . Q^T: two independent accumulator chains, summed.
            floatx16 sacc, sacc1;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                sacc[r] = 0.0f;
                sacc1[r] = 0.0f;
            }
            const float *krow = Kb + lq * KS + lh * NS;
            if (NS % 4 == 0) {
#pragma unroll
                for (int t = 0; t < NS / 4; ++t) {
                    const float4 kv = reinterpret_cast<const float4 *>(krow)[t];
                    sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qr[4 * t + 0], sacc, 0, 0, 0);
                    sacc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qr[4 * t + 1], sacc1, 0, 0, 0);
                    sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qr[4 * t + 2], sacc, 0, 0, 0);
                    sacc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qr[4 * t + 3], sacc1, 0, 0, 0);
                }
            } else {
#pragma unroll
                for (int s = 0; s < NS; ++s)
                    sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(krow[s], qr[s], sacc, 0, 0, 0);
            }
            const int k0 = kt * 32;
            float pv[16];
            float mloc = -INFINITY;
            // only a tile that reaches the wave's first query or T needs the mask
            if (k0 + 31 <= q0 && k0 + 31 < T) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    pv[r] = sacc[r] + sacc1[r];
                    mloc = fmaxf(mloc, pv[r]);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = k0 + 8 * (r >> 2) + 4 * lh + (r & 3);
                    const float sv = sacc[r] + sacc1[r];
                    pv[r] = (key <= qi && key < T) ? sv : -INFINITY;
                    mloc = fmaxf(mloc, pv[r]);
                }
            }
            mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
            const bool need = mloc > m_run + 8.0f;  // always true on the first tile
            if (__any(need)) {
                const float m_new = need ? mloc : m_run;
                const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
                l_run *= alpha;
#pragma unroll
                for (int db = 0; db < NDB; ++db)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
                m_run = m_new;
            }
            float lsum = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                pv[r] = __builtin_amdgcn_exp2f(pv[r] - m_run);
                lsum += pv[r];
            }
            lsum += __shfl_xor(lsum, 32, 64);
            l_run += lsum;
            // O^T += V^T . P^T; lane lq reads the NDB consecutive dims it feeds.
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                const int key = 8 * (s >> 2) + 4 * lh + (s & 3);
                const float *vrow = Vb + key * HD;
                float a[NDB];
                if (NDB == 4) {
                    const float4 v4 = reinterpret_cast<const float4 *>(vrow)[lq];
                    a[0] = v4.x;
                    a[NDB > 1 ? 1 : 0] = v4.y;
                    a[NDB > 2 ? 2 : 0] = v4.z;
                    a[NDB > 3 ? 3 : 0] = v4.w;
                } else if (NDB == 2) {
                    const float2 v2 = reinterpret_cast<const float2 *>(vrow)[lq];
                    a[0] = v2.x;
                    a[NDB > 1 ? 1 : 0] = v2.y;
                } else {
                    a[0] = (HD >= 32 || lq < HD) ? vrow[HD >= 32 ? lq : (lq < HD ? lq : 0)] : 0.0f;
                }
#pragma unroll
                for (int db = 0; db < NDB; ++db)
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[db], pv[s], o[db], 0, 0, 0);
            }
        }
        if (kt + 1 < ntiles) store_tile(cur ^ 1);
        __syncthreads();
    }

    if (p.lse && my_tiles > 0 && lh == 0 && qi < T)
        p.lse[((int64_t)b * p.h + head) * T + qi] = m_run + log2f(l_run);
    // O^T -> LDS as [q][d], then coalesced row stores; the long block's waves
    // first, then the short block's, through the same staging rows.
    float *Os = smem + w4 * 32 * OS;
#pragma unroll
    for (int round = 0; round < 2; ++round) {
        const bool mine = half == round && my_tiles > 0;
        if (mine) {
            const float inv = 1.0f / l_run;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int i = 8 * (r >> 2) + 4 * lh + (r & 3);
                    const int d = NDB * i + db;
                    if (d < HD) Os[lq * OS + d] = o[db][r] * inv;
                }
        }
        __syncthreads();
        if (mine) {
            for (int idx = lane; idx < 32 * HD; idx += 64) {
                const int j = idx / HD, c = idx - j * HD;
                const int q = q0 + j;
                if (q < T)
                    p.out[b * p.sob + head * p.soh + (int64_t)q * p.sot + c] = Os[j * OS + c];
            }
        }
        if (round == 0) __syncthreads();
    }
}

// 16-row strips, 16 waves (heads of 64 and 128, grids of at least one
// 128-row block per CU). The same pairing of a long block (nqb-1-z, waves
// 0-7) with a short one (z, waves 8-15) and the same 32-key K/V tiles shared
// through a double-buffered LDS stage, but each wave owns 16 query rows and
// runs 16x16x4 MFMAs, so a wave needs half the registers (at most 128: four
// waves per SIMD instead of two). Wave w of a block takes strip w (w < 4) or
// 11 - w, so the two waves of a block that share a SIMD (w and w + 4) hold
// strips i and 7 - i: every SIMD carries the same causal work, and the
// barrier that ends each tile waits for no SIMD with more tiles than another.
// A wave stores its rows straight from its accumulators as soon as its last
// tile is done, while the other waves still compute.
//
// Layouts (lane l, g = l/16, i = l%16; register r of an accumulator block is
// row 4g + r of the 16x16 result, column i):
//   S^T block kb (keys 16kb..16kb+15 of the tile, query q0 + i): k-step s
//     pairs the head dims 32g + s (A: K[16kb + i][32g + s] from LDS, B: the
//     lane's own Q[q0 + i][32g + s]); lane l's register r is key 16kb+4g+r.
//   O^T block 4h+e (dims 64h + 4i' + e, i' = 0..15): k-step (kb, r) pairs the
//     keys 16kb + 4g + r (A: V[16kb+4g+r][64h + 4i + e], B: the lane's own P
//     register (kb, r)); lane l's register r' is O[q0 + i][64h + 16g + 4r' + e].
// Row max and sum of a query meet across its four lanes (i, i+16, i+32, i+48)
// through two lane swaps.
template <int HD>
__global__ __launch_bounds__(1024) void attn_fwd16_kernel(AttnP p) {
    static_assert(HD == 64 || HD == 128, "16-row strips take heads of 64 or 128");
    constexpr int NT = 1024;
    constexpr int QB = 128;
    constexpr int NS = HD / 4;      // S^T k-steps per key block (dims per lane group)
    constexpr int NH = HD / 64;     // O^T dim halves: blocks 4h .. 4h+3
    constexpr int KS = HD + 4;      // K row stride (16-byte rows, lanes 4 banks apart)
    constexpr int F4 = 32 * HD / 4; // float4s per K or V tile
    constexpr int PER = F4 / NT;    // 1 (HD 128) or 0.5 (HD 64: half the threads load)
    constexpr int RA = 3;           // LDS operand reads in flight ahead of their MFMAs
    // Two stages of 64 keys (two 32-key tiles each): one barrier per 64 keys.
    // Tile kt lives in stage (kt/2)&1, rows 32*(kt&1) ...
    __shared__ __attribute__((aligned(16))) float smem[2 * 64 * KS + 2 * 64 * HD];
    auto Ks = [&](int kt) { return smem + ((kt >> 1) & 1) * 64 * KS + (kt & 1) * 32 * KS; };
    auto Vs = [&](int kt) { return smem + 128 * KS + ((kt >> 1) & 1) * 64 * HD + (kt & 1) * 32 * HD; };

    // the wave index through readfirstlane: uniform, so what derives from it
    // (strip, rows, tile counts, their tests) is scalar work in scalar registers
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g = lane >> 4, li = lane & 15;
    const int half = wave >> 3, w8 = wave & 7;
    const int strip = w8 < 4 ? w8 : 11 - w8;
    const int head = blockIdx.x, b = blockIdx.y;
    const int long_blk = p.nqb - 1 - (int)blockIdx.z;
    const int qblk = half ? (int)blockIdx.z : long_blk;
    const bool active = half == 0 || qblk < long_blk;  // nqb odd: the middle block once
    const int kvh = head / (p.h / p.hkv);
    const int T = p.t;
    const int ntiles = min(long_blk * QB + QB - 1, T - 1) / 32 + 1;
    const int q0 = qblk * QB + strip * 16;
    const int my_tiles = active && q0 < T ? min(q0 + 15, T - 1) / 32 + 1 : 0;
    const int qi = q0 + li;

    const float *Q = p.q + b * p.sqb + head * p.sqh;
    const float *K = p.k + b * p.skb + kvh * p.skh;
    const float *V = p.v + b * p.svb + kvh * p.svh;

    const float sc = p.scale * 1.4426950408889634f;  // scores in log2 units
    float qr[NS];
    {
        const float4 *src = reinterpret_cast<const float4 *>(Q + (int64_t)min(qi, T - 1) * p.sqt + g * NS);
#pragma unroll
        for (int s = 0; s < NS / 4; ++s) {
            const float4 v = src[s];
            qr[4 * s + 0] = v.x * sc;
            qr[4 * s + 1] = v.y * sc;
            qr[4 * s + 2] = v.z * sc;
            qr[4 * s + 3] = v.w * sc;
        }
    }

    // thread tid loads float4 tid of the K tile and of the V tile (keys past
    // T read row T-1: finite values whose scores are masked)
    // (HD 64: threads past the tile read a copy of another thread's float4
    // and do not store it, so the loads need no branch and can sit inside
    // the MFMA stream)
    const bool loader = PER >= 1 || tid < F4;
    const int ltid = PER >= 1 ? tid : tid % F4;
    const int lj = (4 * ltid) / HD, lc = (4 * ltid) % HD;
    float4 kreg, vreg;
    // Buffer loads over the sequence's T rows: 32-bit offsets (the 64-bit
    // address arithmetic was a dozen VALU instructions per tile, and the VALU
    // takes its cycles from the matrix core), keys past T read zeros (finite;
    // their scores are masked and their P is 0). The host keeps T * stride
    // below 2^29 floats for this kernel.
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(K), (short)0, (int)(4 * (int64_t)T * p.skt), 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(V), (short)0, (int)(4 * (int64_t)T * p.svt), 0x00020000);
    const uint32_t klane = 4u * ((uint32_t)lj * (uint32_t)p.skt + (uint32_t)lc);
    const uint32_t vlane = 4u * ((uint32_t)lj * (uint32_t)p.svt + (uint32_t)lc);
    const uint32_t ktile = 128u * (uint32_t)p.skt, vtile = 128u * (uint32_t)p.svt;
    auto load_tile = [&](int kt) __attribute__((always_inline)) {
        kreg = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rk, klane + (uint32_t)kt * ktile, 0, 0));
        vreg = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rv, vlane + (uint32_t)kt * vtile, 0, 0));
    };
    auto store_tile = [&](int kt) __attribute__((always_inline)) {
        if (loader) {
            *reinterpret_cast<float4 *>(Ks(kt) + lj * KS + lc) = kreg;
            *reinterpret_cast<float4 *>(Vs(kt) + lj * HD + lc) = vreg;
        }
    };

    floatx4 o[4 * NH];
#pragma unroll
    for (int db = 0; db < 4 * NH; ++db) o[db] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.0f;

    // sum / max over a query's four lanes (i, i+16, i+32, i+48). Maxima as
    // bare v_max_f32 / v_max3_f32: fmaxf (and med3 with +inf, which the
    // compiler folds into it) takes a quieting max of each operand it cannot
    // prove canonical first (lane-swapped values, selects), and scores here
    // are finite or -inf, never NaN
    auto vmax = [](float x, float y) __attribute__((always_inline)) {
        float r;
        asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(x), "v"(y));
        return r;
    };
    auto vmax3 = [](float x, float y, float z) __attribute__((always_inline)) {
        float r;
        asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(y), "v"(z));
        return r;
    };
    auto quad_max = [&](float v) __attribute__((always_inline)) {
        auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = vmax(__uint_as_float(a[0]), __uint_as_float(a[1]));
        auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return vmax(__uint_as_float(c[0]), __uint_as_float(c[1]));
    };
    auto quad_sum = [](float v) __attribute__((always_inline)) {
        auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
        auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __uint_as_float(c[0]) + __uint_as_float(c[1]);
    };

    float pv[8];  // P of the current tile
    // scores and softmax of tile kt; the next tile's global loads (tile nxt)
    // are issued between its first MFMAs, not all at once after the barrier
    // V operands: 8 * NH float4 per tile, step i = NH*j + h:
    // V[16(j/4) + 4g + j%4][64h + 4li ..], each feeding 4 MFMAs, read RA ahead;
    // the first RA are issued before the softmax, so P.V starts without waiting
    constexpr int NV = 8 * NH;
    float4 vring[RA + 1];
    auto vread = [&](int kt, int i) __attribute__((always_inline)) {
        const int j = i / NH, h = i % NH;
        return reinterpret_cast<const float4 *>(Vs(kt) + (16 * (j >> 2) + 4 * g + (j & 3)) * HD + 4 * li)[16 * h];
    };
    auto qk_softmax = [&](int kt, int nxt) __attribute__((always_inline)) {
        const float *Kb = Ks(kt);
        // 16 float4 K operands per tile, step i = 2t + kb: K[16kb + li][g*NS + 4t ..],
        // each feeding 4 MFMAs. Steps go in pairs (2t, 2t+1), whose MFMAs
        // alternate between the two accumulators (no MFMA waits on the one
        // before it); a ring of four registers holds the pair in use and the
        // next one, the pair after that read as soon as a pair is used.
        floatx4 sacc[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
        constexpr int NK = 2 * (NS / 4);
        float4 ring[4];
        auto kread = [&](int i) __attribute__((always_inline)) {
            return reinterpret_cast<const float4 *>(Kb + (16 * (i & 1) + li) * KS + g * NS)[i >> 1];
        };
#pragma unroll
        for (int i = 0; i < 4; ++i) ring[i] = kread(i);
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int t = 0; t < NK / 2; ++t) {
            const float4 ka = ring[(2 * t) % 4], kc = ring[(2 * t + 1) % 4];
            sacc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.x, qr[4 * t + 0], sacc[0], 0, 0, 0);
            sacc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(kc.x, qr[4 * t + 0], sacc[1], 0, 0, 0);
            sacc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.y, qr[4 * t + 1], sacc[0], 0, 0, 0);
            sacc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(kc.y, qr[4 * t + 1], sacc[1], 0, 0, 0);
            sacc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.z, qr[4 * t + 2], sacc[0], 0, 0, 0);
            sacc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(kc.z, qr[4 * t + 2], sacc[1], 0, 0, 0);
            sacc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(ka.w, qr[4 * t + 3], sacc[0], 0, 0, 0);
            sacc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(kc.w, qr[4 * t + 3], sacc[1], 0, 0, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
            if (2 * t + 4 < NK) {
                ring[(2 * t) % 4] = kread(2 * t + 4);
                ring[(2 * t + 1) % 4] = kread(2 * t + 5);
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            }
            if (t == 0) {
                load_tile(nxt);
                __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < RA; ++i) vring[i] = vread(kt, i);
        __builtin_amdgcn_sched_group_barrier(0x100, RA, 0);
        __builtin_amdgcn_sched_barrier(0);
        const int k0 = kt * 32;
        // the scores stay in the accumulator registers; diagonal and partial
        // tiles overwrite their masked keys with -inf in place (a full tile
        // moves nothing)
#pragma unroll
        for (int j = 0; j < 8; ++j) pv[j] = sacc[j >> 2][j & 3];
        if (!(k0 + 31 <= q0 && k0 + 31 < T)) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int key = k0 + 16 * (j >> 2) + 4 * g + (j & 3);
                pv[j] = key <= qi && key < T ? pv[j] : -INFINITY;
            }
        }
        float mloc = vmax3(vmax3(vmax3(pv[0], pv[1], pv[2]), pv[3], pv[4]), pv[5], pv[6]);
        mloc = vmax(mloc, pv[7]);
        mloc = quad_max(mloc);
        const bool need = mloc > m_run + 8.0f;  // lazy rescale, as attn_fwd_kernel
        if (__any(need)) {
            const float m_new = need ? mloc : m_run;
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < 4 * NH; ++db)
#pragma unroll
                for (int r = 0; r < 4; ++r) o[db][r] *= alpha;
            m_run = m_new;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) pv[j] = __builtin_amdgcn_exp2f(pv[j] - m_run);
        float lsum = pv[0];
#pragma unroll
        for (int j = 1; j < 8; ++j) lsum += pv[j];
        // the lane's own share: the four lanes of a query rescale together
        // (one m_run), so their shares are summed once, when the strip ends
        l_run += lsum;
    };
    auto pv_apply = [&](int kt) __attribute__((always_inline)) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            if (i + RA < NV) vring[(i + RA) % (RA + 1)] = vread(kt, i + RA);
            const float4 v4 = vring[i % (RA + 1)];
            const int j = i / NH, h = i % NH;
            o[4 * h + 0] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4.x, pv[j], o[4 * h + 0], 0, 0, 0);
            o[4 * h + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4.y, pv[j], o[4 * h + 1], 0, 0, 0);
            o[4 * h + 2] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4.z, pv[j], o[4 * h + 2], 0, 0, 0);
            o[4 * h + 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(v4.w, pv[j], o[4 * h + 3], 0, 0, 0);
            if (i + RA < NV) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
        if (kt == my_tiles - 1) l_run = quad_sum(l_run);
        if (kt == my_tiles - 1 && qi < T) {
            // this strip is done: its rows leave now, straight from the accumulators
            const float inv = 1.0f / l_run;
            float *orow = p.out + b * p.sob + head * p.soh + (int64_t)qi * p.sot;
#pragma unroll
            for (int h = 0; h < NH; ++h)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    *reinterpret_cast<float4 *>(orow + 64 * h + 16 * g + 4 * r) =
                        make_float4(o[4 * h + 0][r] * inv, o[4 * h + 1][r] * inv,
                                    o[4 * h + 2][r] * inv, o[4 * h + 3][r] * inv);
            if (p.lse && g == 0) p.lse[((int64_t)b * p.h + head) * T + qi] = m_run + log2f(l_run);
        }
    };

    load_tile(0);
    store_tile(0);
    if (ntiles > 1) {
        load_tile(1);
        store_tile(1);
    }
    __syncthreads();
    auto step = [&](int kt) __attribute__((always_inline)) {
        // during tile kt, the tile two ahead goes to the other stage
        const int nxt = min(kt + 2, ntiles - 1);  // the last steps reload a tile they never store
        if (kt < my_tiles) {
            qk_softmax(kt, nxt);
            pv_apply(kt);
        } else {
            load_tile(nxt);
        }
        if (kt + 2 < ntiles) store_tile(kt + 2);
    };
    // one stage (two tiles) per iteration: each tile's position in the stage
    // is then a constant, and its LDS offsets immediates
    for (int m = 0; 2 * m < ntiles; ++m) {
        step(2 * m);
        if (2 * m + 1 < ntiles) {
            step(2 * m + 1);
            if (2 * m + 2 < ntiles) __syncthreads();
        }
    }
}

// Key-split variant for grids that would not cover the chip (few batch x head
// pairs, short T: the tiny preset has 32 pairs of 256 rows). A workgroup owns
// 32 query rows; its NWV waves (4, or 8 when a block reaches more than 4 key
// tiles, so no wave walks two tiles while others idle) take the key tiles up
// to the diagonal round-robin (wave w: tiles w, w+NWV, ...), each keeping the
// online softmax of its share,
// with K and V read straight from memory into the MFMA operand layouts (no
// LDS staging; the next tile's loads are in flight during the current one).
// The NWV partial states then merge through LDS in wave order: m = max m_w,
// l = sum l_w 2^(m_w - m), O = sum O_w 2^(m_w - m) / l. Heads up to 64 wide.
template <int HD, int NWV>
__global__ __launch_bounds__(64 * NWV) void attn_fwd_split_kernel(AttnP p) {
    constexpr int NS = HD / 2;
    constexpr int NDB = (HD + 31) / 32;
    constexpr int OS = HD + 1;
    __shared__ float sm_m[NWV][32], sm_l[NWV][32];
    __shared__ float sm_o[NWV][32 * OS];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lq = lane & 31, lh = lane >> 5;
    const int head = blockIdx.x, b = blockIdx.y;
    const int qblk = p.nqb - 1 - (int)blockIdx.z;  // longest rows first
    const int kvh = head / (p.h / p.hkv);
    const int T = p.t;
    const int q0 = qblk * 32;
    const int qi = q0 + lq;
    const int ntiles = min(q0 + 31, T - 1) / 32 + 1;

    const float *Q = p.q + b * p.sqb + head * p.sqh;
    const float *K = p.k + b * p.skb + kvh * p.skh;
    const float *V = p.v + b * p.svb + kvh * p.svh;

    float qr[NS];
    {
        const float *src = Q + (int64_t)min(qi, T - 1) * p.sqt + lh * NS;
#pragma unroll
        for (int s = 0; s < NS; ++s) qr[s] = src[s];
    }
    // Operands of one key tile: kr[s] = K[key lq][lh*NS + s] (S^T's A), and
    // vr[s][db] = V[key 8*(s/4) + 4*lh + s%4][NDB*lq + db] (O^T's A).
    // kn/vn receive the wave's next tile while the current one is used.
    // Every read is unconditional (keys past T read row T-1, head dims past
    // HD read dim HD-1: real, finite values whose scores are masked, whose P
    // is 0, or whose output rows are never stored), so the compiler can keep
    // the next tile's reads in flight instead of waiting on each one.
    float kr[NS], vr[16][NDB], kn[NS], vn[16][NDB];
    auto load_tile = [&](int kt, float (&kd)[NS], float (&vd)[16][NDB])
                         __attribute__((always_inline)) {
        const int key = kt * 32 + lq;
        const float *ks = K + (int64_t)min(key, T - 1) * p.skt + lh * NS;
        if constexpr (NS % 4 == 0) {
#pragma unroll
            for (int s = 0; s < NS / 4; ++s) {
                const float4 v = reinterpret_cast<const float4 *>(ks)[s];
                kd[4 * s + 0] = v.x;
                kd[4 * s + 1] = v.y;
                kd[4 * s + 2] = v.z;
                kd[4 * s + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int s = 0; s < NS; ++s) kd[s] = ks[s];
        }
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const int vk = min(kt * 32 + 8 * (s >> 2) + 4 * lh + (s & 3), T - 1);
            const float *vs = V + (int64_t)vk * p.svt;
            if constexpr (NDB == 2) {
                const float2 v2 = reinterpret_cast<const float2 *>(vs)[lq];
                vd[s][0] = v2.x;
                vd[s][NDB > 1 ? 1 : 0] = v2.y;
            } else {
                vd[s][0] = vs[HD >= 32 ? lq : min(lq, HD - 1)];
            }
        }
    };

    floatx16 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;
    const float sc = p.scale * 1.4426950408889634f;
    float m_run = -INFINITY, l_run = 0.0f;

    if (wave < ntiles) load_tile(wave, kr, vr);
    for (int kt = wave; kt < ntiles; kt += NWV) {
        if (kt + NWV < ntiles) load_tile(kt + NWV, kn, vn);
        floatx16 sacc, sacc1;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            sacc[r] = 0.0f;
            sacc1[r] = 0.0f;
        }
#pragma unroll
        for (int s = 0; s < NS; s += 2) {
            sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(kr[s], qr[s], sacc, 0, 0, 0);
            if (s + 1 < NS)
                sacc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(kr[s + 1], qr[s + 1], sacc1, 0, 0, 0);
        }
        const int k0 = kt * 32;
        float pv[16];
        float mloc = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = k0 + 8 * (r >> 2) + 4 * lh + (r & 3);
            const float sv = (sacc[r] + sacc1[r]) * sc;
            pv[r] = (key <= qi && key < T) ? sv : -INFINITY;
            mloc = fmaxf(mloc, pv[r]);
        }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
        const bool need = mloc > m_run + 8.0f;
        if (__any(need)) {
            const float m_new = need ? mloc : m_run;
            const float alpha = exp2f(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
            m_run = m_new;
        }
        float lsum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            pv[r] = exp2f(pv[r] - m_run);
            lsum += pv[r];
        }
        lsum += __shfl_xor(lsum, 32, 64);
        l_run += lsum;
#pragma unroll
        for (int s = 0; s < 16; ++s)
#pragma unroll
            for (int db = 0; db < NDB; ++db)
                o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vr[s][db], pv[s], o[db], 0, 0, 0);
#pragma unroll
        for (int s = 0; s < NS; ++s) kr[s] = kn[s];
#pragma unroll
        for (int s = 0; s < 16; ++s)
#pragma unroll
            for (int db = 0; db < NDB; ++db) vr[s][db] = vn[s][db];
    }

    if (lh == 0) {
        sm_m[wave][lq] = m_run;
        sm_l[wave][lq] = l_run;
    }
    __syncthreads();
    float mx = sm_m[0][lq];
#pragma unroll
    for (int w = 1; w < NWV; ++w) mx = fmaxf(mx, sm_m[w][lq]);
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < NWV; ++w) L += sm_l[w][lq] * exp2f(sm_m[w][lq] - mx);
    const float f = exp2f(m_run - mx) / L;  // 0 for a wave that saw no key
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int i = 8 * (r >> 2) + 4 * lh + (r & 3);
            const int d = NDB * i + db;
            if (d < HD) sm_o[wave][lq * OS + d] = o[db][r] * f;
        }
    if (p.lse && wave == 0 && lh == 0 && qi < T)
        p.lse[((int64_t)b * p.h + head) * T + qi] = mx + log2f(L);
    __syncthreads();
    for (int idx = tid; idx < 32 * HD; idx += 64 * NWV) {
        const int j = idx / HD, c = idx - j * HD;
        const int q = q0 + j;
        if (q < T) {
            float v = sm_o[0][j * OS + c];
#pragma unroll
            for (int w = 1; w < NWV; ++w) v += sm_o[w][j * OS + c];
            p.out[b * p.sob + head * p.soh + (int64_t)q * p.sot + c] = v;
        }
    }
}

// In-place RoPE (rope.rs:28-32) on heads of a strided layout: element
// (b, h, t, p) at x[b*sb + h*sh + t*st + p], positions t = 0..T-1. One
// workgroup per (b, t) row; its threads walk the row's nh*HD/2 rotation pairs.
// INV rotates by -angle: (x1, x2) -> (x1*c + x2*s, x2*c - x1*s), which is the
// RoPE backward dx1 = dfirst*cos + dsecond*sin, dx2 = dsecond*cos - dfirst*sin.
template <int HD, bool INV>
__global__ __launch_bounds__(256) void rope_rows_kernel(float *__restrict__ x, int64_t sb,
                                                        int64_t sh, int64_t st, int nh, int t,
                                                        const float *__restrict__ cos_t,
                                                        const float *__restrict__ sin_t,
                                                        int half_any) {
    // HD 0: a head of any even width, half_any pairs
    const int HALF = HD ? HD / 2 : half_any;
    const int row = blockIdx.x;
    const int bb = row / t, pos = row - bb * t;
    float *base = x + bb * sb + pos * st;
    const float *cr = cos_t + pos * HALF;
    const float *sr = sin_t + pos * HALF;
    for (int i = threadIdx.x; i < nh * HALF; i += 256) {
        const int hh = i / HALF, c = i - hh * HALF;
        float *r = base + hh * sh;
        const float x1 = r[c], x2 = r[c + HALF];
        const float cs = cr[c], sn = sr[c];
        if (INV) {
            r[c] = x1 * cs + x2 * sn;
            r[c + HALF] = x2 * cs - x1 * sn;
        } else {
            r[c] = x1 * cs - x2 * sn;
            r[c + HALF] = x2 * cs + x1 * sn;
        }
    }
}

template <int HD>
void launch_hd(Context &ctx, const AttnP &p, dim3 grid, bool split, bool rows16) {
    if constexpr (HD <= 64) {
        if (split) {
            if (p.t > 4 * 32)
                hipLaunchKernelGGL((attn_fwd_split_kernel<HD, 8>), grid, dim3(512), 0, ctx.stream, p);
            else
                hipLaunchKernelGGL((attn_fwd_split_kernel<HD, 4>), grid, dim3(256), 0, ctx.stream, p);
            return;
        }
    }
    grid.z = (grid.z + 1) / 2;  // query blocks in pairs
    if constexpr (HD == 64 || HD == 128) {
        if (rows16) {
            hipLaunchKernelGGL((attn_fwd16_kernel<HD>), grid, dim3(1024), 0, ctx.stream, p);
            return;
        }
    }
    hipLaunchKernelGGL((attn_fwd_kernel<HD>), grid, dim3(512), 0, ctx.stream, p);
}

bool al16(const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

}  // namespace

template <bool INV>
void launch_rope_rows(Context &ctx, float *x, int64_t sb, int64_t sh, int64_t st, int nhi,
                      int ti, int64_t hd, const float *cos_t, const float *sin_t, dim3 grid) {
    const dim3 block(256);
    const int half = (int)(hd / 2);
    switch (hd) {
        case 4: hipLaunchKernelGGL((rope_rows_kernel<4, INV>), grid, block, 0, ctx.stream, x, sb, sh, st, nhi, ti, cos_t, sin_t, half); break;
        case 8: hipLaunchKernelGGL((rope_rows_kernel<8, INV>), grid, block, 0, ctx.stream, x, sb, sh, st, nhi, ti, cos_t, sin_t, half); break;
        case 16: hipLaunchKernelGGL((rope_rows_kernel<16, INV>), grid, block, 0, ctx.stream, x, sb, sh, st, nhi, ti, cos_t, sin_t, half); break;
        case 32: hipLaunchKernelGGL((rope_rows_kernel<32, INV>), grid, block, 0, ctx.stream, x, sb, sh, st, nhi, ti, cos_t, sin_t, half); break;
        case 64: hipLaunchKernelGGL((rope_rows_kernel<64, INV>), grid, block, 0, ctx.stream, x, sb, sh, st, nhi, ti, cos_t, sin_t, half); break;
        case 128: hipLaunchKernelGGL((rope_rows_kernel<128, INV>), grid, block, 0, ctx.stream, x, sb, sh, st, nhi, ti, cos_t, sin_t, half); break;
        default: hipLaunchKernelGGL((rope_rows_kernel<0, INV>), grid, block, 0, ctx.stream, x, sb, sh, st, nhi, ti, cos_t, sin_t, half); break;
    }
}

void launch_rope_strided(Context &ctx, float *x, int64_t sb, int64_t sh, int64_t st, int64_t nb,
                         int64_t nh, int64_t t, int64_t hd, const float *cos_t,
                         const float *sin_t, bool inverse) {
    if (nb * t > 0x7fffffff || nh * (hd / 2) > 0x7fffffff) fail(MMH_ERR_SHAPE, "rope: too many rows");
    if (hd <= 0 || hd % 2) fail(MMH_ERR_SHAPE, "rope: head_dim must be even");
    const dim3 grid((unsigned)(nb * t));
    if (inverse)
        launch_rope_rows<true>(ctx, x, sb, sh, st, (int)nh, (int)t, hd, cos_t, sin_t, grid);
    else
        launch_rope_rows<false>(ctx, x, sb, sh, st, (int)nh, (int)t, hd, cos_t, sin_t, grid);
    check_hip(hipGetLastError(), "rope launch");
}

bool native_head(int64_t hd) {
    return hd == 4 || hd == 8 || hd == 16 || hd == 32 || hd == 64 || hd == 128;
}

int64_t kernel_head(int64_t hd) {
    for (int64_t w : {4, 8, 16, 32, 64, 128})
        if (hd <= w) return w;
    return 0;
}

namespace {

// Heads of [nb, nh, t, hd] at strides (sb, sh, st) <-> contiguous heads of hp
// >= hd columns, zero beyond hd: one workgroup per (batch, position) row.
__global__ __launch_bounds__(256) void pad_heads_kernel(const float *__restrict__ src, int64_t sb,
                                                        int64_t sh, int64_t st, int nh, int t,
                                                        int hd, float *__restrict__ dst, int hp) {
    const int row = blockIdx.x;
    const int bb = row / t, pos = row - bb * t;
    const float *s = src + bb * sb + pos * st;
    for (int i = threadIdx.x; i < nh * hp; i += 256) {
        const int hh = i / hp, c = i - hh * hp;
        dst[(((int64_t)bb * nh + hh) * t + pos) * hp + c] = c < hd ? s[hh * sh + c] : 0.0f;
    }
}

__global__ __launch_bounds__(256) void unpad_heads_kernel(const float *__restrict__ src, int hp,
                                                          int nh, int t, int hd,
                                                          float *__restrict__ dst, int64_t sb,
                                                          int64_t sh, int64_t st) {
    const int row = blockIdx.x;
    const int bb = row / t, pos = row - bb * t;
    float *o = dst + bb * sb + pos * st;
    for (int i = threadIdx.x; i < nh * hd; i += 256) {
        const int hh = i / hd, c = i - hh * hd;
        o[hh * sh + c] = src[(((int64_t)bb * nh + hh) * t + pos) * hp + c];
    }
}

}  // namespace

void launch_pad_heads(Context &ctx, const float *src, int64_t sb, int64_t sh, int64_t st,
                      int64_t nb, int64_t nh, int64_t t, int64_t hd, float *dst, int64_t hp) {
    if (nb * t > 0x7fffffff || nh * hp > 0x7fffffff) fail(MMH_ERR_SHAPE, "attention: shape too large");
    hipLaunchKernelGGL(pad_heads_kernel, dim3((unsigned)(nb * t)), dim3(256), 0, ctx.stream, src,
                       sb, sh, st, (int)nh, (int)t, (int)hd, dst, (int)hp);
    check_hip(hipGetLastError(), "pad heads launch");
}

void launch_unpad_heads(Context &ctx, const float *src, int64_t hp, int64_t nb, int64_t nh,
                        int64_t t, int64_t hd, float *dst, int64_t sb, int64_t sh, int64_t st) {
    if (nb * t > 0x7fffffff || nh * hd > 0x7fffffff) fail(MMH_ERR_SHAPE, "attention: shape too large");
    hipLaunchKernelGGL(unpad_heads_kernel, dim3((unsigned)(nb * t)), dim3(256), 0, ctx.stream, src,
                       (int)hp, (int)nh, (int)t, (int)hd, dst, sb, sh, st);
    check_hip(hipGetLastError(), "unpad heads launch");
}

// q and k rotated in place (the forward's RoPE, or its inverse on gradients);
// one launch when the k heads directly follow the q heads in each row (the
// fused QKV layout).
void rope_qk(Context &ctx, float *q, float *k, int64_t sqb, int64_t sqh, int64_t sqt, int64_t skb,
             int64_t skh, int64_t skt, int64_t b, int64_t h, int64_t hkv, int64_t t, int64_t hd,
             const float *cos_t, const float *sin_t, bool inverse) {
    if (k == q + h * sqh && skb == sqb && skh == sqh && skt == sqt) {
        launch_rope_strided(ctx, q, sqb, sqh, sqt, b, h + hkv, t, hd, cos_t, sin_t, inverse);
    } else {
        launch_rope_strided(ctx, q, sqb, sqh, sqt, b, h, t, hd, cos_t, sin_t, inverse);
        launch_rope_strided(ctx, k, skb, skh, skt, b, hkv, t, hd, cos_t, sin_t, inverse);
    }
}

namespace {

// The kernels on heads of a width they take (4, 8, 16, 32, 64 or 128),
// scores scaled by `scale`.
void attention_kernels(Context &ctx, const AttnDesc &d, float scale) {
    const int64_t strides[] = {d.sqb, d.sqh, d.sqt, d.skb, d.skh, d.skt, d.svb, d.svh, d.svt};
    for (int64_t s : strides)
        if (s % 4) fail(MMH_ERR_SHAPE, "attention: strides must be multiples of 4 floats");
    if (!al16(d.q) || !al16(d.k) || !al16(d.v))
        fail(MMH_ERR_ARGUMENT, "attention: q, k and v must be 16-byte aligned");
    AttnP p{};
    p.q = d.q;
    p.k = d.k;
    p.v = d.v;
    p.out = d.out;
    p.lse = d.lse;
    p.sqb = d.sqb; p.sqh = d.sqh; p.sqt = d.sqt;
    p.skb = d.skb; p.skh = d.skh; p.skt = d.skt;
    p.svb = d.svb; p.svh = d.svh; p.svt = d.svt;
    p.sob = d.sob; p.soh = d.soh; p.sot = d.sot;
    p.h = (int)d.h;
    p.hkv = (int)d.hkv;
    p.t = (int)d.t;
    // The key-split kernel when 128-row query blocks would leave CUs idle
    // (heads up to 64 wide).
    const int cus = ctx.cu_count > 0 ? ctx.cu_count : 256;
    const bool split = d.hd <= 64 && d.b * d.h * ((d.t + 127) / 128) < cus;
    p.nqb = (int)(split ? (d.t + 31) / 32 : (d.t + 127) / 128);
    p.scale = scale;
    dim3 grid((unsigned)d.h, (unsigned)d.b, (unsigned)p.nqb);
    // the 16-row kernel stores rows as float4s and reads K and V through
    // 32-bit buffer offsets over the sequence's rows
    const bool rows16 = al16(d.out) && d.sob % 4 == 0 && d.soh % 4 == 0 && d.sot % 4 == 0 &&
                        d.t * std::max(d.skt, d.svt) < (int64_t(1) << 29);
    switch (d.hd) {
        case 4: launch_hd<4>(ctx, p, grid, split, false); break;
        case 8: launch_hd<8>(ctx, p, grid, split, false); break;
        case 16: launch_hd<16>(ctx, p, grid, split, false); break;
        case 32: launch_hd<32>(ctx, p, grid, split, false); break;
        case 64: launch_hd<64>(ctx, p, grid, split, rows16); break;
        default: launch_hd<128>(ctx, p, grid, split, rows16); break;
    }
    check_hip(hipGetLastError(), "attention launch");
}

}  // namespace

void attention(Context &ctx, const AttnDesc &d) {
    if (d.b <= 0 || d.h <= 0 || d.hkv <= 0 || d.t <= 0 || d.hd <= 0)
        fail(MMH_ERR_SHAPE, "attention: empty shape");
    if (d.h % d.hkv != 0) fail(MMH_ERR_SHAPE, "attention: n_heads is not a multiple of n_kv_heads");
    if (d.b > 65535 || d.h > 0x7fffffff || d.t > 0x3fffffff)
        fail(MMH_ERR_SHAPE, "attention: shape too large");
    const int64_t hp = kernel_head(d.hd);
    if (hp == 0 || (!native_head(d.hd) && d.hd % 2))
        fail(MMH_ERR_SHAPE, "attention: head_dim must be 4, 8, 16, 32, 64 or 128, or even and "
                            "below 128");
    // q and k rows are rotated in place before the kernel reads them
    if (d.cos_t)
        rope_qk(ctx, const_cast<float *>(d.q), const_cast<float *>(d.k), d.sqb, d.sqh, d.sqt,
                d.skb, d.skh, d.skt, d.b, d.h, d.hkv, d.t, d.hd, d.cos_t, d.sin_t, false);
    const float scale = 1.0f / sqrtf((float)d.hd);  // attention.rs:82
    if (native_head(d.hd)) {
        attention_kernels(ctx, d, scale);
        return;
    }
    // Other even widths run on the next kernel width: q, k, v copied into
    // heads of hp columns, zero beyond hd (a zero column adds nothing to a
    // score; output columns past hd are dropped), the scale that of hd.
    const int64_t nq = d.b * d.h * d.t * hp, nk = d.b * d.hkv * d.t * hp;
    float *qp = static_cast<float *>(
        ctx.workspace(Context::kPadSlot, (size_t)(2 * nq + 2 * nk) * 4));
    float *kp = qp + nq, *vp = kp + nk, *op = vp + nk;
    launch_pad_heads(ctx, d.q, d.sqb, d.sqh, d.sqt, d.b, d.h, d.t, d.hd, qp, hp);
    launch_pad_heads(ctx, d.k, d.skb, d.skh, d.skt, d.b, d.hkv, d.t, d.hd, kp, hp);
    launch_pad_heads(ctx, d.v, d.svb, d.svh, d.svt, d.b, d.hkv, d.t, d.hd, vp, hp);
    AttnDesc e = d;
    e.q = qp;
    e.k = kp;
    e.v = vp;
    e.out = op;
    e.sqb = e.sob = d.h * d.t * hp;
    e.sqh = e.soh = d.t * hp;
    e.sqt = e.sot = hp;
    e.skb = e.svb = d.hkv * d.t * hp;
    e.skh = e.svh = d.t * hp;
    e.skt = e.svt = hp;
    e.hd = hp;
    e.cos_t = e.sin_t = nullptr;
    attention_kernels(ctx, e, scale);
    launch_unpad_heads(ctx, op, hp, d.b, d.h, d.t, d.hd, d.out, d.sob, d.soh, d.sot);
}

}  // namespace mmh
