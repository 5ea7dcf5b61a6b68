// Backward of the fused causal attention on CDNA4 matrix cores (fp32 MFMA
// 32x32x2). It replaces the reference's chain of closures for
// probs.v, softmax, scale + mask and q.k^T (ops_matmul.rs:100-125,
// ops_reduce.rs:144-175, ops_elementwise.rs:301-306, repeat_interleave
// backward ops_shape.rs:209-219) with two kernels that rebuild the
// probabilities from the forward's saved log-sum-exp and never hold a [T,T]
// tensor:
//
//   dq kernel  (one workgroup = 4 waves x 32 queries of one (batch, head)):
//       D     = rowsum(dO * O)                         (also written for dkv)
//       S^T   = K . Q^T,  P^T = exp2(S^T*scale*log2e - lse2)
//       dP^T  = V . dO^T, dS^T = P^T * (dP^T - D)
//       dQ^T += K^T . dS^T                             (dS^T straight from the
//                                                      accumulators)
//   dkv kernel (one workgroup = 4 waves x 32 keys of one (batch, kv head),
//   or of one query head when GQA partials are wanted, see below):
//       for every query head of the group and every query tile at or after
//       the keys: S = Q . K^T, P, dP = dO . V^T, dS as above,
//       dV^T += dO^T . P and dK^T += Q^T . dS
//
// Every per-row quantity lives in the lane that owns the row, as in the
// forward kernel: with the MFMA layout (lane l: column l%32; register r: row
// 8*(r/4) + 4*(l/32) + r%4), a product whose B operand is an accumulator
// block is summed over the accumulator's rows in that permuted order, which
// the A operand follows. Summing the group's heads inside one workgroup (in
// head order) makes dK and dV deterministic without atomics. With GQA and a
// scratch buffer, each query head gets its own workgroups instead (twice the
// grid at 2 heads per kv head, so the long key blocks near the start of the
// sequence no longer leave CUs waiting) and writes its partial dK, dV; a
// second kernel sums a group's partials in head order. The gradient of
// the scaled scores is dS*scale (attention.rs:83), applied to dQ and dK at
// the end. Entries above the diagonal have P = 0 and contribute nothing.
// Heads of 64 and 128 take the same products with 16 rows per wave
// (attn_bwd_dq16_kernel, attn_bwd_dkv16_kernel below); small grids take the
// strip kernels at the end of the file.
#include <algorithm>

#include "mmh_internal.h"

namespace mmh {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

struct BwdP {
    const float *q, *k, *v, *o, *dout, *lse;
    float *dq, *dk, *dv, *dvec;
    int64_t sqb, sqh, sqt, skb, skh, skt, svb, svh, svt, sob, soh, sot;
    float *part;  // per-query-head partial dK, dV [2][B][H][T][hd], or null
    int h, hkv, t, nqb, nkb;
    float scale;
};

// A raw buffer over everything from base on (32-bit offsets, no range
// check that matters) and its 16-byte load.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_all(const float *base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), (short)0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ float4 ld4b(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

__device__ __forceinline__ floatx16 mfma(float a, float b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// A lane's operand run: NS consecutive floats from src (16-byte aligned when NS % 4 == 0).
template <int NS>
__device__ __forceinline__ void load_run(float (&r)[NS], const float *src) {
    if constexpr (NS % 4 == 0) {
#pragma unroll
        for (int s = 0; s < NS / 4; ++s) {
            const float4 v = reinterpret_cast<const float4 *>(src)[s];
            r[4 * s + 0] = v.x;
            r[4 * s + 1] = v.y;
            r[4 * s + 2] = v.z;
            r[4 * s + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int s = 0; s < NS; ++s) r[s] = src[s];
    }
}

// Operands of the "row-shared" products (B from accumulators): lane lq takes
// dims NDB*lq .. NDB*lq + NDB-1 of one LDS row; block db row i is dim NDB*i+db.
template <int HD, int NDB>
__device__ __forceinline__ void read_dims(float (&a)[NDB], const float *row, int lq) {
    if constexpr (NDB == 4) {
        const float4 v = reinterpret_cast<const float4 *>(row)[lq];
        a[0] = v.x;
        a[1] = v.y;
        a[2] = v.z;
        a[3] = v.w;
    } else if constexpr (NDB == 2) {
        const float2 v = reinterpret_cast<const float2 *>(row)[lq];
        a[0] = v.x;
        a[1] = v.y;
    } else if constexpr (HD >= 32) {
        a[0] = row[lq];
    } else {
        a[0] = lq < HD ? row[lq] : 0.0f;
    }
}

// Two dot-product chains over a lane's run: acc0/acc1 += X[row lq] . Y^T where
// the LDS row xrow holds the A operand and y (registers) the B operand.
template <int NS>
__device__ __forceinline__ void dot_chains(const float *xrow, const float (&y)[NS], floatx16 &acc0,
                                           floatx16 &acc1) {
    if constexpr (NS % 4 == 0) {
#pragma unroll
        for (int t = 0; t < NS / 4; ++t) {
            const float4 xv = reinterpret_cast<const float4 *>(xrow)[t];
            acc0 = mfma(xv.x, y[4 * t + 0], acc0);
            acc1 = mfma(xv.y, y[4 * t + 1], acc1);
            acc0 = mfma(xv.z, y[4 * t + 2], acc0);
            acc1 = mfma(xv.w, y[4 * t + 3], acc1);
        }
    } else {
#pragma unroll
        for (int s = 0; s < NS; ++s) acc0 = mfma(xrow[s], y[s], acc0);
    }
}

template <int HD>
__global__ __launch_bounds__(256, 1) void attn_bwd_dq_kernel(BwdP p) {
    constexpr int NS = HD / 2, NDB = (HD + 31) / 32, KS = HD + 4, OS = HD + 1;
    constexpr int F4 = 32 * HD / 4, PER = (F4 + 255) / 256;
    constexpr int STAGES = 4 * 32 * KS;  // K and V tiles, two stages each
    constexpr int OUT = 128 * OS;
    __shared__ __attribute__((aligned(16))) float smem[STAGES > OUT ? STAGES : OUT];
    auto Ks = [&](int buf) { return smem + buf * 32 * KS; };
    auto Vs = [&](int buf) { return smem + (2 + buf) * 32 * KS; };

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lq = lane & 31, lh = lane >> 5;
    const int head = blockIdx.x, b = blockIdx.y;
    const int qblk = p.nqb - 1 - (int)blockIdx.z;  // longest rows first
    const int kvh = head / (p.h / p.hkv);
    const int T = p.t;
    const int q_first = qblk * 128;
    const int q_last = min(q_first + 127, T - 1);
    const int ntiles = q_last / 32 + 1;
    const int q0 = q_first + wave * 32;
    const int my_tiles = q0 < T ? q0 / 32 + 1 : 0;
    const int qi = q0 + lq;
    const int qc = min(qi, T - 1);

    const float *Q = p.q + b * p.sqb + head * p.sqh;
    const float *K = p.k + b * p.skb + kvh * p.skh;
    const float *V = p.v + b * p.svb + kvh * p.svh;
    const float *O = p.o + b * p.sob + head * p.soh;
    const float *dO = p.dout + b * p.sob + head * p.soh;
    const int64_t rows = ((int64_t)b * p.h + head) * T;

    // qr carries scale * log2(e), so S comes out of the MFMAs in log2 units
    const float sc = p.scale * 1.4426950408889634f;
    float qr[NS], gr[NS];
    load_run<NS>(qr, Q + (int64_t)qc * p.sqt + lh * NS);
#pragma unroll
    for (int s = 0; s < NS; ++s) qr[s] *= sc;
    load_run<NS>(gr, dO + (int64_t)qc * p.sot + lh * NS);
    float dsum = 0.0f;
    {
        const float *orow = O + (int64_t)qc * p.sot + lh * NS;
#pragma unroll
        for (int s = 0; s < NS; ++s) dsum += gr[s] * orow[s];
    }
    dsum += __shfl_xor(dsum, 32, 64);
    const float Dq = dsum;
    const float L2 = p.lse[rows + qc];
    if (lh == 0 && qi < T) p.dvec[rows + qi] = Dq;

    // keys past T read row T-1 (finite values whose P is 0): no predicates
    float4 kreg[PER], vreg[PER];
    auto load_tile = [&](int kt) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int f = tid + i * 256;
            if (F4 % 256 == 0 || f < F4) {
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
            const int f = tid + i * 256;
            if (f < F4) {
                const int j = (4 * f) / HD, c = (4 * f) % HD;
                float *kd = Ks(buf) + j * KS + c;
                kd[0] = kreg[i].x;
                kd[1] = kreg[i].y;
                kd[2] = kreg[i].z;
                kd[3] = kreg[i].w;
                float *vd = Vs(buf) + j * KS + c;
                vd[0] = vreg[i].x;
                vd[1] = vreg[i].y;
                vd[2] = vreg[i].z;
                vd[3] = vreg[i].w;
            }
        }
    };

    floatx16 dq[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) dq[db][r] = 0.0f;

    load_tile(0);
    store_tile(0);
    __syncthreads();
    for (int kt = 0; kt < ntiles; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < ntiles) load_tile(kt + 1);
        if (kt < my_tiles) {
            const float *Kb = Ks(cur);
            const float *Vb = Vs(cur);
            floatx16 s0, s1, g0, g1;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                s0[r] = 0.0f;
                s1[r] = 0.0f;
                g0[r] = 0.0f;
                g1[r] = 0.0f;
            }
            dot_chains<NS>(Kb + lq * KS + lh * NS, qr, s0, s1);
            dot_chains<NS>(Vb + lq * KS + lh * NS, gr, g0, g1);
            const int k0 = kt * 32;
            // only a tile reaching the wave's first query or T needs the mask;
            // exp2 is the hardware's (results below 2^-126 flush to 0)
            const bool full = k0 + 31 <= q0 && k0 + 31 < T;
            float ds[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = k0 + 8 * (r >> 2) + 4 * lh + (r & 3);
                // masked keys enter the exponential as -inf (a select; P = 0)
                const float pr = __builtin_amdgcn_exp2f(full || (key <= qi && key < T) ? (s0[r] + s1[r]) - L2 : -INFINITY);
                ds[r] = pr * ((g0[r] + g1[r]) - Dq);
            }
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                const int key = 8 * (s >> 2) + 4 * lh + (s & 3);
                float a[NDB];
                read_dims<HD, NDB>(a, Kb + key * KS, lq);
#pragma unroll
                for (int db = 0; db < NDB; ++db) dq[db] = mfma(a[db], ds[s], dq[db]);
            }
        }
        if (kt + 1 < ntiles) store_tile(cur ^ 1);
        __syncthreads();
    }

    float *Os = smem + wave * 32 * OS;
    if (my_tiles > 0) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int i = 8 * (r >> 2) + 4 * lh + (r & 3);
                const int d = NDB * i + db;
                if (d < HD) Os[lq * OS + d] = dq[db][r] * p.scale;
            }
    }
    __syncthreads();
    if (my_tiles > 0) {
        for (int idx = lane; idx < 32 * HD; idx += 64) {
            const int j = idx / HD, c = idx - j * HD;
            const int q = q0 + j;
            if (q < T) p.dq[b * p.sqb + head * p.sqh + (int64_t)q * p.sqt + c] = Os[j * OS + c];
        }
    }
}

template <int HD>
__global__ __launch_bounds__(256, 1) void attn_bwd_dkv_kernel(BwdP p) {
    constexpr int NS = HD / 2, NDB = (HD + 31) / 32, KS = HD + 4, OS = HD + 1;
    constexpr int F4 = 32 * HD / 4, PER = (F4 + 255) / 256;
    constexpr int TILE = 2 * 32 * KS + 64;  // Q [32][KS], dO [32][KS], lse2[32], D[32]
    constexpr int STAGES = 2 * TILE;
    constexpr int OUT = 128 * OS;
    __shared__ __attribute__((aligned(16))) float smem[STAGES > OUT ? STAGES : OUT];
    auto Qs = [&](int buf) { return smem + buf * TILE; };
    auto Gs = [&](int buf) { return smem + buf * TILE + 32 * KS; };
    auto Ls = [&](int buf) { return smem + buf * TILE + 64 * KS; };
    auto Ds = [&](int buf) { return smem + buf * TILE + 64 * KS + 32; };

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lq = lane & 31, lh = lane >> 5;
    const int groups = p.h / p.hkv;
    // kv head and the group's heads this workgroup covers: all of them, or
    // one (query head blockIdx.x) when writing partials
    const int kvh = p.part ? (int)blockIdx.x / groups : (int)blockIdx.x;
    const int g0 = p.part ? (int)blockIdx.x - kvh * groups : 0;
    const int ng = p.part ? 1 : groups;
    const int b = blockIdx.y;
    const int kblk = blockIdx.z;  // block 0 sees the most queries and starts first
    const int T = p.t;
    const int k_first = kblk * 128;
    const int k0 = k_first + wave * 32;  // this wave's first key
    const int kj = k0 + lq;
    const int kc = min(kj, T - 1);
    const int qt_first = k_first / 32;
    const int nqt = (T + 31) / 32;
    const int per_head = nqt - qt_first;
    const int total = ng * per_head;
    const int my_first = k0 / 32;  // query tiles before this one are all above the keys

    const float *K = p.k + b * p.skb + kvh * p.skh;
    const float *V = p.v + b * p.svb + kvh * p.svh;
    // kr carries scale * log2(e), so S comes out of the MFMAs in log2 units
    const float sc = p.scale * 1.4426950408889634f;
    float kr[NS], vr[NS];
    load_run<NS>(kr, K + (int64_t)kc * p.skt + lh * NS);
#pragma unroll
    for (int s = 0; s < NS; ++s) kr[s] *= sc;
    load_run<NS>(vr, V + (int64_t)kc * p.svt + lh * NS);

    float4 qreg[PER], greg[PER];
    float lreg = 0.0f;
    auto load_tile = [&](int it) __attribute__((always_inline)) {
        const int g = it / per_head;
        const int qt = qt_first + (it - g * per_head);
        const int head = kvh * groups + g0 + g;
        const float *Qh = p.q + b * p.sqb + head * p.sqh;
        const float *Gh = p.dout + b * p.sob + head * p.soh;
        // rows past T read row T-1 (finite; their P is 0): no predicates
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int f = tid + i * 256;
            if (F4 % 256 == 0 || f < F4) {
                const int j = (4 * f) / HD, c = (4 * f) % HD;
                const int q = min(qt * 32 + j, T - 1);
                qreg[i] = *reinterpret_cast<const float4 *>(Qh + (int64_t)q * p.sqt + c);
                greg[i] = *reinterpret_cast<const float4 *>(Gh + (int64_t)q * p.sot + c);
            }
        }
        {
            // lanes 0-31 fetch the tile's log-sum-exps, 32-63 its D values
            const int q = min(qt * 32 + (tid & 31), T - 1);
            const int64_t at = ((int64_t)b * p.h + head) * T + q;
            lreg = ((tid & 32) ? p.dvec : p.lse)[at];
        }
    };
    auto store_tile = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int f = tid + i * 256;
            if (f < F4) {
                const int j = (4 * f) / HD, c = (4 * f) % HD;
                float *qd = Qs(buf) + j * KS + c;
                qd[0] = qreg[i].x;
                qd[1] = qreg[i].y;
                qd[2] = qreg[i].z;
                qd[3] = qreg[i].w;
                float *gd = Gs(buf) + j * KS + c;
                gd[0] = greg[i].x;
                gd[1] = greg[i].y;
                gd[2] = greg[i].z;
                gd[3] = greg[i].w;
            }
        }
        if (tid < 32)
            Ls(buf)[tid] = lreg;
        else if (tid < 64)
            Ds(buf)[tid - 32] = lreg;
    };

    floatx16 dk[NDB], dv[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            dk[db][r] = 0.0f;
            dv[db][r] = 0.0f;
        }
    load_tile(0);
    store_tile(0);
    __syncthreads();
    for (int it = 0; it < total; ++it) {
        const int cur = it & 1;
        if (it + 1 < total) load_tile(it + 1);
        const int g = it / per_head;
        const int qt = qt_first + (it - g * per_head);
        if (qt >= my_first && k0 < T) {
            const float *Qb = Qs(cur);
            const float *Gb = Gs(cur);
            const float *Lb = Ls(cur);
            const float *Db = Ds(cur);
            floatx16 s0, s1, g0, g1;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                s0[r] = 0.0f;
                s1[r] = 0.0f;
                g0[r] = 0.0f;
                g1[r] = 0.0f;
            }
            dot_chains<NS>(Qb + lq * KS + lh * NS, kr, s0, s1);
            dot_chains<NS>(Gb + lq * KS + lh * NS, vr, g0, g1);
            // the mask only where the tile reaches the wave's keys or T
            const bool full = qt * 32 >= k0 + 31 && qt * 32 + 31 < T && k0 + 31 < T;
            float pv[16], ds[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = 8 * (r >> 2) + 4 * lh + (r & 3);
                const int q = qt * 32 + row;
                const float pr = __builtin_amdgcn_exp2f(full || (kj <= q && q < T && kj < T) ? (s0[r] + s1[r]) - Lb[row] : -INFINITY);
                pv[r] = pr;
                ds[r] = pr * ((g0[r] + g1[r]) - Db[row]);
            }
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                const int row = 8 * (s >> 2) + 4 * lh + (s & 3);
                float ag[NDB], aq[NDB];
                read_dims<HD, NDB>(ag, Gb + row * KS, lq);
                read_dims<HD, NDB>(aq, Qb + row * KS, lq);
#pragma unroll
                for (int db = 0; db < NDB; ++db) {
                    dv[db] = mfma(ag[db], pv[s], dv[db]);
                    dk[db] = mfma(aq[db], ds[s], dk[db]);
                }
            }
        }
        if (it + 1 < total) store_tile(cur ^ 1);
        __syncthreads();
    }

    // dK = scale * dK^T and dV = dV^T, each through LDS as [key][d], then rows.
    float *Os = smem + wave * 32 * OS;
    for (int which = 0; which < 2; ++which) {
        if (k0 < T) {
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int i = 8 * (r >> 2) + 4 * lh + (r & 3);
                    const int d = NDB * i + db;
                    if (d < HD) Os[lq * OS + d] = which == 0 ? dk[db][r] * p.scale : dv[db][r];
                }
        }
        __syncthreads();
        if (k0 < T) {
            float *dst;
            int64_t st;
            if (p.part) {
                const int64_t plane = (int64_t)gridDim.y * p.h * T * HD;
                dst = p.part + which * plane + ((int64_t)b * p.h + blockIdx.x) * T * HD;
                st = HD;
            } else {
                dst = which == 0 ? p.dk + b * p.skb + kvh * p.skh : p.dv + b * p.svb + kvh * p.svh;
                st = which == 0 ? p.skt : p.svt;
            }
            for (int idx = lane; idx < 32 * HD; idx += 64) {
                const int j = idx / HD, c = idx - j * HD;
                const int key = k0 + j;
                if (key < T) dst[(int64_t)key * st + c] = Os[j * OS + c];
            }
        }
        __syncthreads();
    }
}

// ---- 16-row strips (heads of 64 and 128) ------------------------------------
// The products above with 16x16x4 MFMAs and 16 rows (dq: queries, dkv: keys)
// per wave, 8 waves per workgroup (one 128-row block), at most 256 VGPRs: two
// waves per SIMD where the 32-row kernels ran one. The waves of a SIMD (w and
// w + 4) hold strips i and 7 - i, whose causal work is equal; tiles come
// through two LDS stages of 64 rows (one barrier per two 32-row tiles), the
// next tiles' global loads sit between the first MFMAs, and every operand
// read from LDS is issued three MFMA groups ahead through a register ring.
// Layouts (lane l, g = l/16, i = l%16; register r of a 16x16 block is row
// 4g + r, column i):
//   dq:  S^T, dP^T blocks kb (keys 16kb..): k-step s pairs the dims 32g + s
//        (A: K or V rows from LDS, B: the lane's own Q (scaled) or dO);
//        dQ^T block 4h+e (dims 64h + 4i' + e) += K^T . dS^T over the keys
//        16kb + 4g + r (A: K[16kb+4g+r][64h+4i+e], B: the lane's dS register).
//   dkv: S, dP blocks qb (queries 16qb..): A: Q or dO rows from LDS, B: the
//        lane's own K (scaled) or V; dV^T and dK^T blocks += dO^T . P and
//        Q^T . dS over the queries 16qb + 4g + r.
// A lane's register r' of block 4h+e is then dim 64h + 16g + 4r' + e of its
// row, so results leave as float4 rows straight from the accumulators.
typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma16(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float quad_sum(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(c[0]) + __uint_as_float(c[1]);
}

// acc[blk] += X[16 blk + i][32g + s] . y[s] over s: the 2 x NS/4 float4
// operands of an LDS tile (row stride RS). Operands go in pairs (one per
// block, the same y), whose MFMAs alternate between the two accumulators (no
// MFMA waits on the one before it); a ring of four registers holds the pair
// in use and the next, the pair after that read as soon as a pair is used.
// The tile's next global loads (a lambda) are issued after the first pair.
template <int NS, int RS, int NLOAD, class Load>
__device__ __forceinline__ void rows_dot(const float *X, int i, int g, const float (&y)[NS],
                                         floatx4 (&acc)[2], Load &&load) {
    constexpr int N = 2 * (NS / 4);
    float4 ring[4];
    auto rd = [&](int e) __attribute__((always_inline)) {
        return reinterpret_cast<const float4 *>(X + (16 * (e & 1) + i) * RS + g * NS)[e >> 1];
    };
#pragma unroll
    for (int e = 0; e < 4; ++e) ring[e] = rd(e);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int t = 0; t < N / 2; ++t) {
        const float4 xa = ring[(2 * t) % 4], xb = ring[(2 * t + 1) % 4];
        acc[0] = mfma16(xa.x, y[4 * t + 0], acc[0]);
        acc[1] = mfma16(xb.x, y[4 * t + 0], acc[1]);
        acc[0] = mfma16(xa.y, y[4 * t + 1], acc[0]);
        acc[1] = mfma16(xb.y, y[4 * t + 1], acc[1]);
        acc[0] = mfma16(xa.z, y[4 * t + 2], acc[0]);
        acc[1] = mfma16(xb.z, y[4 * t + 2], acc[1]);
        acc[0] = mfma16(xa.w, y[4 * t + 3], acc[0]);
        acc[1] = mfma16(xb.w, y[4 * t + 3], acc[1]);
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
        if (2 * t + 4 < N) {
            ring[(2 * t) % 4] = rd(2 * t + 4);
            ring[(2 * t + 1) % 4] = rd(2 * t + 5);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
        if (NLOAD > 0 && t == 0) {
            load();
            __builtin_amdgcn_sched_group_barrier(0x020, NLOAD, 0);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
}

// acc[4h+e] += Y[16(j/4) + 4g + j%4][64h + 4i + e] . b[j] over the 8 rows j of
// each lane group: 8 * NH float4 operands read RA ahead.
template <int NH, int RS, int RA>
__device__ __forceinline__ void cols_acc(const float *Y, int i, int g, const float (&bv)[8],
                                         floatx4 (&acc)[4 * NH]) {
    constexpr int N = 8 * NH;
    float4 ring[RA + 1];
    auto rd = [&](int e) __attribute__((always_inline)) {
        const int j = e / NH, h = e % NH;
        return reinterpret_cast<const float4 *>(Y + (16 * (j >> 2) + 4 * g + (j & 3)) * RS + 4 * i)[16 * h];
    };
#pragma unroll
    for (int e = 0; e < RA; ++e) ring[e] = rd(e);
    __builtin_amdgcn_sched_group_barrier(0x100, RA, 0);
#pragma unroll
    for (int e = 0; e < N; ++e) {
        if (e + RA < N) ring[(e + RA) % (RA + 1)] = rd(e + RA);
        const float4 y = ring[e % (RA + 1)];
        const int j = e / NH, h = e % NH;
        acc[4 * h + 0] = mfma16(y.x, bv[j], acc[4 * h + 0]);
        acc[4 * h + 1] = mfma16(y.y, bv[j], acc[4 * h + 1]);
        acc[4 * h + 2] = mfma16(y.z, bv[j], acc[4 * h + 2]);
        acc[4 * h + 3] = mfma16(y.w, bv[j], acc[4 * h + 3]);
        if (e + RA < N) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
}

template <int HD>
__global__ __launch_bounds__(512, 1) void attn_bwd_dq16_kernel(BwdP p) {
    static_assert(HD == 64 || HD == 128, "16-row strips take heads of 64 and 128");
    constexpr int NT = 512, NS = HD / 4, NH = HD / 64, KS = HD + 4, RA = 3;
    constexpr int F4 = 32 * HD / 4, PER = F4 / NT;  // float4s of K (and of V) per thread per tile
    // two stages of 64 keys: K rows then V rows; tile kt in stage (kt/2)&1, rows 32*(kt&1)..
    __shared__ __attribute__((aligned(16))) float smem[2 * 2 * 64 * KS];
    auto Ks = [&](int kt) { return smem + ((kt >> 1) & 1) * 128 * KS + (kt & 1) * 32 * KS; };
    auto Vs = [&](int kt) { return Ks(kt) + 64 * KS; };

    // the wave index through readfirstlane: uniform, so what derives from it
    // (strip, rows, tile counts, their tests) is scalar work in scalar registers
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g = lane >> 4, li = lane & 15;
    const int strip = wave < 4 ? wave : 11 - wave;
    const int head = blockIdx.x, b = blockIdx.y;
    const int qblk = p.nqb - 1 - (int)blockIdx.z;  // longest rows first
    const int kvh = head / (p.h / p.hkv);
    const int T = p.t;
    const int ntiles = min(qblk * 128 + 127, T - 1) / 32 + 1;
    const int q0 = qblk * 128 + strip * 16;
    const int my_tiles = q0 < T ? min(q0 + 15, T - 1) / 32 + 1 : 0;
    const int qi = q0 + li, qc = min(qi, T - 1);

    const float *Q = p.q + b * p.sqb + head * p.sqh;
    const float *K = p.k + b * p.skb + kvh * p.skh;
    const float *V = p.v + b * p.svb + kvh * p.svh;
    const float *O = p.o + b * p.sob + head * p.soh;
    const float *dO = p.dout + b * p.sob + head * p.soh;
    const int64_t rows = ((int64_t)b * p.h + head) * T;

    const float sc = p.scale * 1.4426950408889634f;  // S in log2 units
    float qr[NS], gr[NS];
    load_run<NS>(qr, Q + (int64_t)qc * p.sqt + g * NS);
#pragma unroll
    for (int s = 0; s < NS; ++s) qr[s] *= sc;
    load_run<NS>(gr, dO + (int64_t)qc * p.sot + g * NS);
    float dsum = 0.0f;
    {
        const float *orow = O + (int64_t)qc * p.sot + g * NS;
#pragma unroll
        for (int s = 0; s < NS; ++s) dsum += gr[s] * orow[s];
    }
    const float Dq = quad_sum(dsum);
    const float L2 = p.lse[rows + qc];
    if (g == 0 && qi < T) p.dvec[rows + qi] = Dq;

    // thread tid loads float4s tid (and tid + 512 at HD 128) of the K and V
    // tiles (keys past T read row T-1: finite values whose P is 0); named
    // registers, not an array, so they stay out of scratch memory
    float4 kreg0, vreg0, kreg1, vreg1;
    const int j0 = (4 * tid) / HD, c0 = (4 * tid) % HD;
    const int j1 = (4 * (tid + NT)) / HD, c1 = (4 * (tid + NT)) % HD;
    // 32-bit buffer offsets (the host keeps them below 2^31 bytes for these
    // kernels): the 64-bit address arithmetic was VALU work, whose cycles the
    // matrix core loses
    const __amdgpu_buffer_rsrc_t rk = rsrc_all(K), rv = rsrc_all(V);
    const uint32_t skt4 = 4u * (uint32_t)p.skt, svt4 = 4u * (uint32_t)p.svt;
    auto load_tile = [&](int kt) __attribute__((always_inline)) {
        const uint32_t key0 = (uint32_t)min(kt * 32 + j0, T - 1);
        kreg0 = ld4b(rk, key0 * skt4 + 4u * c0);
        vreg0 = ld4b(rv, key0 * svt4 + 4u * c0);
        if constexpr (PER > 1) {
            const uint32_t key1 = (uint32_t)min(kt * 32 + j1, T - 1);
            kreg1 = ld4b(rk, key1 * skt4 + 4u * c1);
            vreg1 = ld4b(rv, key1 * svt4 + 4u * c1);
        }
    };
    auto store_tile = [&](int kt) __attribute__((always_inline)) {
        *reinterpret_cast<float4 *>(Ks(kt) + j0 * KS + c0) = kreg0;
        *reinterpret_cast<float4 *>(Vs(kt) + j0 * KS + c0) = vreg0;
        if constexpr (PER > 1) {
            *reinterpret_cast<float4 *>(Ks(kt) + j1 * KS + c1) = kreg1;
            *reinterpret_cast<float4 *>(Vs(kt) + j1 * KS + c1) = vreg1;
        }
    };

    floatx4 dqa[4 * NH];
#pragma unroll
    for (int db = 0; db < 4 * NH; ++db) dqa[db] = floatx4{0.f, 0.f, 0.f, 0.f};

    load_tile(0);
    store_tile(0);
    if (ntiles > 1) {
        load_tile(1);
        store_tile(1);
    }
    __syncthreads();
    for (int kt = 0; kt < ntiles; ++kt) {
        const int nxt = min(kt + 2, ntiles - 1);  // the last steps reload a tile they never store
        if (kt < my_tiles) {
            floatx4 s[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
            floatx4 dp[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
            rows_dot<NS, KS, 2 * PER>(Ks(kt), li, g, qr, s, [&] { load_tile(nxt); });
            rows_dot<NS, KS, 0>(Vs(kt), li, g, gr, dp, [] {});
            const int k0 = kt * 32;
            const bool full = k0 + 31 <= q0 && k0 + 31 < T;
            // dS = P (dP - D); masked keys enter the exponential as -inf (P = 0)
            // through a select, on the diagonal and partial tiles only (written
            // as one select per key around the exponential, the compiler
            // branched around each exponential instead)
            float ds[8];
            if (full) {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    ds[j] = __builtin_amdgcn_exp2f(s[j >> 2][j & 3] - L2) * (dp[j >> 2][j & 3] - Dq);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int key = k0 + 16 * (j >> 2) + 4 * g + (j & 3);
                    const float x = key <= qi && key < T ? s[j >> 2][j & 3] - L2 : -INFINITY;
                    ds[j] = __builtin_amdgcn_exp2f(x) * (dp[j >> 2][j & 3] - Dq);
                }
            }
            cols_acc<NH, KS, RA>(Ks(kt), li, g, ds, dqa);
            if (kt == my_tiles - 1 && qi < T) {
                float *drow = p.dq + b * p.sqb + head * p.sqh + (int64_t)qi * p.sqt;
#pragma unroll
                for (int h = 0; h < NH; ++h)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        *reinterpret_cast<float4 *>(drow + 64 * h + 16 * g + 4 * r) =
                            make_float4(dqa[4 * h + 0][r] * p.scale, dqa[4 * h + 1][r] * p.scale,
                                        dqa[4 * h + 2][r] * p.scale, dqa[4 * h + 3][r] * p.scale);
            }
        } else {
            load_tile(nxt);
        }
        if (kt + 2 < ntiles) store_tile(kt + 2);
        if ((kt & 1) && kt + 1 < ntiles) __syncthreads();
    }
}

template <int HD>
__global__ __launch_bounds__(512, 1) void attn_bwd_dkv16_kernel(BwdP p) {
    static_assert(HD == 64 || HD == 128, "16-row strips take heads of 64 and 128");
    constexpr int NT = 512, NS = HD / 4, NH = HD / 64, KS = HD + 4, RA = 3;
    constexpr int F4 = 32 * HD / 4, PER = F4 / NT;
    // two stages of 64 queries: Q rows, dO rows, then lse2[64] and D[64];
    // query tile it in stage (it/2)&1, rows 32*(it&1)..
    constexpr int STAGE = 2 * 64 * KS + 128;
    __shared__ __attribute__((aligned(16))) float smem[2 * STAGE];
    auto Qs = [&](int it) { return smem + ((it >> 1) & 1) * STAGE + (it & 1) * 32 * KS; };
    auto Gs = [&](int it) { return Qs(it) + 64 * KS; };
    auto Ls = [&](int it) { return smem + ((it >> 1) & 1) * STAGE + 128 * KS + (it & 1) * 32; };
    auto Ds = [&](int it) { return Ls(it) + 64; };

    // the wave index through readfirstlane: uniform, so what derives from it
    // (strip, rows, tile counts, their tests) is scalar work in scalar registers
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int g = lane >> 4, li = lane & 15;
    const int strip = wave < 4 ? wave : 11 - wave;
    const int groups = p.h / p.hkv;
    const int kvh = p.part ? (int)blockIdx.x / groups : (int)blockIdx.x;
    const int g0 = p.part ? (int)blockIdx.x - kvh * groups : 0;
    const int ng = p.part ? 1 : groups;
    const int b = blockIdx.y;
    const int kblk = blockIdx.z;  // block 0 sees the most queries and starts first
    const int T = p.t;
    const int k_first = kblk * 128;
    const int k0 = k_first + strip * 16;
    const int kj = k0 + li, kc = min(kj, T - 1);
    const int qt_first = k_first / 32;
    const int per_head = (T + 31) / 32 - qt_first;
    const int total = ng * per_head;
    const int my_first = k0 / 32;  // earlier query tiles lie wholly above these keys

    const float *K = p.k + b * p.skb + kvh * p.skh;
    const float *V = p.v + b * p.svb + kvh * p.svh;
    const float sc = p.scale * 1.4426950408889634f;
    float kr[NS], vr[NS];
    load_run<NS>(kr, K + (int64_t)kc * p.skt + g * NS);
#pragma unroll
    for (int s = 0; s < NS; ++s) kr[s] *= sc;
    load_run<NS>(vr, V + (int64_t)kc * p.svt + g * NS);

    float4 qreg0, greg0, qreg1, greg1;  // named registers: no scratch array
    const int j0 = (4 * tid) / HD, c0 = (4 * tid) % HD;
    const int j1 = (4 * (tid + NT)) / HD, c1 = (4 * (tid + NT)) % HD;
    float lreg = 0.0f;
    // 32-bit buffer offsets from the batch element's first head (the host
    // keeps them below 2^31 bytes for these kernels)
    const __amdgpu_buffer_rsrc_t rq = rsrc_all(p.q + b * p.sqb), rg = rsrc_all(p.dout + b * p.sob);
    const uint32_t sqt4 = 4u * (uint32_t)p.sqt, sot4 = 4u * (uint32_t)p.sot;
    auto load_tile = [&](int it) __attribute__((always_inline)) {
        const int hh = it / per_head;
        const int qt = qt_first + (it - hh * per_head);
        const int head = kvh * groups + g0 + hh;
        const uint32_t qh4 = 4u * (uint32_t)(head * p.sqh), gh4 = 4u * (uint32_t)(head * p.soh);
        const uint32_t q0r = (uint32_t)min(qt * 32 + j0, T - 1);  // rows past T: finite, P = 0
        qreg0 = ld4b(rq, qh4 + q0r * sqt4 + 4u * c0);
        greg0 = ld4b(rg, gh4 + q0r * sot4 + 4u * c0);
        if constexpr (PER > 1) {
            const uint32_t q1r = (uint32_t)min(qt * 32 + j1, T - 1);
            qreg1 = ld4b(rq, qh4 + q1r * sqt4 + 4u * c1);
            greg1 = ld4b(rg, gh4 + q1r * sot4 + 4u * c1);
        }
        // lanes 0-31 of each wave fetch the tile's log-sum-exps, 32-63 its D
        const int q = min(qt * 32 + (tid & 31), T - 1);
        lreg = ((tid & 32) ? p.dvec : p.lse)[((int64_t)b * p.h + head) * T + q];
    };
    auto store_tile = [&](int it) __attribute__((always_inline)) {
        *reinterpret_cast<float4 *>(Qs(it) + j0 * KS + c0) = qreg0;
        *reinterpret_cast<float4 *>(Gs(it) + j0 * KS + c0) = greg0;
        if constexpr (PER > 1) {
            *reinterpret_cast<float4 *>(Qs(it) + j1 * KS + c1) = qreg1;
            *reinterpret_cast<float4 *>(Gs(it) + j1 * KS + c1) = greg1;
        }
        if (tid < 32)
            Ls(it)[tid] = lreg;
        else if (tid < 64)
            Ds(it)[tid - 32] = lreg;
    };

    floatx4 dka[4 * NH], dva[4 * NH];
#pragma unroll
    for (int db = 0; db < 4 * NH; ++db) {
        dka[db] = floatx4{0.f, 0.f, 0.f, 0.f};
        dva[db] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    load_tile(0);
    store_tile(0);
    if (total > 1) {
        load_tile(1);
        store_tile(1);
    }
    __syncthreads();
    for (int it = 0; it < total; ++it) {
        const int nxt = min(it + 2, total - 1);
        const int hh = it / per_head;
        const int qt = qt_first + (it - hh * per_head);
        if (qt >= my_first && k0 < T) {
            floatx4 s[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
            floatx4 dp[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
            rows_dot<NS, KS, 2 * PER>(Qs(it), li, g, kr, s, [&] { load_tile(nxt); });
            rows_dot<NS, KS, 0>(Gs(it), li, g, vr, dp, [] {});
            // the tile's lse2 and D for the queries 16qb + 4g + r of this lane
            const float4 l0 = *reinterpret_cast<const float4 *>(Ls(it) + 4 * g);
            const float4 l1 = *reinterpret_cast<const float4 *>(Ls(it) + 16 + 4 * g);
            const float4 d0 = *reinterpret_cast<const float4 *>(Ds(it) + 4 * g);
            const float4 d1 = *reinterpret_cast<const float4 *>(Ds(it) + 16 + 4 * g);
            const float lv[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
            const float dv8[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
            const bool full = qt * 32 >= k0 + 15 && qt * 32 + 31 < T && k0 + 15 < T;
            // masked queries enter the exponential as -inf (P = 0) through a
            // select, on the diagonal and partial tiles only
            float pv[8], ds[8];
            if (full) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    pv[j] = __builtin_amdgcn_exp2f(s[j >> 2][j & 3] - lv[j]);
                    ds[j] = pv[j] * (dp[j >> 2][j & 3] - dv8[j]);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int q = qt * 32 + 16 * (j >> 2) + 4 * g + (j & 3);
                    const float x = kj <= q && q < T && kj < T ? s[j >> 2][j & 3] - lv[j] : -INFINITY;
                    pv[j] = __builtin_amdgcn_exp2f(x);
                    ds[j] = pv[j] * (dp[j >> 2][j & 3] - dv8[j]);
                }
            }
            cols_acc<NH, KS, RA>(Gs(it), li, g, pv, dva);
            cols_acc<NH, KS, RA>(Qs(it), li, g, ds, dka);
        } else {
            load_tile(nxt);
        }
        if (it + 2 < total) store_tile(it + 2);
        if ((it & 1) && it + 1 < total) __syncthreads();
    }

    if (k0 < T && kj < T) {
        float *dkrow, *dvrow;
        if (p.part) {
            const int64_t plane = (int64_t)gridDim.y * p.h * T * HD;
            dkrow = p.part + ((int64_t)b * p.h + blockIdx.x) * T * HD + (int64_t)kj * HD;
            dvrow = dkrow + plane;
        } else {
            dkrow = p.dk + b * p.skb + kvh * p.skh + (int64_t)kj * p.skt;
            dvrow = p.dv + b * p.svb + kvh * p.svh + (int64_t)kj * p.svt;
        }
#pragma unroll
        for (int h = 0; h < NH; ++h)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                *reinterpret_cast<float4 *>(dkrow + 64 * h + 16 * g + 4 * r) =
                    make_float4(dka[4 * h + 0][r] * p.scale, dka[4 * h + 1][r] * p.scale,
                                dka[4 * h + 2][r] * p.scale, dka[4 * h + 3][r] * p.scale);
                *reinterpret_cast<float4 *>(dvrow + 64 * h + 16 * g + 4 * r) =
                    make_float4(dva[4 * h + 0][r], dva[4 * h + 1][r], dva[4 * h + 2][r],
                                dva[4 * h + 3][r]);
            }
    }
}

// ---- small grids ----------------------------------------------------------
// When the 128-row blocks leave CUs idle and the head is at most 64 wide (the
// tiny preset: 4 heads x 8 sequences of 256 rows give 64 workgroups), each
// workgroup owns one 32-row strip (dq: queries; dkv: keys) and its 4 waves
// take the key tiles (dq) or query tiles (dkv) round-robin, reading every
// operand straight from memory into the MFMA layouts (no LDS staging, no
// barrier per tile). The products, the masks and the arithmetic are those of
// the kernels above; the 4 partial accumulators are then summed through LDS
// in wave order (deterministic) and written as rows.

template <int HD>
__global__ __launch_bounds__(256) void attn_bwd_dq_split_kernel(BwdP p) {
    constexpr int NS = HD / 2, NDB = (HD + 31) / 32, OS = HD + 1;
    __shared__ float red[3][NDB * 16][64];
    __shared__ float Os[32 * OS];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lq = lane & 31, lh = lane >> 5;
    const int head = blockIdx.x, b = blockIdx.y;
    const int T = p.t;
    const int nstrips = (T + 31) / 32;
    const int strip = nstrips - 1 - (int)blockIdx.z;  // longest rows first
    const int kvh = head / (p.h / p.hkv);
    const int q0 = strip * 32;
    const int ntiles = strip + 1;  // key tiles 0 .. strip
    const int qi = q0 + lq;
    const int qc = min(qi, T - 1);

    const float *Q = p.q + b * p.sqb + head * p.sqh;
    const float *K = p.k + b * p.skb + kvh * p.skh;
    const float *V = p.v + b * p.svb + kvh * p.svh;
    const float *O = p.o + b * p.sob + head * p.soh;
    const float *dO = p.dout + b * p.sob + head * p.soh;
    const int64_t rows = ((int64_t)b * p.h + head) * T;

    const float sc = p.scale * 1.4426950408889634f;
    float qr[NS], gr[NS];
    load_run<NS>(qr, Q + (int64_t)qc * p.sqt + lh * NS);
#pragma unroll
    for (int s = 0; s < NS; ++s) qr[s] *= sc;
    load_run<NS>(gr, dO + (int64_t)qc * p.sot + lh * NS);
    float dsum = 0.0f;
    {
        const float *orow = O + (int64_t)qc * p.sot + lh * NS;
#pragma unroll
        for (int s = 0; s < NS; ++s) dsum += gr[s] * orow[s];
    }
    dsum += __shfl_xor(dsum, 32, 64);
    const float Dq = dsum;
    const float L2 = p.lse[rows + qc];
    if (wave == 0 && lh == 0 && qi < T) p.dvec[rows + qi] = Dq;

    floatx16 dq[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) dq[db][r] = 0.0f;
    for (int kt = wave; kt < ntiles; kt += 4) {
        const int k0 = kt * 32;
        // keys past T read row T-1 (finite values whose P is 0)
        const int key_l = min(k0 + lq, T - 1);
        floatx16 s0, s1, g0, g1;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s0[r] = 0.0f;
            s1[r] = 0.0f;
            g0[r] = 0.0f;
            g1[r] = 0.0f;
        }
        dot_chains<NS>(K + (int64_t)key_l * p.skt + lh * NS, qr, s0, s1);
        dot_chains<NS>(V + (int64_t)key_l * p.svt + lh * NS, gr, g0, g1);
        const bool full = k0 + 31 <= q0 && k0 + 31 < T;
        float ds[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = k0 + 8 * (r >> 2) + 4 * lh + (r & 3);
            // masked keys enter the exponential as -inf (a select; P = 0)
            const float pr = __builtin_amdgcn_exp2f(full || (key <= qi && key < T) ? (s0[r] + s1[r]) - L2 : -INFINITY);
            ds[r] = pr * ((g0[r] + g1[r]) - Dq);
        }
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const int key = min(k0 + 8 * (s >> 2) + 4 * lh + (s & 3), T - 1);
            float a[NDB];
            read_dims<HD, NDB>(a, K + (int64_t)key * p.skt, lq);
#pragma unroll
            for (int db = 0; db < NDB; ++db) dq[db] = mfma(a[db], ds[s], dq[db]);
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) red[wave - 1][db * 16 + r][lane] = dq[db][r];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float v = dq[db][r];
#pragma unroll
                for (int w = 0; w < 3; ++w) v += red[w][db * 16 + r][lane];
                const int i = 8 * (r >> 2) + 4 * lh + (r & 3);
                const int d = NDB * i + db;
                if (d < HD) Os[lq * OS + d] = v * p.scale;
            }
    }
    __syncthreads();
    for (int idx = tid; idx < 32 * HD; idx += 256) {
        const int j = idx / HD, c = idx - j * HD;
        const int q = q0 + j;
        if (q < T) p.dq[b * p.sqb + head * p.sqh + (int64_t)q * p.sqt + c] = Os[j * OS + c];
    }
}

template <int HD>
__global__ __launch_bounds__(256) void attn_bwd_dkv_split_kernel(BwdP p) {
    constexpr int NS = HD / 2, NDB = (HD + 31) / 32, OS = HD + 1;
    __shared__ float red[3][NDB * 16][64];
    __shared__ float Os[32 * OS];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lq = lane & 31, lh = lane >> 5;
    const int groups = p.h / p.hkv;
    const int kvh = blockIdx.x, b = blockIdx.y;
    const int kstrip = blockIdx.z;  // strip 0 sees the most queries and starts first
    const int T = p.t;
    const int k0 = kstrip * 32;
    const int kj = k0 + lq;
    const int kc = min(kj, T - 1);
    const int nqt = (T + 31) / 32;
    const int per_head = nqt - kstrip;  // query tiles at or after the keys
    const int total = groups * per_head;

    const float *K = p.k + b * p.skb + kvh * p.skh;
    const float *V = p.v + b * p.svb + kvh * p.svh;
    const float sc = p.scale * 1.4426950408889634f;
    float kr[NS], vr[NS];
    load_run<NS>(kr, K + (int64_t)kc * p.skt + lh * NS);
#pragma unroll
    for (int s = 0; s < NS; ++s) kr[s] *= sc;
    load_run<NS>(vr, V + (int64_t)kc * p.svt + lh * NS);

    floatx16 dk[NDB], dv[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            dk[db][r] = 0.0f;
            dv[db][r] = 0.0f;
        }
    for (int it = wave; it < total; it += 4) {
        const int g = it / per_head;
        const int qt = kstrip + (it - g * per_head);
        const int head = kvh * groups + g;
        const float *Qh = p.q + b * p.sqb + head * p.sqh;
        const float *Gh = p.dout + b * p.sob + head * p.soh;
        // rows past T read row T-1 (finite; their P is 0)
        const int qrow = min(qt * 32 + lq, T - 1);
        // lanes 0-31 hold the tile's log-sum-exps, 32-63 its D values
        const float lreg = ((lh != 0) ? p.dvec : p.lse)[((int64_t)b * p.h + head) * T + qrow];
        floatx16 s0, s1, g0, g1;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            s0[r] = 0.0f;
            s1[r] = 0.0f;
            g0[r] = 0.0f;
            g1[r] = 0.0f;
        }
        dot_chains<NS>(Qh + (int64_t)qrow * p.sqt + lh * NS, kr, s0, s1);
        dot_chains<NS>(Gh + (int64_t)qrow * p.sot + lh * NS, vr, g0, g1);
        const bool full = qt * 32 >= k0 + 31 && qt * 32 + 31 < T && k0 + 31 < T;
        float pv[16], ds[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = 8 * (r >> 2) + 4 * lh + (r & 3);
            const int q = qt * 32 + row;
            const float lrow = __shfl(lreg, row, 64), drow = __shfl(lreg, 32 + row, 64);
            const float pr = __builtin_amdgcn_exp2f(full || (kj <= q && q < T && kj < T) ? (s0[r] + s1[r]) - lrow : -INFINITY);
            pv[r] = pr;
            ds[r] = pr * ((g0[r] + g1[r]) - drow);
        }
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const int q = min(qt * 32 + 8 * (s >> 2) + 4 * lh + (s & 3), T - 1);
            float ag[NDB], aq[NDB];
            read_dims<HD, NDB>(ag, Gh + (int64_t)q * p.sot, lq);
            read_dims<HD, NDB>(aq, Qh + (int64_t)q * p.sqt, lq);
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
                dv[db] = mfma(ag[db], pv[s], dv[db]);
                dk[db] = mfma(aq[db], ds[s], dk[db]);
            }
        }
    }
    // dK = scale * dK^T and dV = dV^T: the waves' partials summed in wave
    // order, through LDS as [key][d], then rows.
    for (int which = 0; which < 2; ++which) {
        if (wave > 0) {
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    red[wave - 1][db * 16 + r][lane] = which == 0 ? dk[db][r] : dv[db][r];
        }
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float v = which == 0 ? dk[db][r] : dv[db][r];
#pragma unroll
                    for (int w = 0; w < 3; ++w) v += red[w][db * 16 + r][lane];
                    const int i = 8 * (r >> 2) + 4 * lh + (r & 3);
                    const int d = NDB * i + db;
                    if (d < HD) Os[lq * OS + d] = which == 0 ? v * p.scale : v;
                }
        }
        __syncthreads();
        float *dst = which == 0 ? p.dk + b * p.skb + kvh * p.skh : p.dv + b * p.svb + kvh * p.svh;
        const int64_t st = which == 0 ? p.skt : p.svt;
        for (int idx = tid; idx < 32 * HD; idx += 256) {
            const int j = idx / HD, c = idx - j * HD;
            const int key = k0 + j;
            if (key < T) dst[(int64_t)key * st + c] = Os[j * OS + c];
        }
        __syncthreads();
    }
}

// dK, dV of kv head j = the sum of its group's partials in head order.
// One thread per 4 consecutive dims of one (batch, kv head, key).
__global__ __launch_bounds__(256) void dkv_group_sum_kernel(const float *__restrict__ part, int b,
                                                            int h, int hkv, int t, int hd,
                                                            float *dk, int64_t skb, int64_t skh,
                                                            int64_t skt, float *dv, int64_t svb,
                                                            int64_t svh, int64_t svt) {
    const int groups = h / hkv, q4 = hd / 4;
    const int64_t n = (int64_t)b * hkv * t * q4;
    const int64_t plane = (int64_t)b * h * t * hd;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int c = (int)(i % q4) * 4;
        const int64_t r = i / q4;
        const int key = (int)(r % t);
        const int64_t bk = r / t;
        const int kvh = (int)(bk % hkv), bb = (int)(bk / hkv);
        const float *src = part + (((int64_t)bb * h + (int64_t)kvh * groups) * t + key) * hd + c;
        float4 a = *reinterpret_cast<const float4 *>(src);
        float4 v = *reinterpret_cast<const float4 *>(src + plane);
        for (int g = 1; g < groups; ++g) {
            const float4 x = *reinterpret_cast<const float4 *>(src + (int64_t)g * t * hd);
            const float4 y = *reinterpret_cast<const float4 *>(src + plane + (int64_t)g * t * hd);
            a = make_float4(a.x + x.x, a.y + x.y, a.z + x.z, a.w + x.w);
            v = make_float4(v.x + y.x, v.y + y.y, v.z + y.z, v.w + y.w);
        }
        *reinterpret_cast<float4 *>(dk + bb * skb + kvh * skh + (int64_t)key * skt + c) = a;
        *reinterpret_cast<float4 *>(dv + bb * svb + kvh * svh + (int64_t)key * svt + c) = v;
    }
}

bool al16(const void *ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

}  // namespace

int64_t attention_backward_scratch_floats(int64_t b, int64_t h, int64_t hkv, int64_t t,
                                          int64_t hd) {
    return h > hkv ? 2 * b * h * t * hd : 0;
}

namespace {

// The kernels on heads of a width they take, scores scaled by `scale`; no
// rotation (the caller's).
void backward_kernels(Context &ctx, const AttnBwdDesc &d, float scale) {
    const int64_t strides[] = {d.sqb, d.sqh, d.sqt, d.skb, d.skh, d.skt,
                               d.svb, d.svh, d.svt, d.sob, d.soh, d.sot};
    for (int64_t s : strides)
        if (s % 4) fail(MMH_ERR_SHAPE, "attention backward: strides must be multiples of 4 floats");
    const void *ptrs[] = {d.q, d.k, d.v, d.o, d.dout, d.dq, d.dk, d.dv};
    for (const void *ptr : ptrs)
        if (!al16(ptr)) fail(MMH_ERR_ARGUMENT, "attention backward: buffers must be 16-byte aligned");
    if (d.scratch && !al16(d.scratch))
        fail(MMH_ERR_ARGUMENT, "attention backward: the partials scratch must be 16-byte aligned");
    BwdP p{};
    p.q = d.q;
    p.k = d.k;
    p.v = d.v;
    p.o = d.o;
    p.dout = d.dout;
    p.lse = d.lse;
    p.dq = d.dq;
    p.dk = d.dk;
    p.dv = d.dv;
    p.dvec = d.dvec;
    p.sqb = d.sqb; p.sqh = d.sqh; p.sqt = d.sqt;
    p.skb = d.skb; p.skh = d.skh; p.skt = d.skt;
    p.svb = d.svb; p.svh = d.svh; p.svt = d.svt;
    p.sob = d.sob; p.soh = d.soh; p.sot = d.sot;
    p.h = (int)d.h;
    p.hkv = (int)d.hkv;
    p.t = (int)d.t;
    p.nqb = (int)((d.t + 127) / 128);
    p.nkb = p.nqb;
    p.scale = scale;
    // GQA: per-query-head partials when the caller gave room for them and the
    // head is wide enough for the float4 sum (hd >= 4 always holds).
    // small grids (fewer 128-row blocks than CUs, heads up to 64 wide): the
    // strip kernels, which need no partials (a group's heads are summed in
    // one workgroup)
    const int cus = ctx.cu_count > 0 ? ctx.cu_count : 256;
    const bool split = d.hd <= 64 && d.b * d.h * p.nqb < cus;
    p.part = !split && d.h > d.hkv && d.scratch ? d.scratch : nullptr;
    const dim3 gq((unsigned)d.h, (unsigned)d.b, (unsigned)p.nqb);
    const dim3 gk((unsigned)(p.part ? d.h : d.hkv), (unsigned)d.b, (unsigned)p.nkb);
    const unsigned strips = (unsigned)((d.t + 31) / 32);
    const dim3 sq((unsigned)d.h, (unsigned)d.b, strips), sk((unsigned)d.hkv, (unsigned)d.b, strips);
    const dim3 blk(256);
    // the 16-row kernels read q, k, v and dout through 32-bit byte offsets
    // from a batch element's first row (and head)
    const int64_t span = d.t * std::max(std::max(d.sqt, d.skt), std::max(d.svt, d.sot)) +
                         d.h * std::max(d.sqh, d.soh) + d.hd;
    const bool off32 = span < (int64_t(1) << 29);
#define MMH_BWD_CASE(HD)                                                                   \
    case HD:                                                                               \
        if constexpr (HD <= 64) {                                                          \
            if (split) {                                                                   \
                hipLaunchKernelGGL((attn_bwd_dq_split_kernel<HD>), sq, blk, 0, ctx.stream, p); \
                hipLaunchKernelGGL((attn_bwd_dkv_split_kernel<HD>), sk, blk, 0, ctx.stream, p); \
                break;                                                                     \
            }                                                                              \
        }                                                                                  \
        if constexpr (HD == 64 || HD == 128) {                                             \
          if (off32) {                                                                     \
            hipLaunchKernelGGL((attn_bwd_dq16_kernel<HD>), gq, dim3(512), 0, ctx.stream, p);  \
            hipLaunchKernelGGL((attn_bwd_dkv16_kernel<HD>), gk, dim3(512), 0, ctx.stream, p); \
            break;                                                                         \
          }                                                                                \
        }                                                                                  \
        hipLaunchKernelGGL((attn_bwd_dq_kernel<HD>), gq, blk, 0, ctx.stream, p);           \
        hipLaunchKernelGGL((attn_bwd_dkv_kernel<HD>), gk, blk, 0, ctx.stream, p);          \
        break;
    switch (d.hd) {
        MMH_BWD_CASE(4)
        MMH_BWD_CASE(8)
        MMH_BWD_CASE(16)
        MMH_BWD_CASE(32)
        MMH_BWD_CASE(64)
        MMH_BWD_CASE(128)
    }
#undef MMH_BWD_CASE
    check_hip(hipGetLastError(), "attention backward launch");
    if (p.part) {
        const int64_t n4 = d.b * d.hkv * d.t * (d.hd / 4);
        const unsigned blocks = (unsigned)std::min<int64_t>((n4 + 255) / 256, 4096);
        hipLaunchKernelGGL(dkv_group_sum_kernel, dim3(blocks), dim3(256), 0, ctx.stream, p.part,
                           (int)d.b, (int)d.h, (int)d.hkv, (int)d.t, (int)d.hd, d.dk, d.skb,
                           d.skh, d.skt, d.dv, d.svb, d.svh, d.svt);
        check_hip(hipGetLastError(), "dk/dv group sum launch");
    }
}

}  // namespace

void attention_backward(Context &ctx, const AttnBwdDesc &d) {
    if (d.b <= 0 || d.h <= 0 || d.hkv <= 0 || d.t <= 0 || d.hd <= 0)
        fail(MMH_ERR_SHAPE, "attention backward: empty shape");
    if (d.h % d.hkv != 0)
        fail(MMH_ERR_SHAPE, "attention backward: n_heads is not a multiple of n_kv_heads");
    if (d.b > 65535 || d.h > 65535 || d.t > 0x3fffffff)
        fail(MMH_ERR_SHAPE, "attention backward: shape too large");
    const int64_t hp = kernel_head(d.hd);
    if (hp == 0 || (!native_head(d.hd) && d.hd % 2))
        fail(MMH_ERR_SHAPE, "attention backward: head_dim must be 4, 8, 16, 32, 64 or 128, or "
                            "even and below 128");
    const float scale = 1.0f / sqrtf((float)d.hd);  // attention.rs:82
    if (native_head(d.hd)) {
        backward_kernels(ctx, d, scale);
    } else {
        // Other even widths on the next kernel width (as the forward): q, k,
        // v, o and dO copied into heads of hp columns, zero beyond hd (zero
        // columns change no score, no dP and no rowsum(dO * O)), the
        // gradients' columns below hd copied back; the GQA partials in the
        // same buffer.
        const int64_t nq = d.b * d.h * d.t * hp, nk = d.b * d.hkv * d.t * hp;
        const int64_t part = d.h > d.hkv ? 2 * nq : 0;
        float *qp = static_cast<float *>(
            ctx.workspace(Context::kPadSlot, (size_t)(4 * nq + 4 * nk + part) * 4));
        float *op = qp + nq, *gp = op + nq, *kp = gp + nq, *vp = kp + nk, *dqp = vp + nk,
              *dkp = dqp + nq, *dvp = dkp + nk, *pp = dvp + nk;
        launch_pad_heads(ctx, d.q, d.sqb, d.sqh, d.sqt, d.b, d.h, d.t, d.hd, qp, hp);
        launch_pad_heads(ctx, d.k, d.skb, d.skh, d.skt, d.b, d.hkv, d.t, d.hd, kp, hp);
        launch_pad_heads(ctx, d.v, d.svb, d.svh, d.svt, d.b, d.hkv, d.t, d.hd, vp, hp);
        launch_pad_heads(ctx, d.o, d.sob, d.soh, d.sot, d.b, d.h, d.t, d.hd, op, hp);
        launch_pad_heads(ctx, d.dout, d.sob, d.soh, d.sot, d.b, d.h, d.t, d.hd, gp, hp);
        AttnBwdDesc e = d;
        e.q = qp;
        e.k = kp;
        e.v = vp;
        e.o = op;
        e.dout = gp;
        e.dq = dqp;
        e.dk = dkp;
        e.dv = dvp;
        e.sqb = e.sob = d.h * d.t * hp;
        e.sqh = e.soh = d.t * hp;
        e.sqt = e.sot = hp;
        e.skb = e.svb = d.hkv * d.t * hp;
        e.skh = e.svh = d.t * hp;
        e.skt = e.svt = hp;
        e.hd = hp;
        e.cos_t = e.sin_t = nullptr;
        e.scratch = part ? pp : nullptr;
        backward_kernels(ctx, e, scale);
        launch_unpad_heads(ctx, dqp, hp, d.b, d.h, d.t, d.hd, d.dq, d.sqb, d.sqh, d.sqt);
        launch_unpad_heads(ctx, dkp, hp, d.b, d.hkv, d.t, d.hd, d.dk, d.skb, d.skh, d.skt);
        launch_unpad_heads(ctx, dvp, hp, d.b, d.hkv, d.t, d.hd, d.dv, d.svb, d.svh, d.svt);
    }
    // RoPE backward on dq and dk
    if (d.cos_t)
        rope_qk(ctx, d.dq, d.dk, d.sqb, d.sqh, d.sqt, d.skb, d.skh, d.skt, d.b, d.h, d.hkv, d.t,
                d.hd, d.cos_t, d.sin_t, true);
}

}  // namespace mmh
