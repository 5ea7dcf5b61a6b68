// Fused causal attention on CDNA4 matrix cores (fp32 MFMA 32x32x2), replacing
// the reference's materialised path (midman-nn/src/attention.rs:79-101,146-170):
// repeat_interleave of K/V, Q.K^T, scale, additive -1e9 mask, softmax, P.V.
//
// One wave64 owns 32 query rows of one (batch, head) and walks the key blocks
// of 32 up to the diagonal with an online softmax, so no [T,T] tensor exists.
// It computes the transposed products so that every per-query quantity lives in
// the lane that owns the query:
//   S^T[key][q] = K_blk . Q^T   (A = K from LDS, B = Q from registers)
//   O^T[d][q]  += V^T . P^T     (A = V from LDS, B = P straight from the S^T
//                                accumulators, no LDS round trip)
// With the MFMA layout (lane l: column l%32; register r: row
// 8*(r/4) + 4*(l/32) + r%4), query q = l%32 is fixed per lane in both
// products, so the row max/sum need one cross-lane exchange (lanes l, l^32)
// and the rescale of O is a per-lane scalar.
//
// RoPE (rope.rs:28-32) is applied in registers to Q and while staging K into
// LDS, with explicitly rounded multiplies and adds, so rotated values equal
// the reference's bit for bit. The score scale is applied after the dot
// product as attention.rs:83 does. Keys above the diagonal are skipped: the
// reference's -1e9 mask gives them exp(.) == 0 exactly. Query head j reads kv
// head j / (H/Hkv) (repeat_interleave, ops_shape.rs:192-200).
#include "mmh_internal.h"

namespace mmh {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

struct AttnP {
    const float *q, *k, *v;
    float *out;
    int64_t sqb, sqh, sqt, skb, skh, skt, svb, svh, svt, sob, soh, sot;
    int h, hkv, t, nqb;
    float scale;
    const float *cos_t, *sin_t;
};

template <int HD, bool ROPE>
__global__ __launch_bounds__(64) void attn_fwd_kernel(AttnP p) {
    constexpr int HALF = HD / 2;
    constexpr int NS = HD / 2;            // MFMA k-steps over the head dim
    constexpr int NDB = (HD + 31) / 32;   // 32-wide blocks of the head dim
    __shared__ float Ks[32][HD + 1];
    __shared__ float Vs[32][HD];

    const int lane = threadIdx.x;
    const int lq = lane & 31, lh = lane >> 5;
    const int head = blockIdx.x, b = blockIdx.y;
    const int qb = p.nqb - 1 - (int)blockIdx.z;  // longest rows first
    const int kvh = head / (p.h / p.hkv);
    const int T = p.t;
    const int q0 = qb * 32;

    const float *Q = p.q + b * p.sqb + head * p.sqh;
    const float *K = p.k + b * p.skb + kvh * p.skh;
    const float *V = p.v + b * p.svb + kvh * p.svh;

    // ---- stage Q through LDS, pick this lane's operand values, rotate ----
    for (int idx = lane; idx < 32 * HD; idx += 64) {
        const int j = idx / HD, c = idx - j * HD;
        Ks[j][c] = (q0 + j < T) ? Q[(int64_t)(q0 + j) * p.sqt + c] : 0.0f;
    }
    __syncthreads();
    float qr[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) qr[s] = Ks[lq][2 * s + lh];
    __syncthreads();
    if (ROPE) {
        const int pos = min(q0 + lq, T - 1);
        float rot[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int pd = 2 * s + lh;
            if (pd < HALF) {
                const float cs = p.cos_t[pos * HALF + pd], sn = p.sin_t[pos * HALF + pd];
                rot[s] = __fsub_rn(__fmul_rn(qr[s], cs), __fmul_rn(qr[s + HALF / 2], sn));
            } else {
                const int pp = pd - HALF;
                const float cs = p.cos_t[pos * HALF + pp], sn = p.sin_t[pos * HALF + pp];
                rot[s] = __fadd_rn(__fmul_rn(qr[s], cs), __fmul_rn(qr[s - HALF / 2], sn));
            }
        }
#pragma unroll
        for (int s = 0; s < NS; ++s) qr[s] = rot[s];
    }

    floatx16 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    const int qi = q0 + lq;

    for (int kb = 0; kb <= qb; ++kb) {
        const int k0 = kb * 32;
        // K block (rotated) and V block into LDS.
        for (int idx = lane; idx < 32 * HALF; idx += 64) {
            const int j = idx / HALF, c = idx - j * HALF;
            const int key = k0 + j;
            float y1 = 0.0f, y2 = 0.0f;
            if (key < T) {
                const float x1 = K[(int64_t)key * p.skt + c], x2 = K[(int64_t)key * p.skt + c + HALF];
                if (ROPE) {
                    const float cs = p.cos_t[key * HALF + c], sn = p.sin_t[key * HALF + c];
                    y1 = __fsub_rn(__fmul_rn(x1, cs), __fmul_rn(x2, sn));
                    y2 = __fadd_rn(__fmul_rn(x2, cs), __fmul_rn(x1, sn));
                } else {
                    y1 = x1;
                    y2 = x2;
                }
            }
            Ks[j][c] = y1;
            Ks[j][c + HALF] = y2;
        }
        for (int idx = lane; idx < 32 * HD; idx += 64) {
            const int j = idx / HD, c = idx - j * HD;
            Vs[j][c] = (k0 + j < T) ? V[(int64_t)(k0 + j) * p.svt + c] : 0.0f;
        }
        __syncthreads();

        // S^T = K . Q^T over the head dim.
        floatx16 sacc;
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[r] = 0.0f;
#pragma unroll
        for (int s = 0; s < NS; ++s)
            sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(Ks[lq][2 * s + lh], qr[s], sacc, 0, 0, 0);

        // Scale, mask, online softmax for query qi (shared by lanes l, l^32).
        float pv[16];
        float mloc = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = k0 + 8 * (r >> 2) + 4 * lh + (r & 3);
            const float sv = __fmul_rn(sacc[r], p.scale);
            const bool ok = key <= qi && key < T;
            pv[r] = ok ? sv : -INFINITY;
            mloc = fmaxf(mloc, pv[r]);
        }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
        const float m_new = fmaxf(m_run, mloc);
        const float alpha = expf(m_run - m_new);
        float lsum = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            pv[r] = expf(pv[r] - m_new);
            lsum += pv[r];
        }
        lsum += __shfl_xor(lsum, 32, 64);
        l_run = l_run * alpha + lsum;
        m_run = m_new;

        // O^T += V^T . P^T; P^T's operand is pv[s] in place.
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
#pragma unroll
            for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
            const int dcol = db * 32 + lq;
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                const int key = 8 * (s >> 2) + 4 * lh + (s & 3);
                const float a = (HD >= 32 || dcol < HD) ? Vs[key][dcol < HD ? dcol : 0] : 0.0f;
                o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, pv[s], o[db], 0, 0, 0);
            }
        }
        __syncthreads();
    }

    if (qi < T) {
        const float inv = 1.0f / l_run;
        float *O = p.out + b * p.sob + head * p.soh + (int64_t)qi * p.sot;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int d = db * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                if (d < HD) O[d] = o[db][r] * inv;
            }
    }
}

template <int HD>
void launch_hd(Context &ctx, const AttnP &p, dim3 grid, bool rope) {
    if (rope)
        hipLaunchKernelGGL((attn_fwd_kernel<HD, true>), grid, dim3(64), 0, ctx.stream, p);
    else
        hipLaunchKernelGGL((attn_fwd_kernel<HD, false>), grid, dim3(64), 0, ctx.stream, p);
}

}  // namespace

void attention(Context &ctx, const AttnDesc &d) {
    if (d.b <= 0 || d.h <= 0 || d.hkv <= 0 || d.t <= 0 || d.hd <= 0)
        fail(MMH_ERR_SHAPE, "attention: empty shape");
    if (d.h % d.hkv != 0) fail(MMH_ERR_SHAPE, "attention: n_heads is not a multiple of n_kv_heads");
    if (d.b > 65535 || d.h > 0x7fffffff || d.t > 0x3fffffff)
        fail(MMH_ERR_SHAPE, "attention: shape too large");
    AttnP p{};
    p.q = d.q;
    p.k = d.k;
    p.v = d.v;
    p.out = d.out;
    p.sqb = d.sqb; p.sqh = d.sqh; p.sqt = d.sqt;
    p.skb = d.skb; p.skh = d.skh; p.skt = d.skt;
    p.svb = d.svb; p.svh = d.svh; p.svt = d.svt;
    p.sob = d.sob; p.soh = d.soh; p.sot = d.sot;
    p.h = (int)d.h;
    p.hkv = (int)d.hkv;
    p.t = (int)d.t;
    p.nqb = (int)((d.t + 31) / 32);
    p.scale = 1.0f / sqrtf((float)d.hd);  // attention.rs:82
    p.cos_t = d.cos_t;
    p.sin_t = d.sin_t;
    const bool rope = d.cos_t != nullptr;
    dim3 grid((unsigned)d.h, (unsigned)d.b, (unsigned)p.nqb);
    switch (d.hd) {
        case 4: launch_hd<4>(ctx, p, grid, rope); break;
        case 8: launch_hd<8>(ctx, p, grid, rope); break;
        case 16: launch_hd<16>(ctx, p, grid, rope); break;
        case 32: launch_hd<32>(ctx, p, grid, rope); break;
        case 64: launch_hd<64>(ctx, p, grid, rope); break;
        case 128: launch_hd<128>(ctx, p, grid, rope); break;
        default: fail(MMH_ERR_SHAPE, "attention: head_dim must be 4, 8, 16, 32, 64 or 128");
    }
    check_hip(hipGetLastError(), "attention launch");
}

}  // namespace mmh
