/*
 * mm_oracle.c -- CPU restatement of the midman-ai decoder path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and the CPU timing baseline.
 * The product never links or calls it. See mm_oracle.h for which check pins
 * which function.
 *
 * Build rules that make this a faithful restatement (the reference is Rust
 * built without FMA contraction or fast-math):
 *   -ffp-contract=off, no -ffast-math, glibc libm for expf/logf/powf and the
 *   f64 log/sqrt/sin/cos/pow the reference calls (rng.rs:78-82,
 *   rope.rs:73-77, ops_reduce.rs:112/256/257, ops_elementwise.rs:240/336).
 * Every per-element sum runs in the reference's order. Multi-threading splits
 * work by output rows (or by attention head), which never changes the order of
 * any element's sum, so the results are the same bits at any thread count.
 */
#include "mm_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* RNG: crates/midman-foundation/src/rng.rs                                  */
/* ------------------------------------------------------------------------ */

/* rng.rs:16-22 */
static uint64_t splitmix64(uint64_t *state) {
    *state += 0x9E3779B97F4A7C15ULL;
    uint64_t z = *state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

static inline uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

/* rng.rs:36-41 */
void mmo_rng_seed(mmo_rng *r, uint64_t seed) {
    uint64_t sm = seed;
    for (int i = 0; i < 4; i++) r->s[i] = splitmix64(&sm);
    r->has_spare = 0;
    r->spare = 0.0f;
}

/* rng.rs:44-55, xoshiro256** */
uint64_t mmo_rng_next_u64(mmo_rng *r) {
    uint64_t *s = r->s;
    const uint64_t result = rotl64(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return result;
}

/* rng.rs:58-60 */
float mmo_rng_next_f32(mmo_rng *r) {
    return (float)(mmo_rng_next_u64(r) >> 40) * (1.0f / 16777216.0f);
}

/* rng.rs:63-65 */
double mmo_rng_next_f64(mmo_rng *r) {
    return (double)(mmo_rng_next_u64(r) >> 11) * (1.0 / 9007199254740992.0);
}

/* rng.rs:78-83: one Box-Muller pair from two consecutive draws, u1 = 1 -
 * next_f64, u2 = next_f64; *c is the value returned, *s the cached spare. */
static void box_muller(uint64_t x1, uint64_t x2, float *c, float *s) {
    const double u1 = 1.0 - (double)(x1 >> 11) * (1.0 / 9007199254740992.0);
    const double u2 = (double)(x2 >> 11) * (1.0 / 9007199254740992.0);
    const double radius = sqrt(-2.0 * log(u1));
    const double theta = 6.283185307179586 * u2; /* std::f64::consts::TAU */
    *s = (float)(radius * sin(theta));
    *c = (float)(radius * cos(theta));
}

/* rng.rs:74-84, Box-Muller with a cached spare that persists across calls. */
float mmo_rng_normal(mmo_rng *r) {
    if (r->has_spare) {
        r->has_spare = 0;
        return r->spare;
    }
    const uint64_t x1 = mmo_rng_next_u64(r);
    const uint64_t x2 = mmo_rng_next_u64(r);
    float c;
    box_muller(x1, x2, &c, &r->spare);
    r->has_spare = 1;
    return c;
}

/* rng.rs:91-105, Lemire's nearly-divisionless method. */
uint64_t mmo_rng_below(mmo_rng *r, uint64_t n) {
    if (n == 0) return 0; /* the reference panics; callers never pass 0 */
    unsigned __int128 product = (unsigned __int128)mmo_rng_next_u64(r) * n;
    uint64_t low = (uint64_t)product;
    if (low < n) {
        const uint64_t threshold = (0 - n) % n;
        while (low < threshold) {
            product = (unsigned __int128)mmo_rng_next_u64(r) * n;
            low = (uint64_t)product;
        }
    }
    return (uint64_t)(product >> 64);
}

void mmo_rng_fork(mmo_rng *r, uint64_t stream, mmo_rng *out) {
    /* rng.rs:117-119: wrapping multiply by the golden-ratio constant, xor */
    mmo_rng_seed(out, mmo_rng_next_u64(r) ^ (stream * 0x9E3779B97F4A7C15ull));
}

void mmo_rng_shuffle_u64(mmo_rng *r, uint64_t *items, uint64_t n) {
    /* rng.rs:108-113 */
    for (uint64_t i = n ? n - 1 : 0; i >= 1; i--) {
        const uint64_t j = mmo_rng_below(r, i + 1);
        const uint64_t t = items[i];
        items[i] = items[j];
        items[j] = t;
    }
}

void mmo_permutation(uint64_t n, uint64_t seed, uint64_t epoch, uint64_t *out) {
    /* batch.rs:244-248 */
    mmo_rng base, f;
    for (uint64_t i = 0; i < n; i++) out[i] = i;
    mmo_rng_seed(&base, seed);
    mmo_rng_fork(&base, epoch, &f);
    mmo_rng_shuffle_u64(&f, out, n);
}

/* ------------------------------------------------------------------------ */
/* Config: crates/midman-model-config/src/config.rs, presets.rs              */
/* ------------------------------------------------------------------------ */

static int divides(int64_t a, int64_t b) { return b != 0 && (a / b) * b == a; }

/* config.rs:106-138 */
int32_t mmo_config_validate(const mmo_config *c) {
    if (!c) return MMO_ERR_ARGUMENT;
    if (c->vocab_size <= 0 || c->d_model <= 0 || c->n_layers <= 0 || c->n_heads <= 0 ||
        c->n_kv_heads <= 0 || c->d_ff <= 0 || c->max_seq_len <= 0)
        return MMO_ERR_CONFIG;
    if (!(isfinite(c->rope_theta) && c->rope_theta > 0.0f)) return MMO_ERR_CONFIG;
    if (!(isfinite(c->norm_eps) && c->norm_eps > 0.0f)) return MMO_ERR_CONFIG;
    if (!divides(c->d_model, c->n_heads)) return MMO_ERR_CONFIG;
    if (!divides(c->n_heads, c->n_kv_heads)) return MMO_ERR_CONFIG;
    if ((c->d_model / c->n_heads) & 1) return MMO_ERR_CONFIG;
    return MMO_OK;
}

/* config.rs:158-185 */
int64_t mmo_param_count(const mmo_config *c) {
    if (mmo_config_validate(c) != MMO_OK) return -1;
    const int64_t d = c->d_model, kv = c->n_kv_heads * (c->d_model / c->n_heads);
    const int64_t embedding = c->vocab_size * d;
    const int64_t attention = c->n_layers * (2 * d * d + 2 * d * kv);
    const int64_t mlp = c->n_layers * 3 * d * c->d_ff;
    const int64_t norms = c->n_layers * 2 * d + d;
    const int64_t head = c->tie_embeddings ? 0 : embedding;
    return embedding + attention + mlp + norms + head;
}

/* presets.rs:52-83 */
int32_t mmo_preset(int32_t which, mmo_config *out) {
    static const int64_t dims[6][6] = {
        {64, 2, 4, 4, 176, 128},      {128, 4, 4, 4, 344, 256},
        {384, 6, 6, 6, 1024, 512},    {768, 12, 12, 12, 2048, 1024},
        {1024, 24, 16, 8, 2816, 2048}, {2048, 20, 16, 8, 5632, 2048},
    };
    static const int64_t vocab[6] = {256, 4096, 32000, 32000, 32000, 32000};
    if (which < 0 || which > 5 || !out) return MMO_ERR_ARGUMENT;
    out->vocab_size = vocab[which];
    out->d_model = dims[which][0];
    out->n_layers = dims[which][1];
    out->n_heads = dims[which][2];
    out->n_kv_heads = dims[which][3];
    out->d_ff = dims[which][4];
    out->max_seq_len = dims[which][5];
    out->rope_theta = 10000.0f;
    out->norm_eps = 1e-5f;
    out->tie_embeddings = 1;
    return MMO_OK;
}

/* Splits [0, n) into nthreads contiguous ranges run on pthreads. */
typedef void (*range_fn)(void *ctx, int64_t lo, int64_t hi);
typedef struct {
    range_fn fn;
    void *ctx;
    int64_t lo, hi;
} range_task;

static void *range_thread(void *arg) {
    range_task *t = (range_task *)arg;
    if (t->lo < t->hi) t->fn(t->ctx, t->lo, t->hi);
    return NULL;
}

static void parallel_for(int64_t n, int32_t nthreads, range_fn fn, void *ctx) {
    if (nthreads <= 1 || n < 2) {
        fn(ctx, 0, n);
        return;
    }
    if (nthreads > 64) nthreads = 64;
    if (nthreads > n) nthreads = (int32_t)n;
    pthread_t th[64];
    range_task tasks[64];
    for (int32_t i = 0; i < nthreads; i++) {
        tasks[i].fn = fn;
        tasks[i].ctx = ctx;
        tasks[i].lo = n * i / nthreads;
        tasks[i].hi = n * (i + 1) / nthreads;
    }
    for (int32_t i = 1; i < nthreads; i++) pthread_create(&th[i], NULL, range_thread, &tasks[i]);
    range_thread(&tasks[0]);
    for (int32_t i = 1; i < nthreads; i++) pthread_join(th[i], NULL);
}

/* ------------------------------------------------------------------------ */
/* Init: model.rs:51-83, init.rs:33-40, tensor.rs:158-162                    */
/* ------------------------------------------------------------------------ */

/* Tensor::randn: each value is std * normal() as an f32 product. */
static void randn_seq(float *dst, int64_t n, float std, mmo_rng *r) {
    for (int64_t i = 0; i < n; i++) dst[i] = std * mmo_rng_normal(r);
}

/* The same values with the transcendental work spread over threads: the
 * draws are taken from the stream in order (a chunk at a time), and pair j of
 * a chunk turns draws 2j, 2j+1 into values 2j, 2j+1, exactly what the
 * sequential loop computes for them; a cached spare is used first and an odd
 * last value comes from mmo_rng_normal, which caches its pair's spare. */
typedef struct {
    const uint64_t *draws;
    float *out;
    float std;
} randn_chunk;

static void randn_pairs(void *ctx, int64_t lo, int64_t hi) {
    const randn_chunk *k = (const randn_chunk *)ctx;
    for (int64_t j = lo; j < hi; j++) {
        float c, s;
        box_muller(k->draws[2 * j], k->draws[2 * j + 1], &c, &s);
        k->out[2 * j] = k->std * c;
        k->out[2 * j + 1] = k->std * s;
    }
}

static int32_t g_init_threads = 1; /* set by mmo_init_weights_mt for its call */

static void randn(float *dst, int64_t n, float std, mmo_rng *r) {
    if (g_init_threads <= 1 || n < (1 << 16)) {
        randn_seq(dst, n, std, r);
        return;
    }
    int64_t i = 0;
    if (r->has_spare) dst[i++] = std * mmo_rng_normal(r);
    const int64_t pairs = (n - i) / 2, chunk = (int64_t)1 << 20;
    uint64_t *draws = (uint64_t *)malloc((size_t)(pairs < chunk ? pairs : chunk) * 2 * 8 + 16);
    for (int64_t base = 0; base < pairs; base += chunk) {
        const int64_t cnt = pairs - base < chunk ? pairs - base : chunk;
        for (int64_t j = 0; j < 2 * cnt; j++) draws[j] = mmo_rng_next_u64(r);
        randn_chunk k = {draws, dst + i + 2 * base, std};
        parallel_for(cnt, g_init_threads, randn_pairs, &k);
    }
    free(draws);
    if ((n - i) & 1) dst[n - 1] = std * mmo_rng_normal(r);
}

void mmo_randn(mmo_rng *r, float *dst, int64_t n, float std) { randn(dst, n, std, r); }

static void ones(float *dst, int64_t n) {
    for (int64_t i = 0; i < n; i++) dst[i] = 1.0f;
}

int32_t mmo_init_weights(const mmo_config *c, float std, mmo_rng *r, float *w, int64_t n) {
    const int64_t total = mmo_param_count(c);
    if (total < 0) return MMO_ERR_CONFIG;
    if (!(isfinite(std) && std > 0.0f) || !r || !w) return MMO_ERR_ARGUMENT;
    if (n != total) return MMO_ERR_SHAPE;
    const int64_t d = c->d_model, ff = c->d_ff, kv = c->n_kv_heads * (d / c->n_heads);
    /* Init::scaled: out_std = std / (2.0 * n_layers as f32).sqrt() (init.rs:38) */
    const float out_std = std / sqrtf(2.0f * (float)c->n_layers);
    float *p = w;
    randn(p, c->vocab_size * d, std, r); /* embed_tokens (embedding.rs:25-35) */
    p += c->vocab_size * d;
    for (int64_t l = 0; l < c->n_layers; l++) { /* block.rs:45-58 */
        ones(p, d); p += d;                     /* attn_norm */
        randn(p, d * d, std, r); p += d * d;    /* q_proj (attention.rs:205-213) */
        randn(p, d * kv, std, r); p += d * kv;  /* k_proj */
        randn(p, d * kv, std, r); p += d * kv;  /* v_proj */
        randn(p, d * d, out_std, r); p += d * d;/* o_proj */
        ones(p, d); p += d;                     /* mlp_norm */
        randn(p, d * ff, std, r); p += d * ff;  /* gate_proj (mlp.rs:44-50) */
        randn(p, d * ff, std, r); p += d * ff;  /* up_proj */
        randn(p, ff * d, out_std, r); p += ff * d; /* down_proj */
    }
    ones(p, d); p += d; /* final_norm */
    if (!c->tie_embeddings) {
        randn(p, d * c->vocab_size, std, r); /* lm_head */
        p += d * c->vocab_size;
    }
    return (p - w == total) ? MMO_OK : MMO_ERR_SHAPE;
}

/* mmo_init_weights with the normals' arithmetic on nthreads threads: the same
 * bits (the draw order is unchanged). Not reentrant across threads. */
int32_t mmo_init_weights_mt(const mmo_config *c, float std, mmo_rng *r, float *w, int64_t n,
                            int32_t nthreads) {
    g_init_threads = nthreads;
    const int32_t st = mmo_init_weights(c, std, r, w, n);
    g_init_threads = 1;
    return st;
}

/* lab.rs:194-203 */
void mmo_lab_tokens(mmo_rng *r, int64_t vocab, int64_t batch, int64_t seq, int32_t *inputs,
                    int32_t *targets) {
    int32_t *tok = (int32_t *)malloc(sizeof(int32_t) * (size_t)(seq + 1));
    for (int64_t b = 0; b < batch; b++) {
        for (int64_t i = 0; i <= seq; i++) tok[i] = (int32_t)mmo_rng_below(r, (uint64_t)vocab);
        memcpy(inputs + b * seq, tok, sizeof(int32_t) * (size_t)seq);
        memcpy(targets + b * seq, tok + 1, sizeof(int32_t) * (size_t)seq);
    }
    free(tok);
}

/* ------------------------------------------------------------------------ */
/* Threads: split [0, n) into contiguous ranges                              */
/* ------------------------------------------------------------------------ */

/* ------------------------------------------------------------------------ */
/* GEMM: kernels.rs:49-108 (scalar) and kernels_avx.rs:177-204 (4x16 tile)   */
/* ------------------------------------------------------------------------ */

/* Every C[i][j] receives A[i][p]*B[p][j] for p ascending, each product
 * rounded and then added, starting from C's value: the scalar i-p-j loop of
 * kernels.rs:89-97. The 4x16 register tile below keeps that per-element order
 * exactly (it is the layout of the reference AVX kernel, kernels_avx.rs:177-204,
 * with a separate multiply and add), and blocking over columns and p does not
 * change it either: C[i][j] is the running sum, whichever loop holds it. */
typedef float v8 __attribute__((vector_size(32)));
typedef float v8u __attribute__((vector_size(32), aligned(4)));

#define KB 256
#define JP 256

typedef struct {
    const float *a, *b;
    float *c;
    int64_t m, k, n;
} gemm_args;

static void gemm_rows(void *ctx, int64_t i_lo, int64_t i_hi) {
    const gemm_args *g = (const gemm_args *)ctx;
    const float *a = g->a, *b = g->b;
    float *c = g->c;
    const int64_t k = g->k, n = g->n;
    for (int64_t j0 = 0; j0 < n; j0 += JP) {
        const int64_t j1 = j0 + JP < n ? j0 + JP : n;
        for (int64_t p0 = 0; p0 < k; p0 += KB) {
            const int64_t p1 = p0 + KB < k ? p0 + KB : k;
            int64_t i = i_lo;
            for (; i + 4 <= i_hi; i += 4) {
                int64_t j = j0;
                for (; j + 16 <= j1; j += 16) {
                    v8 acc[4][2];
                    for (int r = 0; r < 4; r++) {
                        acc[r][0] = *(const v8u *)(c + (i + r) * n + j);
                        acc[r][1] = *(const v8u *)(c + (i + r) * n + j + 8);
                    }
                    for (int64_t p = p0; p < p1; p++) {
                        const v8 b0 = *(const v8u *)(b + p * n + j);
                        const v8 b1 = *(const v8u *)(b + p * n + j + 8);
                        for (int r = 0; r < 4; r++) {
                            const float av = a[(i + r) * k + p];
                            const v8 va = {av, av, av, av, av, av, av, av};
                            acc[r][0] = acc[r][0] + va * b0;
                            acc[r][1] = acc[r][1] + va * b1;
                        }
                    }
                    for (int r = 0; r < 4; r++) {
                        *(v8u *)(c + (i + r) * n + j) = acc[r][0];
                        *(v8u *)(c + (i + r) * n + j + 8) = acc[r][1];
                    }
                }
                for (int r = 0; r < 4; r++) { /* column tail */
                    float *crow = c + (i + r) * n;
                    const float *arow = a + (i + r) * k;
                    for (int64_t p = p0; p < p1; p++) {
                        const float av = arow[p];
                        const float *brow = b + p * n;
                        for (int64_t jj = j; jj < j1; jj++) crow[jj] += av * brow[jj];
                    }
                }
            }
            for (; i < i_hi; i++) { /* row tail */
                float *crow = c + i * n;
                const float *arow = a + i * k;
                for (int64_t p = p0; p < p1; p++) {
                    const float av = arow[p];
                    const float *brow = b + p * n;
                    for (int64_t jj = j0; jj < j1; jj++) crow[jj] += av * brow[jj];
                }
            }
        }
    }
}

void mmo_gemm_nn(const float *a, const float *b, float *c, int64_t m, int64_t k, int64_t n,
                 int32_t nthreads) {
    if (m <= 0 || n <= 0 || k <= 0) return;
    gemm_args g = {a, b, c, m, k, n};
    parallel_for(m, nthreads, gemm_rows, &g);
}

/* [rows, cols] -> [cols, rows] */
static float *transpose_copy(const float *x, int64_t rows, int64_t cols) {
    float *t = (float *)malloc(sizeof(float) * (size_t)(rows * cols));
    for (int64_t r = 0; r < rows; r++)
        for (int64_t q = 0; q < cols; q++) t[q * rows + r] = x[r * cols + q];
    return t;
}

/* kernels.rs:66-75: B [n,k] is copied into [k,n], then gemm_nn. */
void mmo_gemm_nt(const float *a, const float *b, float *c, int64_t m, int64_t k, int64_t n,
                 int32_t nthreads) {
    if (m <= 0 || n <= 0 || k <= 0) return;
    float *bt = transpose_copy(b, n, k);
    mmo_gemm_nn(a, bt, c, m, k, n, nthreads);
    free(bt);
}

/* kernels.rs:100-108 sums A[p][i]*B[p][j] over p ascending for every (i,j);
 * copying A [k,m] to [m,k] and running gemm_nn gives each element the same
 * sum in the same order. */
void mmo_gemm_tn(const float *a, const float *b, float *c, int64_t m, int64_t k, int64_t n,
                 int32_t nthreads) {
    if (m <= 0 || n <= 0 || k <= 0) return;
    float *at = transpose_copy(a, k, m);
    mmo_gemm_nn(at, b, c, m, k, n, nthreads);
    free(at);
}

/* ops_matmul.rs:62-74: dA = gemm_nt(g, B) into zeros, dB = gemm_tn(A, g) into zeros. */
void mmo_matmul_backward(const float *a, const float *b, const float *dc, float *da, float *db,
                         int64_t rows, int64_t k, int64_t n, int32_t nthreads) {
    if (da) {
        memset(da, 0, sizeof(float) * (size_t)(rows * k));
        mmo_gemm_nt(dc, b, da, rows, n, k, nthreads);
    }
    if (db) {
        memset(db, 0, sizeof(float) * (size_t)(k * n));
        mmo_gemm_tn(a, dc, db, k, rows, n, nthreads);
    }
}

/* ------------------------------------------------------------------------ */
/* Layer ops                                                                 */
/* ------------------------------------------------------------------------ */

/* ops_shape.rs:230-257 */
int32_t mmo_embedding(const float *table, int64_t v, int64_t d, const int32_t *ids, int64_t n,
                      float *out) {
    for (int64_t i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= v) return MMO_ERR_INDEX;
    for (int64_t i = 0; i < n; i++)
        memcpy(out + i * d, table + (int64_t)ids[i] * d, sizeof(float) * (size_t)d);
    return MMO_OK;
}

/* norm.rs:36-38: x*x -> sum_axis (sequential f32, ops_reduce.rs:38-47) ->
 * scale(1/len) (ops_reduce.rs:91) -> add_scalar(eps) -> powf(-0.5) ->
 * x*inv -> *w. */
void mmo_rms_norm(const float *x, const float *w, int64_t rows, int64_t d, float eps,
                  float *out) {
    const float inv_len = 1.0f / (float)d;
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + r * d;
        float total = 0.0f;
        for (int64_t j = 0; j < d; j++) {
            const float sq = xr[j] * xr[j];
            total += sq;
        }
        const float mean = total * inv_len;
        const float inv = powf(mean + eps, -0.5f);
        for (int64_t j = 0; j < d; j++) {
            const float y = xr[j] * inv;
            out[r * d + j] = y * w[j];
        }
    }
}

/* rope.rs:71-79: angles in f64, stored as f32. */
void mmo_rope_tables(int64_t head_dim, int64_t max_seq_len, float theta, float *cos_t,
                     float *sin_t) {
    const int64_t half = head_dim / 2;
    for (int64_t pos = 0; pos < max_seq_len; pos++) {
        for (int64_t i = 0; i < half; i++) {
            const double frequency = pow((double)theta, -(double)i / (double)half);
            const double angle = (double)pos * frequency;
            cos_t[pos * half + i] = (float)cos(angle);
            sin_t[pos * half + i] = (float)sin(angle);
        }
    }
}

/* rope.rs:28-32: concat(x1*cos - x2*sin, x2*cos + x1*sin), each op rounded. */
void mmo_apply_rope(const float *x, int64_t bh, int64_t t, int64_t hd, const float *cos_t,
                    const float *sin_t, float *out) {
    const int64_t half = hd / 2;
    for (int64_t m = 0; m < bh; m++) {
        for (int64_t pos = 0; pos < t; pos++) {
            const float *xr = x + (m * t + pos) * hd;
            float *o = out + (m * t + pos) * hd;
            const float *cr = cos_t + pos * half, *sr = sin_t + pos * half;
            for (int64_t i = 0; i < half; i++) {
                const float x1 = xr[i], x2 = xr[i + half];
                const float a = x1 * cr[i], b = x2 * sr[i];
                const float c = x2 * cr[i], e = x1 * sr[i];
                o[i] = a - b;
                o[i + half] = c + e;
            }
        }
    }
}

typedef struct {
    const float *q, *k, *v;
    float *out;
    float *probs; /* [B,H,T,T] or NULL: the probabilities, 0 above the diagonal */
    int64_t h, hkv, t, hd;
} attn_args;

/* One (batch, head) per index. attention.rs:79-85 and :97-101:
 *   scores = (q . k^T) * scale + mask, softmax over the last axis
 *   (ops_reduce.rs:102-120), context = probs . v, all through gemm_nn
 *   (ops_matmul.rs:87-96) with the key head j / (H/Hkv) (repeat_interleave,
 *   ops_shape.rs:192-200).
 * Masked entries (key > query) are skipped: the reference gives them
 * score*scale - 1e9, which never exceeds a row's unmasked maximum, whose
 * exp(. - max) is exactly 0.0f, and which add 0.0 to the softmax sum and
 * +-0.0 to each context sum; skipping them leaves every result bit the same. */
static void attn_heads(void *ctx, int64_t lo, int64_t hi) {
    const attn_args *g = (const attn_args *)ctx;
    const int64_t t = g->t, hd = g->hd, groups = g->h / g->hkv;
    const float scale = 1.0f / sqrtf((float)hd);
    float *kt = (float *)malloc(sizeof(float) * (size_t)(hd * t));
    float *row = (float *)malloc(sizeof(float) * (size_t)t);
    for (int64_t bh = lo; bh < hi; bh++) {
        const int64_t b = bh / g->h, h = bh % g->h;
        const int64_t kvh = h / groups;
        const float *q = g->q + bh * t * hd;
        const float *k = g->k + (b * g->hkv + kvh) * t * hd;
        const float *v = g->v + (b * g->hkv + kvh) * t * hd;
        float *o = g->out + bh * t * hd;
        for (int64_t j = 0; j < t; j++)
            for (int64_t p = 0; p < hd; p++) kt[p * t + j] = k[j * hd + p];
        for (int64_t i = 0; i < t; i++) {
            const int64_t len = i + 1;
            for (int64_t j = 0; j < len; j++) row[j] = 0.0f;
            for (int64_t p = 0; p < hd; p++) { /* gemm_nn order: p ascending */
                const float qv = q[i * hd + p];
                const float *kr = kt + p * t;
                for (int64_t j = 0; j < len; j++) row[j] += qv * kr[j];
            }
            float mx = -INFINITY;
            for (int64_t j = 0; j < len; j++) {
                row[j] = row[j] * scale + 0.0f; /* .scale(scale).add(mask) */
                mx = fmaxf(mx, row[j]);
            }
            float sum = 0.0f;
            for (int64_t j = 0; j < len; j++) {
                const float e = expf(row[j] - mx);
                row[j] = e;
                sum += e;
            }
            const float inv = 1.0f / sum;
            for (int64_t j = 0; j < len; j++) row[j] *= inv;
            if (g->probs) {
                float *pr = g->probs + (bh * t + i) * t;
                for (int64_t j = 0; j < t; j++) pr[j] = j < len ? row[j] : 0.0f;
            }
            float *orow = o + i * hd;
            for (int64_t d = 0; d < hd; d++) orow[d] = 0.0f;
            for (int64_t j = 0; j < len; j++) {
                const float pj = row[j];
                const float *vr = v + j * hd;
                for (int64_t d = 0; d < hd; d++) orow[d] += pj * vr[d];
            }
        }
    }
    free(kt);
    free(row);
}

void mmo_causal_attention(const float *q, const float *k, const float *v, int64_t b, int64_t h,
                          int64_t hkv, int64_t t, int64_t hd, float *out, int32_t nthreads) {
    attn_args g = {q, k, v, out, NULL, h, hkv, t, hd};
    parallel_for(b * h, nthreads, attn_heads, &g);
}

/* [B,T,H,hd] <-> [B,H,T,hd] (reshape + permute(0,2,1,3), attention.rs:161,168) */
static void split_heads(const float *x, int64_t ld, int64_t off, int64_t b, int64_t t,
                        int64_t heads, int64_t hd, float *out) {
    for (int64_t bb = 0; bb < b; bb++)
        for (int64_t tt = 0; tt < t; tt++)
            for (int64_t hh = 0; hh < heads; hh++)
                memcpy(out + ((bb * heads + hh) * t + tt) * hd,
                       x + (bb * t + tt) * ld + off + hh * hd, sizeof(float) * (size_t)hd);
}

static void merge_heads(const float *x, int64_t b, int64_t t, int64_t heads, int64_t hd,
                        float *out) {
    for (int64_t bb = 0; bb < b; bb++)
        for (int64_t hh = 0; hh < heads; hh++)
            for (int64_t tt = 0; tt < t; tt++)
                memcpy(out + (bb * t + tt) * heads * hd + hh * hd,
                       x + ((bb * heads + hh) * t + tt) * hd, sizeof(float) * (size_t)hd);
}

static float *zalloc(int64_t n) { return (float *)calloc((size_t)n, sizeof(float)); }

/* attention.rs:146-170 */
void mmo_attention_forward(const float *x, const float *wq, const float *wk, const float *wv,
                           const float *wo, const float *cos_t, const float *sin_t, int64_t b,
                           int64_t t, int64_t d, int64_t h, int64_t hkv, float *out,
                           int32_t nthreads) {
    const int64_t hd = d / h, kv = hkv * hd, n = b * t;
    float *qp = zalloc(n * d), *kp = zalloc(n * kv), *vp = zalloc(n * kv);
    mmo_gemm_nn(x, wq, qp, n, d, d, nthreads);
    mmo_gemm_nn(x, wk, kp, n, d, kv, nthreads);
    mmo_gemm_nn(x, wv, vp, n, d, kv, nthreads);
    float *qh = zalloc(n * d), *kh = zalloc(n * kv), *vh = zalloc(n * kv);
    split_heads(qp, d, 0, b, t, h, hd, qh);
    split_heads(kp, kv, 0, b, t, hkv, hd, kh);
    split_heads(vp, kv, 0, b, t, hkv, hd, vh);
    mmo_apply_rope(qh, b * h, t, hd, cos_t, sin_t, qp);   /* qp now rotated q */
    mmo_apply_rope(kh, b * hkv, t, hd, cos_t, sin_t, kp); /* kp now rotated k */
    float *ctx = zalloc(n * d);
    mmo_causal_attention(qp, kp, vh, b, h, hkv, t, hd, ctx, nthreads);
    merge_heads(ctx, b, t, h, hd, qh); /* qh reused as merged [B,T,d] */
    memset(out, 0, sizeof(float) * (size_t)(n * d));
    mmo_gemm_nn(qh, wo, out, n, d, d, nthreads);
    free(qp); free(kp); free(vp); free(qh); free(kh); free(vh); free(ctx);
}

/* ops_elementwise.rs:239-241 and :355-364: silu(x) = x * (1 / (1 + e^-x)) */
static inline float silu(float x) {
    const float s = 1.0f / (1.0f + expf(-x));
    return x * s;
}

/* mlp.rs:20-24 */
void mmo_swiglu(const float *x, const float *wg, const float *wu, const float *wd, int64_t rows,
                int64_t d, int64_t ff, float *out, int32_t nthreads) {
    float *g = zalloc(rows * ff), *u = zalloc(rows * ff);
    mmo_gemm_nn(x, wg, g, rows, d, ff, nthreads);
    mmo_gemm_nn(x, wu, u, rows, d, ff, nthreads);
    for (int64_t i = 0; i < rows * ff; i++) g[i] = silu(g[i]) * u[i];
    memset(out, 0, sizeof(float) * (size_t)(rows * d));
    mmo_gemm_nn(g, wd, out, rows, ff, d, nthreads);
    free(g);
    free(u);
}

/* ops_reduce.rs:253-258, one row each */
int32_t mmo_cross_entropy_rows(const float *logits, const int32_t *targets, int64_t n,
                               int64_t v, float *row_loss) {
    for (int64_t i = 0; i < n; i++)
        if (targets[i] < 0 || targets[i] >= v) return MMO_ERR_INDEX;
    for (int64_t i = 0; i < n; i++) {
        const float *row = logits + i * v;
        float mx = -INFINITY;
        for (int64_t j = 0; j < v; j++) mx = fmaxf(mx, row[j]);
        float sum = 0.0f;
        for (int64_t j = 0; j < v; j++) sum += expf(row[j] - mx);
        const float lse = mx + logf(sum);
        row_loss[i] = lse - row[targets[i]];
    }
    return MMO_OK;
}

/* ops_reduce.rs:236-259 */
int32_t mmo_cross_entropy(const float *logits, const int32_t *targets, int64_t n, int64_t v,
                          float *loss) {
    if (n <= 0 || v <= 0) return MMO_ERR_SHAPE;
    float *rows = (float *)malloc(sizeof(float) * (size_t)n);
    const int32_t st = mmo_cross_entropy_rows(logits, targets, n, v, rows);
    if (st != MMO_OK) {
        free(rows);
        return st;
    }
    double total = 0.0;
    for (int64_t i = 0; i < n; i++) total += (double)rows[i];
    *loss = (float)(total / (double)n);
    free(rows);
    return MMO_OK;
}

static void add_inplace(float *x, const float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) x[i] = x[i] + y[i];
}

/* block.rs:77-81: h = x + attn(norm1(x)); y = h + mlp(norm2(h)) */
int32_t mmo_block_forward(const mmo_config *c, const float *bw, const float *cos_t,
                          const float *sin_t, const float *x, int64_t b, int64_t t, float *out,
                          int32_t nthreads) {
    const int64_t d = c->d_model, ff = c->d_ff, hd = d / c->n_heads,
                  kv = c->n_kv_heads * hd, n = b * t;
    const float *attn_norm = bw, *wq = attn_norm + d, *wk = wq + d * d, *wv = wk + d * kv,
                *wo = wv + d * kv, *mlp_norm = wo + d * d, *wg = mlp_norm + d,
                *wu = wg + d * ff, *wd = wu + d * ff;
    float *xn = zalloc(n * d), *tmp = zalloc(n * d);
    mmo_rms_norm(x, attn_norm, n, d, c->norm_eps, xn);
    mmo_attention_forward(xn, wq, wk, wv, wo, cos_t, sin_t, b, t, d, c->n_heads, c->n_kv_heads,
                          tmp, nthreads);
    memcpy(out, x, sizeof(float) * (size_t)(n * d));
    add_inplace(out, tmp, n * d);
    mmo_rms_norm(out, mlp_norm, n, d, c->norm_eps, xn);
    mmo_swiglu(xn, wg, wu, wd, n, d, ff, tmp, nthreads);
    add_inplace(out, tmp, n * d);
    free(xn);
    free(tmp);
    return MMO_OK;
}

static int64_t block_param_count(const mmo_config *c) {
    const int64_t d = c->d_model, kv = c->n_kv_heads * (d / c->n_heads);
    return 2 * d + 2 * d * d + 2 * d * kv + 3 * d * c->d_ff;
}

/* model.rs:127-165 */
int32_t mmo_forward(const mmo_config *c, const float *w, const int32_t *ids, int64_t b,
                    int64_t t, float *logits, int32_t nthreads) {
    if (mmo_config_validate(c) != MMO_OK) return MMO_ERR_CONFIG;
    if (b <= 0 || t <= 0 || t > c->max_seq_len) return MMO_ERR_ARGUMENT;
    const int64_t d = c->d_model, v = c->vocab_size, n = b * t, hd = d / c->n_heads;
    float *x = zalloc(n * d), *y = zalloc(n * d);
    const int32_t st = mmo_embedding(w, v, d, ids, n, x);
    if (st != MMO_OK) {
        free(x);
        free(y);
        return st;
    }
    float *cos_t = zalloc(c->max_seq_len * hd / 2), *sin_t = zalloc(c->max_seq_len * hd / 2);
    mmo_rope_tables(hd, c->max_seq_len, c->rope_theta, cos_t, sin_t);
    const float *bw = w + v * d;
    for (int64_t l = 0; l < c->n_layers; l++) {
        mmo_block_forward(c, bw, cos_t, sin_t, x, b, t, y, nthreads);
        float *sw = x; x = y; y = sw;
        bw += block_param_count(c);
    }
    const float *final_norm = bw;
    mmo_rms_norm(x, final_norm, n, d, c->norm_eps, y);
    memset(logits, 0, sizeof(float) * (size_t)(n * v));
    if (c->tie_embeddings)
        mmo_gemm_nt(y, w, logits, n, d, v, nthreads); /* x . E^T, E^T materialized */
    else
        mmo_gemm_nn(y, final_norm + d, logits, n, d, v, nthreads);
    free(x); free(y); free(cos_t); free(sin_t);
    return MMO_OK;
}

/* model.rs:174-183 */
int32_t mmo_forward_loss(const mmo_config *c, const float *w, const int32_t *ids,
                         const int32_t *targets, int64_t b, int64_t t, float *logits,
                         float *loss, int32_t nthreads) {
    if (mmo_config_validate(c) != MMO_OK) return MMO_ERR_CONFIG;
    if (b <= 0 || t <= 0) return MMO_ERR_ARGUMENT;
    const int64_t n = b * t, v = c->vocab_size;
    for (int64_t i = 0; i < n; i++)
        if (targets[i] < 0 || targets[i] >= v) return MMO_ERR_INDEX;
    float *own = logits ? NULL : zalloc(n * v);
    float *lg = logits ? logits : own;
    int32_t st = mmo_forward(c, w, ids, b, t, lg, nthreads);
    if (st == MMO_OK) st = mmo_cross_entropy(lg, targets, n, v, loss);
    free(own);
    return st;
}

/* ------------------------------------------------------------------------ */
/* Backward: the autograd closures of the ops above, and the training step   */
/* ------------------------------------------------------------------------ */
/*
 * Each closure is restated with the reference's per-element arithmetic. Where
 * one tensor receives gradients from several consumers (the residual stream,
 * x in both x*x and x*inv of a norm, the input of the q/k/v projections), the
 * reference adds them in its graph-traversal order (autograd.rs:69-125,
 * accumulate :44-56); here they are added in the fixed order each function
 * states. A sum of a few such terms may differ from the reference's in the
 * last bit; the golden gradient norms (1e-4 relative) absorb that.
 */

/* ops_reduce.rs:261-275: d = exp(z-max)/sum*scale, then d[t] -= scale, with
 * scale = g/N. */
int32_t mmo_cross_entropy_backward(const float *logits, const int32_t *targets, int64_t n,
                                   int64_t v, float g, float *dlogits) {
    if (n <= 0 || v <= 0) return MMO_ERR_SHAPE;
    for (int64_t i = 0; i < n; i++)
        if (targets[i] < 0 || targets[i] >= v) return MMO_ERR_INDEX;
    const float scale = g / (float)n;
    for (int64_t i = 0; i < n; i++) {
        const float *row = logits + i * v;
        float *drow = dlogits + i * v;
        float mx = -INFINITY;
        for (int64_t j = 0; j < v; j++) mx = fmaxf(mx, row[j]);
        float sum = 0.0f;
        for (int64_t j = 0; j < v; j++) sum += expf(row[j] - mx);
        for (int64_t j = 0; j < v; j++) drow[j] = expf(row[j] - mx) / sum * scale;
        drow[targets[i]] -= scale;
    }
    return MMO_OK;
}

/* ops_shape.rs:261-269: dtable[id] += g row, ids in order. Accumulates. */
void mmo_embedding_backward(const int32_t *ids, int64_t n, const float *g, int64_t d,
                            float *dtable) {
    for (int64_t i = 0; i < n; i++) {
        float *t = dtable + (int64_t)ids[i] * d;
        const float *gr = g + i * d;
        for (int64_t j = 0; j < d; j++) t[j] += gr[j];
    }
}

/* norm.rs:36-38 backward, through y = (x*inv)*w (mul, ops_elementwise.rs:
 * 123-198), inv = (mean(x*x) + eps)^-0.5 (powf :335-337, add_scalar :309-312,
 * mean_axis = sum_axis then scale, ops_reduce.rs:34-92):
 *   dy0 = dy*w; dw = sum over rows of dy*y0; dinv = sum_j dy0*x;
 *   ds = dinv*(-0.5*a^-1.5)*(1/d); dx = (dy0*inv + ds*x) + ds*x.
 * dx receives only the norm's share (the caller adds the residual branch);
 * dw is overwritten. */
void mmo_rms_norm_backward(const float *x, const float *w, const float *dy, int64_t rows,
                           int64_t d, float eps, float *dx, float *dw) {
    const float inv_len = 1.0f / (float)d;
    for (int64_t j = 0; j < d; j++) dw[j] = 0.0f;
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + r * d, *gr = dy + r * d;
        float *o = dx + r * d;
        float total = 0.0f;
        for (int64_t j = 0; j < d; j++) {
            const float sq = xr[j] * xr[j];
            total += sq;
        }
        const float a = total * inv_len + eps;
        const float inv = powf(a, -0.5f);
        float dinv = 0.0f;
        for (int64_t j = 0; j < d; j++) {
            const float g0 = gr[j] * w[j];
            const float prod = g0 * xr[j];
            dinv += prod;
            const float y0 = xr[j] * inv;
            const float gw = gr[j] * y0;
            dw[j] += gw;
        }
        const float da = dinv * (-0.5f * powf(a, -1.5f));
        const float ds = da * inv_len;
        for (int64_t j = 0; j < d; j++) {
            const float g0 = gr[j] * w[j];
            const float direct = g0 * inv;
            const float t = ds * xr[j];
            const float partial = direct + t;
            o[j] = partial + t;
        }
    }
}

/* rope.rs:28-32 backward: the halves route through narrow/concat and the
 * products give dx1 = dfirst*cos + dsecond*sin, dx2 = dsecond*cos - dfirst*sin
 * (the sub's right operand receives -dfirst). */
void mmo_rope_backward(const float *dy, int64_t bh, int64_t t, int64_t hd, const float *cos_t,
                       const float *sin_t, float *dx) {
    const int64_t half = hd / 2;
    for (int64_t m = 0; m < bh; m++) {
        for (int64_t pos = 0; pos < t; pos++) {
            const float *gr = dy + (m * t + pos) * hd;
            float *o = dx + (m * t + pos) * hd;
            const float *cr = cos_t + pos * half, *sr = sin_t + pos * half;
            for (int64_t i = 0; i < half; i++) {
                const float df = gr[i], dsec = gr[i + half];
                const float a = df * cr[i], b = dsec * sr[i];
                const float c = dsec * cr[i], e = df * sr[i];
                o[i] = a + b;
                o[i + half] = c - e;
            }
        }
    }
}

typedef struct {
    const float *q, *k, *v, *dout;
    float *dq, *dk_h, *dv_h; /* dk_h/dv_h per query head, [B,H,T,hd] */
    int64_t h, hkv, t, hd;
} attn_bwd_args;

/* One (batch, head) per index. The forward's probabilities are rebuilt with
 * the forward's own operations, then the closures run in reverse:
 *   context = probs.v       (batched matmul backward, ops_matmul.rs:100-125):
 *       dprobs = dctx.v^T, dv = probs^T.dctx (query rows ascending)
 *   probs = softmax(scores) (ops_reduce.rs:144-175): ds = p*(g - sum g*p)
 *   scores = raw*scale + mask: draw = ds*scale
 *   raw = q.k^T:            dq = draw.k, dk = draw^T.q (query rows ascending)
 * Entries above the diagonal carry p = 0, so their terms are +-0 and are
 * skipped without changing a bit. */
static void attn_bwd_heads(void *ctx, int64_t lo, int64_t hi) {
    const attn_bwd_args *g = (const attn_bwd_args *)ctx;
    const int64_t t = g->t, hd = g->hd, groups = g->h / g->hkv;
    const float scale = 1.0f / sqrtf((float)hd);
    float *kt = (float *)malloc(sizeof(float) * (size_t)(hd * t));
    float *row = (float *)malloc(sizeof(float) * (size_t)t);
    float *dp = (float *)malloc(sizeof(float) * (size_t)t);
    for (int64_t bh = lo; bh < hi; bh++) {
        const int64_t b = bh / g->h, h = bh % g->h;
        const int64_t kvh = h / groups;
        const float *q = g->q + bh * t * hd;
        const float *k = g->k + (b * g->hkv + kvh) * t * hd;
        const float *v = g->v + (b * g->hkv + kvh) * t * hd;
        const float *dout = g->dout + bh * t * hd;
        float *dq = g->dq + bh * t * hd;
        float *dk = g->dk_h + bh * t * hd, *dv = g->dv_h + bh * t * hd;
        memset(dq, 0, sizeof(float) * (size_t)(t * hd));
        memset(dk, 0, sizeof(float) * (size_t)(t * hd));
        memset(dv, 0, sizeof(float) * (size_t)(t * hd));
        for (int64_t j = 0; j < t; j++)
            for (int64_t p = 0; p < hd; p++) kt[p * t + j] = k[j * hd + p];
        for (int64_t i = 0; i < t; i++) {
            const int64_t len = i + 1;
            /* probabilities, exactly as the forward (attn_heads) */
            for (int64_t j = 0; j < len; j++) row[j] = 0.0f;
            for (int64_t p = 0; p < hd; p++) {
                const float qv = q[i * hd + p];
                const float *kr = kt + p * t;
                for (int64_t j = 0; j < len; j++) row[j] += qv * kr[j];
            }
            float mx = -INFINITY;
            for (int64_t j = 0; j < len; j++) {
                row[j] = row[j] * scale + 0.0f;
                mx = fmaxf(mx, row[j]);
            }
            float sum = 0.0f;
            for (int64_t j = 0; j < len; j++) {
                const float e = expf(row[j] - mx);
                row[j] = e;
                sum += e;
            }
            const float inv = 1.0f / sum;
            for (int64_t j = 0; j < len; j++) row[j] *= inv;
            /* dprobs = dctx . v^T (gemm_nt: p ascending over hd) */
            const float *go = dout + i * hd;
            for (int64_t j = 0; j < len; j++) dp[j] = 0.0f;
            for (int64_t p = 0; p < hd; p++) {
                const float gv = go[p];
                for (int64_t j = 0; j < len; j++) {
                    const float prod = gv * v[j * hd + p];
                    dp[j] += prod;
                }
            }
            /* dv += probs^T . dctx, row i's turn */
            for (int64_t j = 0; j < len; j++) {
                const float pj = row[j];
                float *dvr = dv + j * hd;
                for (int64_t p = 0; p < hd; p++) {
                    const float prod = pj * go[p];
                    dvr[p] += prod;
                }
            }
            /* softmax backward, then the scale */
            float dot = 0.0f;
            for (int64_t j = 0; j < len; j++) {
                const float prod = dp[j] * row[j];
                dot += prod;
            }
            for (int64_t j = 0; j < len; j++) {
                const float diff = dp[j] - dot;
                const float ds = row[j] * diff;
                dp[j] = ds * scale;
            }
            /* dq[i] = draw . k (gemm_nt over j ascending); dk += draw^T . q */
            float *dqr = dq + i * hd;
            for (int64_t j = 0; j < len; j++) {
                const float dj = dp[j];
                const float *kr = k + j * hd;
                float *dkr = dk + j * hd;
                for (int64_t p = 0; p < hd; p++) {
                    const float a = dj * kr[p];
                    dqr[p] += a;
                    const float bq = q[i * hd + p] * dj;
                    dkr[p] += bq;
                }
            }
        }
    }
    free(kt);
    free(row);
    free(dp);
}

/* attention.rs:79-101 backward. dout [B,H,T,hd] -> dq [B,H,T,hd],
 * dk/dv [B,Hkv,T,hd]; the copies of a shared key/value head are summed in
 * head order (repeat_interleave backward, ops_shape.rs:209-219). */
void mmo_causal_attention_backward(const float *q, const float *k, const float *v,
                                   const float *dout, int64_t b, int64_t h, int64_t hkv,
                                   int64_t t, int64_t hd, float *dq, float *dk, float *dv,
                                   int32_t nthreads) {
    const int64_t per = t * hd, groups = h / hkv;
    float *dk_h = zalloc(b * h * per), *dv_h = zalloc(b * h * per);
    attn_bwd_args g = {q, k, v, dout, dq, dk_h, dv_h, h, hkv, t, hd};
    parallel_for(b * h, nthreads, attn_bwd_heads, &g);
    memset(dk, 0, sizeof(float) * (size_t)(b * hkv * per));
    memset(dv, 0, sizeof(float) * (size_t)(b * hkv * per));
    for (int64_t bb = 0; bb < b; bb++)
        for (int64_t kvh = 0; kvh < hkv; kvh++) {
            float *dko = dk + (bb * hkv + kvh) * per, *dvo = dv + (bb * hkv + kvh) * per;
            for (int64_t r = 0; r < groups; r++) {
                const float *dks = dk_h + (bb * h + kvh * groups + r) * per;
                const float *dvs = dv_h + (bb * h + kvh * groups + r) * per;
                for (int64_t e = 0; e < per; e++) {
                    dko[e] += dks[e];
                    dvo[e] += dvs[e];
                }
            }
        }
    free(dk_h);
    free(dv_h);
}

/* ops_elementwise.rs:239-241 */
static inline float sigmoid_value(float x) { return 1.0f / (1.0f + expf(-x)); }

/* The h = silu(g) * u step of mlp.rs:20-24 backward: dsilu = dh*u, du = dh*silu(g)
 * (mul), dg = dsilu * s*(1 + g*(1 - s)) (silu, ops_elementwise.rs:355-364). */
void mmo_silu_mul_backward(const float *gate, const float *up, const float *dh, int64_t n,
                           float *dgate, float *dup) {
    for (int64_t i = 0; i < n; i++) {
        const float x = gate[i];
        const float sv = silu(x);
        const float dsilu = dh[i] * up[i];
        dup[i] = dh[i] * sv;
        const float s = sigmoid_value(x);
        const float one_minus = 1.0f - s;
        const float inner = x * one_minus;
        const float deriv = s * (1.0f + inner);
        dgate[i] = dsilu * deriv;
    }
}

/* Saved forward values of one block. */
typedef struct {
    float *x, *xn1, *q, *k, *v, *ctx, *hres, *xn2, *g, *u, *a;
} block_cache;

/* Parameter segments in reference order: offsets, sizes and ranks. */
static int64_t param_segments(const mmo_config *c, int64_t *off, int64_t *size, int32_t *rank) {
    const int64_t d = c->d_model, ff = c->d_ff, v = c->vocab_size,
                  kv = c->n_kv_heads * (d / c->n_heads);
    int64_t count = 0, at = 0;
#define SEG(sz, rk)                 \
    do {                            \
        off[count] = at;            \
        size[count] = (sz);         \
        rank[count] = (rk);         \
        at += (sz);                 \
        count++;                    \
    } while (0)
    SEG(v * d, 2);
    for (int64_t l = 0; l < c->n_layers; l++) {
        SEG(d, 1);
        SEG(d * d, 2);
        SEG(d * kv, 2);
        SEG(d * kv, 2);
        SEG(d * d, 2);
        SEG(d, 1);
        SEG(d * ff, 2);
        SEG(d * ff, 2);
        SEG(ff * d, 2);
    }
    SEG(d, 1);
    if (!c->tie_embeddings) SEG(d * v, 2);
#undef SEG
    return count;
}

int64_t mmo_param_segments(const mmo_config *c, int64_t *offsets, int64_t *sizes,
                           int32_t *ranks) {
    if (mmo_config_validate(c) != MMO_OK) return MMO_ERR_CONFIG;
    return param_segments(c, offsets, sizes, ranks);
}

/* model.rs:174-183 and every closure beneath it: the loss, and the gradient of
 * every parameter in the flat layout of w (overwritten). The forward is the
 * same sequence of operations as mmo_forward, keeping what the backward reads.
 * Gradient sums across branches (fixed order here):
 *   residual stream: dx = d(out) + d(norm branch);
 *   q/k/v input: dxn = dq.Wq^T + dk.Wk^T + dv.Wv^T, gate/up: dg.Wg^T + du.Wu^T;
 *   tied table: d(head) + d(embedding). */
int32_t mmo_forward_backward(const mmo_config *c, const float *w, const int32_t *ids,
                             const int32_t *targets, int64_t b, int64_t t, float *loss,
                             float *grads, int32_t nthreads) {
    if (mmo_config_validate(c) != MMO_OK) return MMO_ERR_CONFIG;
    if (b <= 0 || t <= 0 || t > c->max_seq_len) return MMO_ERR_ARGUMENT;
    const int64_t d = c->d_model, v = c->vocab_size, n = b * t, ff = c->d_ff,
                  nh = c->n_heads, hkv = c->n_kv_heads, hd = d / nh, kv = hkv * hd,
                  L = c->n_layers;
    for (int64_t i = 0; i < n; i++) {
        if (ids[i] < 0 || ids[i] >= v) return MMO_ERR_INDEX;
        if (targets[i] < 0 || targets[i] >= v) return MMO_ERR_INDEX;
    }
    const int64_t np = mmo_param_count(c), bp = block_param_count(c);
    memset(grads, 0, sizeof(float) * (size_t)np);
    float *cos_t = zalloc(c->max_seq_len * hd / 2), *sin_t = zalloc(c->max_seq_len * hd / 2);
    mmo_rope_tables(hd, c->max_seq_len, c->rope_theta, cos_t, sin_t);

    /* ---- forward, keeping each block's values ---- */
    block_cache *bc = (block_cache *)calloc((size_t)L, sizeof(block_cache));
    float *x = zalloc(n * d);
    mmo_embedding(w, v, d, ids, n, x);
    float *tmp_a = zalloc(n * d), *tmp_b = zalloc(n * kv), *tmp_c = zalloc(n * kv);
    for (int64_t l = 0; l < L; l++) {
        const float *bw = w + v * d + l * bp;
        const float *attn_norm = bw, *wq = attn_norm + d, *wk = wq + d * d, *wv = wk + d * kv,
                    *wo = wv + d * kv, *mlp_norm = wo + d * d, *wg = mlp_norm + d,
                    *wu = wg + d * ff, *wd = wu + d * ff;
        block_cache *s = &bc[l];
        s->x = x;
        s->xn1 = zalloc(n * d);
        mmo_rms_norm(x, attn_norm, n, d, c->norm_eps, s->xn1);
        memset(tmp_a, 0, sizeof(float) * (size_t)(n * d));
        memset(tmp_b, 0, sizeof(float) * (size_t)(n * kv));
        memset(tmp_c, 0, sizeof(float) * (size_t)(n * kv));
        mmo_gemm_nn(s->xn1, wq, tmp_a, n, d, d, nthreads);
        mmo_gemm_nn(s->xn1, wk, tmp_b, n, d, kv, nthreads);
        mmo_gemm_nn(s->xn1, wv, tmp_c, n, d, kv, nthreads);
        float *qh = zalloc(n * d), *kh = zalloc(n * kv);
        s->q = zalloc(n * d);
        s->k = zalloc(n * kv);
        s->v = zalloc(n * kv);
        split_heads(tmp_a, d, 0, b, t, nh, hd, qh);
        split_heads(tmp_b, kv, 0, b, t, hkv, hd, kh);
        split_heads(tmp_c, kv, 0, b, t, hkv, hd, s->v);
        mmo_apply_rope(qh, b * nh, t, hd, cos_t, sin_t, s->q);
        mmo_apply_rope(kh, b * hkv, t, hd, cos_t, sin_t, s->k);
        mmo_causal_attention(s->q, s->k, s->v, b, nh, hkv, t, hd, qh, nthreads);
        s->ctx = zalloc(n * d);
        merge_heads(qh, b, t, nh, hd, s->ctx);
        free(qh);
        free(kh);
        memset(tmp_a, 0, sizeof(float) * (size_t)(n * d));
        mmo_gemm_nn(s->ctx, wo, tmp_a, n, d, d, nthreads);
        s->hres = zalloc(n * d);
        memcpy(s->hres, x, sizeof(float) * (size_t)(n * d));
        add_inplace(s->hres, tmp_a, n * d);
        s->xn2 = zalloc(n * d);
        mmo_rms_norm(s->hres, mlp_norm, n, d, c->norm_eps, s->xn2);
        s->g = zalloc(n * ff);
        s->u = zalloc(n * ff);
        s->a = zalloc(n * ff);
        mmo_gemm_nn(s->xn2, wg, s->g, n, d, ff, nthreads);
        mmo_gemm_nn(s->xn2, wu, s->u, n, d, ff, nthreads);
        for (int64_t i = 0; i < n * ff; i++) s->a[i] = silu(s->g[i]) * s->u[i];
        memset(tmp_a, 0, sizeof(float) * (size_t)(n * d));
        mmo_gemm_nn(s->a, wd, tmp_a, n, ff, d, nthreads);
        x = zalloc(n * d);
        memcpy(x, s->hres, sizeof(float) * (size_t)(n * d));
        add_inplace(x, tmp_a, n * d);
    }
    const float *final_norm = w + v * d + L * bp;
    float *xf = x, *yf = zalloc(n * d), *logits = zalloc(n * v);
    mmo_rms_norm(xf, final_norm, n, d, c->norm_eps, yf);
    if (c->tie_embeddings)
        mmo_gemm_nt(yf, w, logits, n, d, v, nthreads);
    else
        mmo_gemm_nn(yf, final_norm + d, logits, n, d, v, nthreads);
    mmo_cross_entropy(logits, targets, n, v, loss);

    /* ---- backward ---- */
    float *dlogits = zalloc(n * v);
    mmo_cross_entropy_backward(logits, targets, n, v, 1.0f, dlogits);
    float *dy = zalloc(n * d);
    float *gfinal = grads + v * d + L * bp;
    if (c->tie_embeddings) {
        /* logits = y . E^T with E^T materialized (model.rs:163): d(E^T) =
         * y^T . dlogits, transposed back into dE. */
        /* dy = gemm_nt(dlogits, E^T): the copy of (E^T)^T is E itself */
        mmo_gemm_nn(dlogits, w, dy, n, v, d, nthreads);
        float *det = zalloc(d * v);
        mmo_gemm_tn(yf, dlogits, det, d, n, v, nthreads);
        for (int64_t j = 0; j < d; j++)
            for (int64_t r = 0; r < v; r++) grads[r * d + j] = det[j * v + r];
        free(det);
    } else {
        const float *head = final_norm + d;
        mmo_gemm_nt(dlogits, head, dy, n, v, d, nthreads);
        mmo_gemm_tn(yf, dlogits, gfinal + d, d, n, v, nthreads);
    }
    free(dlogits);
    float *dx = zalloc(n * d);
    mmo_rms_norm_backward(xf, final_norm, dy, n, d, c->norm_eps, dx, gfinal);

    float *dxn = zalloc(n * d), *dctx = zalloc(n * d), *dh = zalloc(n * ff),
          *dg = zalloc(n * ff), *du = zalloc(n * ff), *dnorm = zalloc(n * d);
    float *doh = zalloc(n * d), *dqh = zalloc(n * d), *dkh = zalloc(n * kv),
          *dvh = zalloc(n * kv), *dqr = zalloc(n * d), *dkr = zalloc(n * kv),
          *dqf = zalloc(n * d), *dkf = zalloc(n * kv), *dvf = zalloc(n * kv);
    for (int64_t l = L - 1; l >= 0; l--) {
        const float *bw = w + v * d + l * bp;
        float *gw = grads + v * d + l * bp;
        const float *attn_norm = bw, *wq = attn_norm + d, *wk = wq + d * d, *wv = wk + d * kv,
                    *wo = wv + d * kv, *mlp_norm = wo + d * d, *wg = mlp_norm + d,
                    *wu = wg + d * ff, *wd = wu + d * ff;
        float *g_attn_norm = gw, *g_wq = g_attn_norm + d, *g_wk = g_wq + d * d,
              *g_wv = g_wk + d * kv, *g_wo = g_wv + d * kv, *g_mlp_norm = g_wo + d * d,
              *g_wg = g_mlp_norm + d, *g_wu = g_wg + d * ff, *g_wd = g_wu + d * ff;
        block_cache *s = &bc[l];
        /* y = hres + a.Wd: dx is d(y) */
        mmo_matmul_backward(s->a, wd, dx, dh, g_wd, n, ff, d, nthreads);
        mmo_silu_mul_backward(s->g, s->u, dh, n * ff, dg, du);
        mmo_matmul_backward(s->xn2, wg, dg, dxn, g_wg, n, d, ff, nthreads);
        mmo_matmul_backward(s->xn2, wu, du, dnorm, g_wu, n, d, ff, nthreads);
        add_inplace(dxn, dnorm, n * d);
        mmo_rms_norm_backward(s->hres, mlp_norm, dxn, n, d, c->norm_eps, dnorm, g_mlp_norm);
        add_inplace(dx, dnorm, n * d); /* dx is now d(hres) */
        /* hres = x + ctx.Wo */
        mmo_matmul_backward(s->ctx, wo, dx, dctx, g_wo, n, d, d, nthreads);
        split_heads(dctx, d, 0, b, t, nh, hd, doh);
        mmo_causal_attention_backward(s->q, s->k, s->v, doh, b, nh, hkv, t, hd, dqh, dkh, dvh,
                                      nthreads);
        mmo_rope_backward(dqh, b * nh, t, hd, cos_t, sin_t, dqr);
        mmo_rope_backward(dkh, b * hkv, t, hd, cos_t, sin_t, dkr);
        merge_heads(dqr, b, t, nh, hd, dqf);
        merge_heads(dkr, b, t, hkv, hd, dkf);
        merge_heads(dvh, b, t, hkv, hd, dvf);
        mmo_matmul_backward(s->xn1, wq, dqf, dxn, g_wq, n, d, d, nthreads);
        mmo_matmul_backward(s->xn1, wk, dkf, dnorm, g_wk, n, d, kv, nthreads);
        add_inplace(dxn, dnorm, n * d);
        mmo_matmul_backward(s->xn1, wv, dvf, dnorm, g_wv, n, d, kv, nthreads);
        add_inplace(dxn, dnorm, n * d);
        mmo_rms_norm_backward(s->x, attn_norm, dxn, n, d, c->norm_eps, dnorm, g_attn_norm);
        add_inplace(dx, dnorm, n * d); /* dx is now d(x) of this block */
    }
    mmo_embedding_backward(ids, n, dx, d, grads);

    for (int64_t l = 0; l < L; l++) {
        block_cache *s = &bc[l];
        free(s->x); free(s->xn1); free(s->q); free(s->k); free(s->v); free(s->ctx);
        free(s->hres); free(s->xn2); free(s->g); free(s->u); free(s->a);
    }
    free(bc);
    free(xf); free(yf); free(logits); free(dy); free(dx); free(dxn); free(dctx); free(dh);
    free(dg); free(du); free(dnorm); free(doh); free(dqh); free(dkh); free(dvh); free(dqr);
    free(dkr); free(dqf); free(dkf); free(dvf); free(tmp_a); free(tmp_b); free(tmp_c);
    free(cos_t); free(sin_t);
    return MMO_OK;
}

/* clip.rs:30-33: sqrt of the f64 sum of squares, in parameter order. */
float mmo_global_norm(const float *g, int64_t n) {
    double sum = 0.0;
    for (int64_t i = 0; i < n; i++) sum += (double)g[i] * (double)g[i];
    return (float)sqrt(sum);
}

/* clip.rs:42-60: returns the norm before clipping; scales by
 * max/(norm + 1e-6) when norm > max. A non-finite norm is an error and
 * nothing changes. */
int32_t mmo_clip_global_norm(float *g, int64_t n, float max_norm, float *norm_out) {
    if (!(isfinite(max_norm) && max_norm > 0.0f)) return MMO_ERR_ARGUMENT;
    const float norm = mmo_global_norm(g, n);
    *norm_out = norm;
    if (!isfinite(norm)) return MMO_ERR_ARGUMENT;
    if (norm > max_norm) {
        const float factor = max_norm / (norm + 1e-6f);
        for (int64_t i = 0; i < n; i++) g[i] *= factor;
    }
    return MMO_OK;
}

/* schedule.rs:54-66 */
float mmo_warmup_cosine_lr(float max_lr, float min_lr, uint64_t warmup, uint64_t total,
                           uint64_t step) {
    const double mx = (double)max_lr, mn = (double)min_lr;
    if (step < warmup) return (float)(mx * (double)(step + 1) / (double)warmup);
    if (step >= total) return min_lr;
    const double progress = (double)(step - warmup) / (double)(total - warmup);
    return (float)(mn + 0.5 * (mx - mn) * (1.0 + cos(3.14159265358979323846 * progress)));
}

/* adamw.rs:180-214 for one parameter at optimizer step t (counting from 1):
 * bias terms in f64 (:185-187), then per element in f32, left to right. */
void mmo_adamw_update(float *w, const float *g, float *m, float *v, int64_t n, int32_t decays,
                      uint64_t t, float lr, float beta1, float beta2, float eps,
                      float weight_decay) {
    const double tt = (double)t;
    const float bias1 = (float)(1.0 - pow((double)beta1, tt));
    const float bias2_sqrt = (float)sqrt(1.0 - pow((double)beta2, tt));
    const float step_size = lr / bias1;
    const float decay = decays ? 1.0f - lr * weight_decay : 1.0f;
    for (int64_t i = 0; i < n; i++) {
        const float grad = g[i];
        w[i] *= decay;
        m[i] = beta1 * m[i] + (1.0f - beta1) * grad;
        v[i] = beta2 * v[i] + (1.0f - beta2) * grad * grad;
        w[i] -= step_size * m[i] / (sqrtf(v[i]) / bias2_sqrt + eps);
    }
}

/* AdamW::step over the flat parameter list (rank >= 2 parameters decay).
 * *steps is the optimizer's step count (incremented). */
int32_t mmo_adamw_step(const mmo_config *c, float *w, const float *g, float *m, float *v,
                       float lr, float beta1, float beta2, float eps, float weight_decay,
                       uint64_t *steps) {
    if (!(isfinite(lr) && lr >= 0.0f)) return MMO_ERR_ARGUMENT;
    const int64_t np = mmo_param_count(c);
    for (int64_t i = 0; i < np; i++)
        if (!isfinite(g[i])) return MMO_ERR_ARGUMENT;
    if (9 * c->n_layers + 3 > 4096) return MMO_ERR_CONFIG;
    int64_t off[4096], size[4096];
    int32_t rank[4096];
    const int64_t segs = param_segments(c, off, size, rank);
    *steps += 1;
    for (int64_t s = 0; s < segs; s++)
        mmo_adamw_update(w + off[s], g + off[s], m + off[s], v + off[s], size[s], rank[s] >= 2,
                         *steps, lr, beta1, beta2, eps, weight_decay);
    return MMO_OK;
}

/* Lab::new (lab.rs:159-214) and Lab::step_once (lab.rs:263-283): weights and
 * tokens from one Rng(seed), then `steps` training steps, each
 * lr = schedule(step), loss + gradients, norm = clip(grads), AdamW(lr).
 * hyper = {max_lr, min_lr, warmup_steps, total_steps, weight_decay,
 * clip_norm, beta1, beta2} (lab.rs:29-46), eps 1e-8 (lab.rs:192).
 * weights may be NULL; otherwise it receives the final weights. */
int32_t mmo_lab_train(const mmo_config *c, const double *hyper, uint64_t seed, int64_t batch,
                      int64_t seq, int64_t steps, float *losses, float *grad_norms, float *lrs,
                      float *weights, int32_t nthreads) {
    if (mmo_config_validate(c) != MMO_OK) return MMO_ERR_CONFIG;
    const int64_t np = mmo_param_count(c), n = batch * seq;
    float *w = zalloc(np), *g = zalloc(np), *m = zalloc(np), *vv = zalloc(np);
    int32_t *inputs = (int32_t *)malloc(sizeof(int32_t) * (size_t)n);
    int32_t *targets = (int32_t *)malloc(sizeof(int32_t) * (size_t)n);
    mmo_rng r;
    mmo_rng_seed(&r, seed);
    mmo_init_weights(c, 0.02f, &r, w, np);
    mmo_lab_tokens(&r, c->vocab_size, batch, seq, inputs, targets);
    const float max_lr = (float)hyper[0], min_lr = (float)hyper[1];
    const uint64_t warmup = (uint64_t)hyper[2], total = (uint64_t)hyper[3];
    const float wd = (float)hyper[4], clip = (float)hyper[5], b1 = (float)hyper[6],
                b2 = (float)hyper[7];
    uint64_t opt_steps = 0;
    int32_t st = MMO_OK;
    for (int64_t s = 0; s < steps && st == MMO_OK; s++) {
        const float lr = mmo_warmup_cosine_lr(max_lr, min_lr, warmup, total, (uint64_t)s);
        float loss = 0.0f, norm = 0.0f;
        st = mmo_forward_backward(c, w, inputs, targets, batch, seq, &loss, g, nthreads);
        if (st != MMO_OK) break;
        if (!isfinite(loss)) {
            st = MMO_ERR_ARGUMENT;
            break;
        }
        st = mmo_clip_global_norm(g, np, clip, &norm);
        if (st != MMO_OK) break;
        st = mmo_adamw_step(c, w, g, m, vv, lr, b1, b2, 1e-8f, wd, &opt_steps);
        if (losses) losses[s] = loss;
        if (grad_norms) grad_norms[s] = norm;
        if (lrs) lrs[s] = lr;
    }
    if (weights) memcpy(weights, w, sizeof(float) * (size_t)np);
    free(w); free(g); free(m); free(vv); free(inputs); free(targets);
    return st;
}
