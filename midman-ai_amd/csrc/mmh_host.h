// Host-only declarations (no HIP headers), shared by host_math.cpp (built with
// g++) and the HIP translation units.
#pragma once

#include <cstddef>
#include <cstdint>

namespace mmh {

// midman-foundation/src/rng.rs restated: SplitMix64 seeding, xoshiro256**,
// Box-Muller normals with a cached spare, Lemire's below().
struct HostRng {
    uint64_t s[4];
    bool has_spare = false;
    float spare = 0.0f;
    static HostRng seed(uint64_t seed);
    uint64_t next_u64();
    double next_f64();
    float normal();
    uint64_t below(uint64_t n);
    // rng.rs:117-119: a generator for a numbered stream; advances this one.
    HostRng fork(uint64_t stream);
};

// Tensor::randn (tensor.rs:158-162) for n values: dst[i] = std * normal(),
// the same bits as the sequential loop, with the transcendental work spread
// over threads.
void randn_parallel(HostRng &rng, float *dst, int64_t n, float stdv);

// RotaryTables::new (rope.rs:54-85): [max_seq_len, head_dim/2] cos and sin.
void rope_tables_host(int64_t head_dim, int64_t max_seq_len, float theta, float *cos_t,
                      float *sin_t);

// SHA-256 (FIPS 180-4; midman-data/src/hash.rs), incremental: update with
// pieces of any size, then finalize once.
struct Sha256 {
    uint32_t h[8];
    uint8_t buf[64];
    size_t nbuf = 0;
    uint64_t total = 0;
    Sha256();
    void update(const uint8_t *p, size_t n);
    void finalize(uint8_t out[32]);
};
void sha256(const uint8_t *p, size_t n, uint8_t out[32]);
// The compression path: mode 0 = the best the CPU has, 1 = portable, 2 = the
// x86 SHA extensions when present. Returns the path in use (1 or 2).
int sha256_select(int mode);

}  // namespace mmh
