// Host-side arithmetic that must match the reference bit for bit: the seeded
// RNG (midman-foundation/src/rng.rs), Tensor::randn (tensor.rs:158-162), the
// rotary tables (midman-nn/src/rope.rs:71-79) and the warmup-cosine learning
// rate (midman-optim/src/schedule.rs:25-66).
//
// Built with g++ -ffp-contract=off and glibc's libm, the toolchain the
// reference's Rust path matches on x86-64 (no FMA contraction; log, sqrt, sin,
// cos and pow from the platform libm, rng.rs:11-13).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "mmh_error.h"
#include "mmh_host.h"

namespace mmh {

namespace {

uint64_t splitmix64(uint64_t &state) {  // rng.rs:16-22
    state += 0x9E3779B97F4A7C15ULL;
    uint64_t z = state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

inline double to_f64(uint64_t x) {  // rng.rs:63-65
    return (double)(x >> 11) * (1.0 / 9007199254740992.0);
}

// One Box-Muller pair from two consecutive draws (rng.rs:78-83): returns the
// cos value, writes the sin value (the cached spare).
inline float box_muller(uint64_t x1, uint64_t x2, float *spare) {
    const double u1 = 1.0 - to_f64(x1);
    const double u2 = to_f64(x2);
    const double radius = std::sqrt(-2.0 * std::log(u1));
    const double theta = 6.283185307179586 * u2;  // TAU
    *spare = (float)(radius * std::sin(theta));
    return (float)(radius * std::cos(theta));
}

}  // namespace

HostRng HostRng::seed(uint64_t seed) {  // rng.rs:36-41
    HostRng r;
    uint64_t sm = seed;
    for (int i = 0; i < 4; ++i) r.s[i] = splitmix64(sm);
    r.has_spare = false;
    r.spare = 0.0f;
    return r;
}

uint64_t HostRng::next_u64() {  // rng.rs:44-55
    const uint64_t result = rotl(s[1] * 5, 7) * 9;
    const uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return result;
}

double HostRng::next_f64() { return to_f64(next_u64()); }

float HostRng::normal() {  // rng.rs:74-84
    if (has_spare) {
        has_spare = false;
        return spare;
    }
    const uint64_t a = next_u64();
    const uint64_t b = next_u64();
    const float c = box_muller(a, b, &spare);
    has_spare = true;
    return c;
}

uint64_t HostRng::below(uint64_t n) {  // rng.rs:91-105
    unsigned __int128 product = (unsigned __int128)next_u64() * n;
    uint64_t low = (uint64_t)product;
    if (low < n) {
        const uint64_t threshold = (0 - n) % n;
        while (low < threshold) {
            product = (unsigned __int128)next_u64() * n;
            low = (uint64_t)product;
        }
    }
    return (uint64_t)(product >> 64);
}

HostRng HostRng::fork(uint64_t stream) {  // rng.rs:117-119
    return HostRng::seed(next_u64() ^ (stream * 0x9E3779B97F4A7C15ull));
}

// The stream of pairs is generated sequentially in chunks (xoshiro is cheap);
// the transcendental work of each chunk is split over threads. Pair i's two
// draws and its position in dst are fixed by i alone, so the bits equal the
// sequential loop's.
void randn_parallel(HostRng &rng, float *dst, int64_t n, float stdv) {
    int64_t i = 0;
    if (n <= 0) return;
    if (rng.has_spare) {
        dst[i++] = stdv * rng.spare;
        rng.has_spare = false;
    }
    const int64_t pairs = (n - i) / 2;
    const bool odd = ((n - i) & 1) != 0;
    unsigned hw = std::thread::hardware_concurrency();
    const int nthreads = (int)std::max(1u, std::min(hw ? hw : 1u, 16u));
    const int64_t chunk = int64_t(1) << 20;
    std::vector<uint64_t> draws((size_t)std::min<int64_t>(pairs, chunk) * 2 + 2);
    for (int64_t base = 0; base < pairs; base += chunk) {
        const int64_t cnt = std::min(chunk, pairs - base);
        for (int64_t j = 0; j < 2 * cnt; ++j) draws[(size_t)j] = rng.next_u64();
        float *out = dst + i + 2 * base;
        auto work = [&](int64_t lo, int64_t hi) {
            for (int64_t j = lo; j < hi; ++j) {
                float sp;
                const float c = box_muller(draws[(size_t)(2 * j)], draws[(size_t)(2 * j + 1)], &sp);
                out[2 * j] = stdv * c;
                out[2 * j + 1] = stdv * sp;
            }
        };
        if (cnt < 65536 || nthreads == 1) {
            work(0, cnt);
        } else {
            std::vector<std::thread> pool;
            for (int t = 1; t < nthreads; ++t)
                pool.emplace_back(work, cnt * t / nthreads, cnt * (t + 1) / nthreads);
            work(0, cnt / nthreads);
            for (auto &th : pool) th.join();
        }
    }
    if (odd) dst[n - 1] = stdv * rng.normal();  // leaves the spare cached
}

void rope_tables_host(int64_t head_dim, int64_t max_seq_len, float theta, float *cos_t,
                      float *sin_t) {  // rope.rs:71-79
    const int64_t half = head_dim / 2;
    for (int64_t pos = 0; pos < max_seq_len; ++pos) {
        for (int64_t i = 0; i < half; ++i) {
            const double frequency = std::pow((double)theta, -(double)i / (double)half);
            const double angle = (double)pos * frequency;
            cos_t[pos * half + i] = (float)std::cos(angle);
            sin_t[pos * half + i] = (float)std::sin(angle);
        }
    }
}

}  // namespace mmh

extern "C" {

int32_t mmh_warmup_cosine_lr(float max_lr, float min_lr, uint64_t warmup_steps,
                             uint64_t total_steps, uint64_t step, float *lr_out) {
    return mmh::guard([&] {
        if (!lr_out) mmh::fail(MMH_ERR_ARGUMENT, "lr is a null pointer");
        // schedule.rs:25-48
        if (!(std::isfinite(max_lr) && max_lr > 0.0f))
            mmh::fail(MMH_ERR_ARGUMENT, "schedule: max_lr must be positive and finite");
        if (!(std::isfinite(min_lr) && min_lr >= 0.0f && min_lr <= max_lr))
            mmh::fail(MMH_ERR_ARGUMENT, "schedule: min_lr must be in [0, max_lr]");
        if (warmup_steps >= total_steps)
            mmh::fail(MMH_ERR_ARGUMENT, "schedule: warmup_steps must be below total_steps");
        // schedule.rs:54-66
        const double mx = (double)max_lr, mn = (double)min_lr;
        if (step < warmup_steps) {
            *lr_out = (float)(mx * (double)(step + 1) / (double)warmup_steps);
        } else if (step >= total_steps) {
            *lr_out = min_lr;
        } else {
            const double progress =
                (double)(step - warmup_steps) / (double)(total_steps - warmup_steps);
            *lr_out = (float)(mn + 0.5 * (mx - mn) * (1.0 + std::cos(M_PI * progress)));
        }
        return MMH_OK;
    });
}

}  // extern "C"
