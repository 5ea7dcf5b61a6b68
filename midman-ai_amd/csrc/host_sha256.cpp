// SHA-256 (FIPS 180-4) for the token-shard checksum (midman-data/src/hash.rs,
// used by shard.rs:132 and :205).
//
// Two compression paths over the same state: the x86 SHA extensions
// (sha256rnds2 / sha256msg1 / sha256msg2, the arrangement Intel describes in
// "Intel SHA Extensions", 2013), chosen at run time when the CPU has them, and
// a portable one. The round constants and the initial state are derived here
// from their definitions (the first 32 bits of the fractional parts of the
// cube roots of the first 64 primes, and of the square roots of the first 8)
// rather than typed in.
#include <cpuid.h>
#include <immintrin.h>

#include <atomic>
#include <cstdint>
#include <cstring>

#include "mmh_host.h"

namespace mmh {

namespace {

struct Constants {
    alignas(16) uint32_t k[64];
    uint32_t h0[8];
};

// floor(cbrt(n)) and floor(sqrt(n)) for n < 2^110, by bisection.
uint64_t icbrt(unsigned __int128 n) {
    uint64_t lo = 0, hi = (uint64_t)1 << 37;  // (2^37)^3 = 2^111 > n
    while (hi - lo > 1) {
        const uint64_t mid = lo + (hi - lo) / 2;
        const unsigned __int128 c = (unsigned __int128)mid * mid * mid;
        if (c <= n) lo = mid; else hi = mid;
    }
    return lo;
}

uint64_t isqrt(unsigned __int128 n) {
    uint64_t lo = 0, hi = (uint64_t)1 << 56;
    while (hi - lo > 1) {
        const uint64_t mid = lo + (hi - lo) / 2;
        if ((unsigned __int128)mid * mid <= n) lo = mid; else hi = mid;
    }
    return lo;
}

Constants make_constants() {
    Constants c;
    int primes[64], count = 0;
    for (int p = 2; count < 64; ++p) {
        bool prime = true;
        for (int q = 2; q * q <= p; ++q)
            if (p % q == 0) { prime = false; break; }
        if (prime) primes[count++] = p;
    }
    // frac(cbrt(p)) * 2^32 = floor(cbrt(p * 2^96)) mod 2^32
    for (int i = 0; i < 64; ++i)
        c.k[i] = (uint32_t)icbrt((unsigned __int128)primes[i] << 96);
    // frac(sqrt(p)) * 2^32 = floor(sqrt(p * 2^64)) mod 2^32
    for (int i = 0; i < 8; ++i) c.h0[i] = (uint32_t)isqrt((unsigned __int128)primes[i] << 64);
    return c;
}

const Constants &constants() {
    static const Constants c = make_constants();
    return c;
}

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

void compress_portable(uint32_t h[8], const uint8_t *p, size_t blocks) {
    const uint32_t *K = constants().k;
    uint32_t w[64];
    for (; blocks; --blocks, p += 64) {
        for (int t = 0; t < 16; ++t)
            w[t] = (uint32_t)p[4 * t] << 24 | (uint32_t)p[4 * t + 1] << 16 |
                   (uint32_t)p[4 * t + 2] << 8 | (uint32_t)p[4 * t + 3];
        for (int t = 16; t < 64; ++t) {
            const uint32_t s0 = rotr(w[t - 15], 7) ^ rotr(w[t - 15], 18) ^ (w[t - 15] >> 3);
            const uint32_t s1 = rotr(w[t - 2], 17) ^ rotr(w[t - 2], 19) ^ (w[t - 2] >> 10);
            w[t] = w[t - 16] + s0 + w[t - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6],
                 hh = h[7];
        for (int t = 0; t < 64; ++t) {
            const uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
            const uint32_t ch = (e & f) ^ (~e & g);
            const uint32_t t1 = hh + S1 + ch + K[t] + w[t];
            const uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
            const uint32_t maj = (a & b) ^ (a & c) ^ (b & c);
            const uint32_t t2 = S0 + maj;
            hh = g;
            g = f;
            f = e;
            e = d + t1;
            d = c;
            c = b;
            b = a;
            a = t1 + t2;
        }
        h[0] += a; h[1] += b; h[2] += c; h[3] += d;
        h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
    }
}

// The state lives in two registers as (A, B, E, F) and (C, D, G, H), the
// order sha256rnds2 takes; each call does two rounds with the two message +
// constant words in the low half of its third operand. The schedule keeps
// four groups of four words: group g >= 4 is
//   msg2(msg1(W[g-4], W[g-3]) + (W[g-2] words 1..3, W[g-1] word 0), W[g-1]).
__attribute__((target("sha,sse4.1,ssse3"))) void compress_shani(uint32_t h[8], const uint8_t *p,
                                                                size_t blocks) {
    const uint32_t *K = constants().k;
    const __m128i bswap = _mm_set_epi64x(0x0c0d0e0f08090a0bll, 0x0405060700010203ll);
    __m128i t = _mm_loadu_si128((const __m128i *)&h[0]);   // a b c d
    __m128i s1 = _mm_loadu_si128((const __m128i *)&h[4]);  // e f g h
    t = _mm_shuffle_epi32(t, 0xB1);                        // b a d c
    s1 = _mm_shuffle_epi32(s1, 0x1B);                      // h g f e
    __m128i s0 = _mm_alignr_epi8(t, s1, 8);                // f e b a = ABEF
    s1 = _mm_blend_epi16(s1, t, 0xF0);                     // h g d c = CDGH
    for (; blocks; --blocks, p += 64) {
        const __m128i save0 = s0, save1 = s1;
        __m128i w[4];
        for (int g = 0; g < 16; ++g) {
            __m128i cur;
            if (g < 4) {
                cur = _mm_shuffle_epi8(_mm_loadu_si128((const __m128i *)(p + 16 * g)), bswap);
            } else {
                const __m128i a = _mm_sha256msg1_epu32(w[g & 3], w[(g + 1) & 3]);
                const __m128i b = _mm_alignr_epi8(w[(g + 3) & 3], w[(g + 2) & 3], 4);
                cur = _mm_sha256msg2_epu32(_mm_add_epi32(a, b), w[(g + 3) & 3]);
            }
            w[g & 3] = cur;
            __m128i m = _mm_add_epi32(cur, _mm_load_si128((const __m128i *)&K[4 * g]));
            s1 = _mm_sha256rnds2_epu32(s1, s0, m);
            m = _mm_shuffle_epi32(m, 0x0E);
            s0 = _mm_sha256rnds2_epu32(s0, s1, m);
        }
        s0 = _mm_add_epi32(s0, save0);
        s1 = _mm_add_epi32(s1, save1);
    }
    t = _mm_shuffle_epi32(s0, 0x1B);       // a b e f -> reversed
    s1 = _mm_shuffle_epi32(s1, 0xB1);      // d c h g
    s0 = _mm_blend_epi16(t, s1, 0xF0);     // a b c d
    s1 = _mm_alignr_epi8(s1, t, 8);        // e f g h
    _mm_storeu_si128((__m128i *)&h[0], s0);
    _mm_storeu_si128((__m128i *)&h[4], s1);
}

bool cpu_has_sha() {
    unsigned a = 0, b = 0, c = 0, d = 0;
    if (!__get_cpuid(1, &a, &b, &c, &d)) return false;
    const bool ssse3 = c & (1u << 9), sse41 = c & (1u << 19);
    if (!__get_cpuid_count(7, 0, &a, &b, &c, &d)) return false;
    return ssse3 && sse41 && (b & (1u << 29));
}

// 0 = not chosen yet, 1 = portable, 2 = SHA extensions.
std::atomic<int> g_impl{0};

int impl() {
    int v = g_impl.load(std::memory_order_relaxed);
    if (!v) {
        v = cpu_has_sha() ? 2 : 1;
        g_impl.store(v, std::memory_order_relaxed);
    }
    return v;
}

void compress(uint32_t h[8], const uint8_t *p, size_t blocks) {
    if (impl() == 2) compress_shani(h, p, blocks);
    else compress_portable(h, p, blocks);
}

}  // namespace

int sha256_select(int mode) {
    if (mode == 1) g_impl.store(1);
    else if (mode == 2 && cpu_has_sha()) g_impl.store(2);
    else if (mode == 0) g_impl.store(cpu_has_sha() ? 2 : 1);
    return impl();
}

Sha256::Sha256() {
    std::memcpy(h, constants().h0, sizeof h);
}

void Sha256::update(const uint8_t *p, size_t n) {
    if (n == 0) return;  // p may be null for an empty piece
    total += n;
    if (nbuf) {
        const size_t take = n < 64 - nbuf ? n : 64 - nbuf;
        std::memcpy(buf + nbuf, p, take);
        nbuf += take;
        p += take;
        n -= take;
        if (nbuf < 64) return;
        compress(h, buf, 1);
        nbuf = 0;
    }
    if (n >= 64) {
        compress(h, p, n / 64);
        p += n / 64 * 64;
        n %= 64;
    }
    if (n) std::memcpy(buf, p, n);
    nbuf = n;
}

void Sha256::finalize(uint8_t out[32]) {
    const uint64_t bits = total * 8;
    uint8_t pad[72] = {0x80};
    const size_t padlen = (nbuf < 56 ? 56 : 120) - nbuf;
    for (int i = 0; i < 8; ++i) pad[padlen + i] = (uint8_t)(bits >> (56 - 8 * i));
    update(pad, padlen + 8);
    for (int i = 0; i < 8; ++i)
        for (int j = 0; j < 4; ++j) out[4 * i + j] = (uint8_t)(h[i] >> (24 - 8 * j));
}

void sha256(const uint8_t *p, size_t n, uint8_t out[32]) {
    Sha256 s;
    s.update(p, n);
    s.finalize(out);
}

}  // namespace mmh
