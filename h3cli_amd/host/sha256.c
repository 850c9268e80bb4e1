/* SHA-256 as FIPS 180-4 section 6.2 defines it. The 64 round constants and the
 * 8 initial hash words are the first 32 bits of the fractional parts of the cube
 * roots of the first 64 primes and of the square roots of the first 8 (FIPS
 * 180-4 4.2.2, 5.3.3); they are derived here exactly, with integer roots, once. */
#include "sha256.h"
#include <pthread.h>
#include <string.h>

static uint32_t round_k[64], initial_h[8];
static pthread_once_t constants_once = PTHREAD_ONCE_INIT;

/* floor(p^(1/n) * 2^32) mod 2^32 for n = 2 or 3: the largest x with
 * x^n <= p * 2^(32 n), by bisection in 128-bit integers. */
static uint32_t root_fraction(unsigned p, int n) {
    typedef unsigned __int128 u128;
    const u128 target = (u128)p << (32 * n);
    uint64_t lo = 0, hi = (uint64_t)1 << 40;                  /* p < 2^9: roots < 2^(32 + 3) */
    while (hi - lo > 1) {
        uint64_t mid = lo + (hi - lo) / 2;
        u128 v = (u128)mid * mid;
        if (n == 3) v *= mid;
        if (v <= target) lo = mid; else hi = mid;
    }
    return (uint32_t)lo;
}

static void derive_constants(void) {
    unsigned primes[64], count = 0;
    for (unsigned c = 2; count < 64; c++) {
        int prime = 1;
        for (unsigned i = 0; i < count && primes[i] * primes[i] <= c; i++)
            if (c % primes[i] == 0) { prime = 0; break; }
        if (prime) primes[count++] = c;
    }
    for (unsigned i = 0; i < 64; i++) round_k[i] = root_fraction(primes[i], 3);
    for (unsigned i = 0; i < 8; i++) initial_h[i] = root_fraction(primes[i], 2);
}

static inline uint32_t rotr32(uint32_t x, unsigned r) { return (x >> r) | (x << (32 - r)); }

static void compress(uint32_t h[8], const uint8_t m[64]) {
    uint32_t w[64];
    for (unsigned t = 0; t < 16; t++)
        w[t] = (uint32_t)m[4 * t] << 24 | (uint32_t)m[4 * t + 1] << 16 | (uint32_t)m[4 * t + 2] << 8 | m[4 * t + 3];
    for (unsigned t = 16; t < 64; t++) {
        const uint32_t s0 = rotr32(w[t - 15], 7) ^ rotr32(w[t - 15], 18) ^ (w[t - 15] >> 3);
        const uint32_t s1 = rotr32(w[t - 2], 17) ^ rotr32(w[t - 2], 19) ^ (w[t - 2] >> 10);
        w[t] = w[t - 16] + s0 + w[t - 7] + s1;
    }
    uint32_t v[8];
    memcpy(v, h, sizeof(v));
    for (unsigned t = 0; t < 64; t++) {
        const uint32_t e = v[4], a = v[0];
        const uint32_t ch = (e & v[5]) ^ (~e & v[6]);
        const uint32_t maj = (a & v[1]) ^ (a & v[2]) ^ (v[1] & v[2]);
        const uint32_t t1 = v[7] + (rotr32(e, 6) ^ rotr32(e, 11) ^ rotr32(e, 25)) + ch + round_k[t] + w[t];
        const uint32_t t2 = (rotr32(a, 2) ^ rotr32(a, 13) ^ rotr32(a, 22)) + maj;
        memmove(v + 1, v, 7 * sizeof(uint32_t));
        v[4] += t1;
        v[0] = t1 + t2;
    }
    for (unsigned i = 0; i < 8; i++) h[i] += v[i];
}

void h3hip_sha256_init(h3hip_sha256 *s) {
    pthread_once(&constants_once, derive_constants);
    memcpy(s->h, initial_h, sizeof(s->h));
    s->length = 0;
}

void h3hip_sha256_update(h3hip_sha256 *s, const void *data, size_t bytes) {
    const uint8_t *p = (const uint8_t *)data;
    size_t fill = (size_t)(s->length % 64);
    s->length += bytes;
    if (fill) {
        size_t take = 64 - fill < bytes ? 64 - fill : bytes;
        memcpy(s->block + fill, p, take);
        p += take; bytes -= take; fill += take;
        if (fill < 64) return;
        compress(s->h, s->block);
    }
    for (; bytes >= 64; p += 64, bytes -= 64) compress(s->h, p);
    memcpy(s->block, p, bytes);
}

void h3hip_sha256_final(h3hip_sha256 *s, uint8_t digest[32]) {
    const uint64_t bits = s->length * 8;
    size_t fill = (size_t)(s->length % 64);
    s->block[fill++] = 0x80;
    if (fill > 56) {
        memset(s->block + fill, 0, 64 - fill);
        compress(s->h, s->block);
        fill = 0;
    }
    memset(s->block + fill, 0, 56 - fill);
    for (unsigned i = 0; i < 8; i++) s->block[56 + i] = (uint8_t)(bits >> (56 - 8 * i));
    compress(s->h, s->block);
    for (unsigned i = 0; i < 32; i++) digest[i] = (uint8_t)(s->h[i / 4] >> (24 - 8 * (i % 4)));
    memset(s, 0, sizeof(*s));
}
