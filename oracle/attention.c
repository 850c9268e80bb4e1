/* CPU oracle — TEST INFRASTRUCTURE ONLY (see oracle.h). Attention restatements. */
#include "oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int oracle_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

float oracle_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16; float f; memcpy(&f, &u, 4); return f;
}

uint16_t oracle_f32_to_bf16(float f) {
    uint32_t u; memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1f, man = h & 0x3ff, u;
    if (exp == 0) {
        if (!man) u = sign;
        else { /* subnormal: man * 2^-24 */
            float f = (float)man * 5.9604644775390625e-8f;
            memcpy(&u, &f, 4); u |= sign;
        }
    } else if (exp == 31) u = sign | 0x7f800000u | (man << 13);
    else u = sign | ((exp + 112) << 23) | (man << 13);
    float f; memcpy(&f, &u, 4); return f;
}

/* One (row, head) of the online-softmax operator of src/cuda/cuda_attention.cuh:7-51:
 * keys in tiles; the tile's scores are dot products accumulated by fmaf in
 * channel order, then multiplied by the scale (scale_mode 0); the running max is
 * updated once per tile with alpha = expf(old - new); the tile's weights
 * expf(score - new) are summed into the denominator, and the value accumulator
 * is rescaled by alpha then accumulates weight * v by fmaf in key order. */
static void online_row(float *out, const float *q, const float *k, const float *v, unsigned seq,
                       unsigned heads, unsigned dim, float scale, unsigned tile, unsigned row,
                       unsigned head, const uint8_t *mask, unsigned block, unsigned kblocks,
                       unsigned row0, float *w, float *acc) {
    const float *qr = q + ((size_t)row * heads + head) * dim;
    float maximum = -INFINITY, denominator = 0.f;
    for (unsigned d = 0; d < dim; d++) acc[d] = 0.f;
    unsigned step = mask ? block : tile;
    for (unsigned first = 0; first < seq; first += step) {
        if (mask && !mask[(size_t)(row / block) * kblocks + first / block]) continue;
        unsigned count = seq - first < step ? seq - first : step;
        float next = maximum;
        for (unsigned j = 0; j < count; j++) {
            const float *kr = k + ((size_t)(first + j) * heads + head) * dim;
            float dot = 0.f;
            for (unsigned d = 0; d < dim; d++) dot = fmaf(qr[d], kr[d], dot);
            w[j] = dot * scale;
            next = fmaxf(next, w[j]);
        }
        float alpha = expf(maximum - next), tile_sum = 0.f;
        for (unsigned j = 0; j < count; j++) { w[j] = expf(w[j] - next); tile_sum += w[j]; }
        denominator = denominator * alpha + tile_sum;
        maximum = next;
        for (unsigned d = 0; d < dim; d++) {
            float value = acc[d] * alpha;
            for (unsigned j = 0; j < count; j++)
                value = fmaf(w[j], v[((size_t)(first + j) * heads + head) * dim + d], value);
            acc[d] = value;
        }
    }
    float *o = out + ((size_t)(row - row0) * heads + head) * dim;
    for (unsigned d = 0; d < dim; d++) o[d] = denominator > 0.f ? acc[d] / denominator : 0.f;
}

static void run_rows(float *out, const float *q, const float *k, const float *v, unsigned seq,
                     unsigned heads, unsigned dim, float scale, unsigned tile, const uint8_t *mask,
                     unsigned block, unsigned row0, unsigned row1) {
    unsigned kblocks = mask ? (seq + block - 1) / block : 0;
    unsigned step = mask ? block : tile;
    long total = (long)(row1 - row0) * heads;
#pragma omp parallel
    {
        float *w = malloc(sizeof(float) * step), *acc = malloc(sizeof(float) * dim);
#pragma omp for schedule(dynamic, 16)
        for (long i = 0; i < total; i++) {
            unsigned head = (unsigned)(i % heads), row = row0 + (unsigned)(i / heads);
            online_row(out, q, k, v, seq, heads, dim, scale, tile, row, head, mask, block, kblocks, row0, w, acc);
        }
        free(w); free(acc);
    }
}

void oracle_attention(float *out, const float *q, const float *k, const float *v, unsigned seq,
                      unsigned heads, unsigned dim, float scale, unsigned tile, unsigned row0,
                      unsigned row1) {
    run_rows(out, q, k, v, seq, heads, dim, scale, tile ? tile : 64, NULL, 0, row0, row1);
}

void oracle_attention_masked(float *out, const float *q, const float *k, const float *v,
                             unsigned seq, unsigned heads, unsigned dim, float scale,
                             const uint8_t *mask, unsigned block, unsigned row0, unsigned row1) {
    run_rows(out, q, k, v, seq, heads, dim, scale, block, mask, block, row0, row1);
}

void oracle_attention_f64(double *out, const float *q, const float *k, const float *v,
                          unsigned seq, unsigned heads, unsigned dim, double scale,
                          unsigned row0, unsigned row1) {
    long total = (long)(row1 - row0) * heads;
#pragma omp parallel
    {
        double *s = malloc(sizeof(double) * seq);
#pragma omp for schedule(dynamic, 4)
        for (long i = 0; i < total; i++) {
            unsigned head = (unsigned)(i % heads), row = row0 + (unsigned)(i / heads);
            const float *qr = q + ((size_t)row * heads + head) * dim;
            double m = -INFINITY, l = 0;
            for (unsigned j = 0; j < seq; j++) {
                const float *kr = k + ((size_t)j * heads + head) * dim;
                double dot = 0;
                for (unsigned d = 0; d < dim; d++) dot += (double)qr[d] * kr[d];
                s[j] = dot * scale;
                if (s[j] > m) m = s[j];
            }
            for (unsigned j = 0; j < seq; j++) { s[j] = exp(s[j] - m); l += s[j]; }
            double *o = out + ((size_t)(row - row0) * heads + head) * dim;
            for (unsigned d = 0; d < dim; d++) o[d] = 0;
            for (unsigned j = 0; j < seq; j++) {
                const float *vr = v + ((size_t)j * heads + head) * dim;
                for (unsigned d = 0; d < dim; d++) o[d] += s[j] * vr[d];
            }
            for (unsigned d = 0; d < dim; d++) o[d] /= l;
        }
        free(s);
    }
}
