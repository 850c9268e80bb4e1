/* CPU oracle — TEST INFRASTRUCTURE ONLY (see oracle.h). Sage quantization and
 * quantized-operand attention. The operation order of the
 * K mean and of every scale/code follows the stated contract exactly, so the
 * integer codes and fp32 scales are comparable bit for bit with the device. */
#include "oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define D 128u
#define PARTIAL_ROWS 256u

/* e4m3fn value of a code (sign, 4-bit exponent bias 7, 3-bit mantissa; 0x7f NaN). */
float oracle_e4m3_to_f32(uint8_t c) {
    unsigned e = (c >> 3) & 15u, m = c & 7u;
    float mag;
    if ((c & 0x7f) == 0x7f) return NAN;
    if (e == 0) mag = ldexpf((float)m, -9);
    else mag = ldexpf(1.0f + (float)m / 8.0f, (int)e - 7);
    return (c & 0x80) ? -mag : mag;
}

/* Encode by exhaustive nearest-value search over the 127 non-negative finite
 * codes, ties to the even code (even mantissa LSB), saturating at 448. This is
 * deliberately a different algorithm from the device's bit manipulation. */
uint8_t oracle_f32_to_e4m3(float x) {
    if (isnan(x)) return (uint8_t)(signbit(x) ? 0xff : 0x7f);
    uint8_t sign = signbit(x) ? 0x80 : 0x00;
    double a = fabs((double)x);
    unsigned best = 0;
    double best_err = INFINITY;
    for (unsigned c = 0; c <= 0x7e; c++) {
        double val = oracle_e4m3_to_f32((uint8_t)c), err = fabs(val - a);
        if (err < best_err || (err == best_err && (c & 1u) == 0)) { best = c; best_err = err; }
    }
    return sign | (uint8_t)best;
}

unsigned oracle_sage_v_position(unsigned j) {
    /* Key j of a 64-key tile is held by lane half hf = (j%8)/4 as byte
     * mb*16 + r of its P operand, mb = j/32, r = ((j%32)/8)*4 + j%4. */
    unsigned mb = j / 32, j32 = j % 32, hf = (j32 % 8) / 4, r = (j32 / 8) * 4 + j32 % 4;
    return hf * 32 + mb * 16 + r;
}

void oracle_k_mean_f64(const uint16_t *k, unsigned seq, unsigned heads, double *mean) {
    for (unsigned h = 0; h < heads; h++)
        for (unsigned d = 0; d < D; d++) {
            double s = 0;
            for (unsigned r = 0; r < seq; r++) s += oracle_bf16_to_f32(k[((size_t)r * heads + h) * D + d]);
            mean[h * D + d] = s / seq;
        }
}

static int8_t code_int8(float x, float scale) {
    float q = x / scale;
    int c = (int)(q + (q >= 0.f ? 0.5f : -0.5f));
    return (int8_t)(c > 127 ? 127 : c < -127 ? -127 : c);
}

void oracle_sage_pack(const uint16_t *q, const uint16_t *k, const uint16_t *v, unsigned seq,
                      unsigned heads, int8_t *q8, int8_t *k8, uint8_t *v8, float *q_scale,
                      float *k_scale, float *v_scale, uint16_t *k_mean) {
    unsigned padded = (seq + 63) / 64 * 64, blocks = padded / 64;
    unsigned partials = (seq + PARTIAL_ROWS - 1) / PARTIAL_ROWS;
    float *recip = malloc(sizeof(float) * heads * D);
#pragma omp parallel for
    for (unsigned h = 0; h < heads; h++) {
        for (unsigned d = 0; d < D; d++) {
            /* K sum: fp32, rows of each 256-row partial in order, partials in order. */
            float total = 0.f, vmax = 0.f;
            for (unsigned p = 0; p < partials; p++) {
                float part = 0.f;
                unsigned end = (p + 1) * PARTIAL_ROWS < seq ? (p + 1) * PARTIAL_ROWS : seq;
                for (unsigned r = p * PARTIAL_ROWS; r < end; r++) {
                    size_t at = ((size_t)r * heads + h) * D + d;
                    part = part + oracle_bf16_to_f32(k[at]);
                    float y = fabsf(oracle_bf16_to_f32(v[at]));
                    if (y > vmax) vmax = y;
                }
                total = total + part;
            }
            k_mean[h * D + d] = oracle_f32_to_bf16(total / (float)seq);
            v_scale[h * D + d] = vmax / 448.0f;
            recip[h * D + d] = vmax > 0.f ? 448.0f / vmax : 0.f;
        }
        for (unsigned b = 0; b < blocks; b++) {
            for (int which = 0; which < 2; which++) {
                const uint16_t *src = which ? k : q;
                float vals[64 * D], amax = 0.f;
                for (unsigned i = 0; i < 64; i++)
                    for (unsigned d = 0; d < D; d++) {
                        unsigned r = b * 64 + i;
                        float x = 0.f;
                        if (r < seq) {
                            x = oracle_bf16_to_f32(src[((size_t)r * heads + h) * D + d]);
                            if (which) x = oracle_bf16_to_f32(oracle_f32_to_bf16(x - oracle_bf16_to_f32(k_mean[h * D + d])));
                        }
                        vals[i * D + d] = x;
                        if (fabsf(x) > amax) amax = fabsf(x);
                    }
                float scale = fmaf(amax, 1.0f / 127.0f, 1e-7f);
                (which ? k_scale : q_scale)[h * blocks + b] = scale;
                int8_t *dst = (which ? k8 : q8) + ((size_t)h * padded + b * 64) * D;
                for (unsigned i = 0; i < 64 * D; i++) dst[i] = code_int8(vals[i], scale);
            }
            for (unsigned d = 0; d < D; d++)
                for (unsigned j = 0; j < 64; j++) {
                    unsigned r = b * 64 + j;
                    float x = r < seq ? oracle_bf16_to_f32(v[((size_t)r * heads + h) * D + d]) : 0.f;
                    v8[((size_t)h * D + d) * padded + b * 64 + oracle_sage_v_position(j)] =
                        oracle_f32_to_e4m3(x * recip[h * D + d]);
                }
        }
    }
    free(recip);
}

void oracle_sage_attention(double *out, const int8_t *q8, const int8_t *k8, const uint8_t *v8,
                           const float *q_scale, const float *k_scale, const float *v_scale,
                           unsigned seq, unsigned heads, float scale, const uint8_t *mask,
                           unsigned block, unsigned row0, unsigned row1) {
    unsigned padded = (seq + 63) / 64 * 64, blocks = padded / 64;
    unsigned kblocks = mask ? (seq + block - 1) / block : 0;
    long total = (long)(row1 - row0) * heads;
#pragma omp parallel
    {
        double *s = malloc(sizeof(double) * seq);
#pragma omp for schedule(dynamic, 4)
        for (long i = 0; i < total; i++) {
            unsigned h = (unsigned)(i % heads), row = row0 + (unsigned)(i / heads);
            const int8_t *qr = q8 + ((size_t)h * padded + row) * D;
            double m = -INFINITY, l = 0;
            for (unsigned j = 0; j < seq; j++) {
                if (mask && !mask[(size_t)(row / block) * kblocks + j / block]) { s[j] = -INFINITY; continue; }
                const int8_t *kr = k8 + ((size_t)h * padded + j) * D;
                int32_t dot = 0;
                for (unsigned d = 0; d < D; d++) dot += (int32_t)qr[d] * kr[d];
                s[j] = (double)dot * q_scale[h * blocks + row / 64] * k_scale[h * blocks + j / 64] * scale;
                if (s[j] > m) m = s[j];
            }
            double *o = out + ((size_t)(row - row0) * heads + h) * D;
            for (unsigned d = 0; d < D; d++) o[d] = 0;
            if (m == -INFINITY) continue;
            for (unsigned j = 0; j < seq; j++) { s[j] = exp(s[j] - m); l += s[j]; }
            for (unsigned j = 0; j < seq; j++) {
                if (s[j] == 0) continue;
                for (unsigned d = 0; d < D; d++) {
                    uint8_t c = v8[((size_t)h * D + d) * padded + (j / 64) * 64 + oracle_sage_v_position(j % 64)];
                    o[d] += s[j] * oracle_e4m3_to_f32(c);
                }
            }
            for (unsigned d = 0; d < D; d++) o[d] = o[d] * v_scale[h * D + d] / l;
        }
        free(s);
    }
}
