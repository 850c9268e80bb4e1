/* FP8 W8A8 projection (reference src/cuda/cuda_quant.cuh:26-104, 339-398), CPU
 * restatement. TEST INFRASTRUCTURE ONLY: used by tests/ as the checker of the
 * HIP FP8 packing and GEMM.
 *
 * Tensorwide E4M3 packing (cuda_quant.cuh:26-49): amax = max |x| over the
 * tensor, scale = max(amax / 448, 1e-20) (IEEE division), code = E4M3 of
 * x / scale, round to nearest even, saturating at 448 (__NV_SATFINITE); rows
 * beyond the tensor pack as 0. The GEMM is the cuBLASLt contract the reference
 * configures (cuda_quant.cuh:362-394): D = bf16(sx * sw * sum_k x8 * w8) with
 * W [N, K] and X [M, K] both K-contiguous. */
#include "oracle.h"
#include <math.h>
#include <stdint.h>
#include <string.h>

/* Returns 1 if any input is not finite (the reference's quantizer fault). */
int oracle_fp8_pack(uint8_t *codes, float *scale_out, const uint16_t *x, size_t count, size_t padded_count) {
    float amax = 0.f;
    int bad = 0;
    for (size_t i = 0; i < count; i++) {
        float v = oracle_bf16_to_f32(x[i]);
        if (!isfinite(v)) { bad = 1; continue; }
        if (fabsf(v) > amax) amax = fabsf(v);
    }
    float scale = amax / 448.f;
    if (scale < 1e-20f) scale = 1e-20f;
    *scale_out = scale;
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < padded_count; i++)
        codes[i] = i < count ? oracle_f32_to_e4m3(oracle_bf16_to_f32(x[i]) / scale) : 0;
    return bad;
}

/* y [m, n] BF16 = bf16((float)(sum) * (sx * sw)); the sum of E4M3 products is
 * accumulated in double, where it is exact for |K| <= 2^20 (each product has
 * at most 8 significant bits between 2^-18 and 2^18). */
void oracle_fp8_gemm(uint16_t *y, const uint8_t *x8, float sx, const uint8_t *w8, float sw, unsigned m, unsigned n,
                     unsigned k) {
    float table[256];
    for (unsigned c = 0; c < 256; c++) table[c] = oracle_e4m3_to_f32((uint8_t)c);
    const float s = sx * sw;
#pragma omp parallel for schedule(static)
    for (unsigned r = 0; r < m; r++)
        for (unsigned c = 0; c < n; c++) {
            double sum = 0;
            const uint8_t *xr = x8 + (size_t)r * k, *wr = w8 + (size_t)c * k;
            for (unsigned i = 0; i < k; i++) sum += (double)table[xr[i]] * (double)table[wr[i]];
            y[(size_t)r * n + c] = oracle_f32_to_bf16((float)sum * s);
        }
}

/* ---- NVFP4 W4A4 (cuda_quant.cuh:21-25, 36-39, 50-72) ----
 * Tensorwide global scale g = max(amax / 2688, 1e-20) (2688 = 6 * 448); per
 * 16-column block a UE4M3 scale sf = E4M3(max(blockmax / (6 g), 2^-9)), RNE,
 * saturating; codes = E2M1 of x * (1 / (sf * g)), RNE, two per byte (low
 * nibble first). Scales sit in cuBLASLt's VEC16 tiled layout
 * ((row / 128) * tiles + block / 4) * 512 + (row % 32) * 16 + ((row % 128) / 32) * 4
 * + block % 4, tiles = ceil(k / 64), rows padded to 128 and blocks to 4 (zero
 * bytes where nothing is written). global slot: {g, g * weight_g (activations)
 * or 1 (weights), 0, 0}. */

/* E2M1 value of a 4-bit code: sign bit 3, exponent bits 2:1 (bias 1), mantissa bit 0. */
float oracle_e2m1_to_f32(uint8_t c) {
    static const float mag[8] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
    return (c & 8) ? -mag[c & 7] : mag[c & 7];
}

/* Nearest E2M1 by exhaustive search, ties to the even code, saturating at 6. */
uint8_t oracle_f32_to_e2m1(float x) {
    const uint8_t sign = signbit(x) ? 8 : 0;
    const double a = fabs((double)x);
    unsigned best = 0;
    double err = INFINITY;
    for (unsigned c = 0; c < 8; c++) {
        double e = fabs(oracle_e2m1_to_f32((uint8_t)c) - a);
        if (e < err || (e == err && (c & 1u) == 0)) { best = c; err = e; }
    }
    return sign | (uint8_t)best;
}

size_t oracle_nvfp4_scale_index(unsigned row, unsigned block, unsigned k) {
    const unsigned tiles = (k / 16 + 3) / 4;
    return ((size_t)(row / 128) * tiles + block / 4) * 512 + (row % 32) * 16 + ((row % 128) / 32) * 4 + block % 4;
}

/* codes: padded * k / 2 bytes; scales: the tiled plane (zeroed by the caller);
 * global_out[4]. weight_global: the weight's g for an activation, or <= 0. */
int oracle_nvfp4_pack(uint8_t *codes, uint8_t *scales, float *global_out, const uint16_t *x, unsigned rows,
                      unsigned padded, unsigned k, float weight_global) {
    float amax = 0.f;
    int bad = 0;
    for (size_t i = 0; i < (size_t)rows * k; i++) {
        float v = oracle_bf16_to_f32(x[i]);
        if (!isfinite(v)) { bad = 1; continue; }
        if (fabsf(v) > amax) amax = fabsf(v);
    }
    float g = amax / 2688.f;
    if (g < 1e-20f) g = 1e-20f;
    global_out[0] = g;
    global_out[1] = weight_global > 0.f ? g * weight_global : 1.f;
    global_out[2] = global_out[3] = 0.f;
    const unsigned blocks = k / 16;
#pragma omp parallel for schedule(static)
    for (size_t b = 0; b < (size_t)padded * blocks; b++) {
        const unsigned row = (unsigned)(b / blocks), col = (unsigned)(b % blocks);
        float v[16], m = 0.f;
        for (unsigned j = 0; j < 16; j++) {
            v[j] = row < rows ? oracle_bf16_to_f32(x[(size_t)row * k + col * 16 + j]) : 0.f;
            if (fabsf(v[j]) > m) m = fabsf(v[j]);
        }
        float t = m / (6.f * g);
        if (t < 0.001953125f) t = 0.001953125f;
        const uint8_t sf = oracle_f32_to_e4m3(t);
        const float r = 1.f / (oracle_e4m3_to_f32(sf) * g);
        scales[oracle_nvfp4_scale_index(row, col, k)] = sf;
        for (unsigned j = 0; j < 8; j++)
            codes[b * 8 + j] = (uint8_t)(oracle_f32_to_e2m1(v[2 * j] * r) | (oracle_f32_to_e2m1(v[2 * j + 1] * r) << 4));
    }
    return bad;
}

/* y [m, n] BF16 = bf16(alpha * sum_k (w4 sfw)(x4 sfx)): the cuBLASLt VEC16
 * UE4M3 contract with alpha = the activation's global[1] (= gx * gw). Each
 * dequantized value is exact in float; the sum is accumulated in double. */
void oracle_nvfp4_gemm(uint16_t *y, const uint8_t *x4, const uint8_t *xs, const uint8_t *w4, const uint8_t *ws,
                       float alpha, unsigned m, unsigned n, unsigned k) {
#pragma omp parallel for schedule(static)
    for (unsigned r = 0; r < m; r++)
        for (unsigned c = 0; c < n; c++) {
            double sum = 0;
            for (unsigned i = 0; i < k; i++) {
                const uint8_t xc = (x4[((size_t)r * k + i) / 2] >> ((i % 2) * 4)) & 15;
                const uint8_t wc = (w4[((size_t)c * k + i) / 2] >> ((i % 2) * 4)) & 15;
                const double xv = oracle_e2m1_to_f32(xc) * oracle_e4m3_to_f32(xs[oracle_nvfp4_scale_index(r, i / 16, k)]);
                const double wv = oracle_e2m1_to_f32(wc) * oracle_e4m3_to_f32(ws[oracle_nvfp4_scale_index(c, i / 16, k)]);
                sum += xv * wv;
            }
            y[(size_t)r * n + c] = oracle_f32_to_bf16((float)sum * alpha);
        }
}
