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
