/* SOL routed attention (reference src/cuda/cuda_sol.cu:92-310), CPU restatement.
 * TEST INFRASTRUCTURE ONLY: used by tests/ as the checker of the HIP SOL path.
 *
 * Layout metadata: h3_sol_block {u32 protect, i32 first_frame, i32 last_frame,
 * u32 rows} per block (src/denoise/sol.h:7), passed as int32 [blocks][4].
 * Q/K/V: BF16 bits [seq][heads][128]. */
#include "oracle.h"
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bf(uint16_t b) { return oracle_bf16_to_f32(b); }

/* Block centroids (cuda_sol.cu:96-104): per head, block and channel, an fp32
 * sum over the block's rows in order, divided by the row count, rounded to
 * BF16. out: [heads][blocks][128]. */
void oracle_sol_summary(uint16_t *out, const uint16_t *x, unsigned seq, unsigned heads, unsigned block) {
    const unsigned blocks = (seq + block - 1) / block;
#pragma omp parallel for collapse(2)
    for (unsigned h = 0; h < heads; h++)
        for (unsigned b = 0; b < blocks; b++) {
            const unsigned start = b * block, len = seq - start < block ? seq - start : block;
            for (unsigned d = 0; d < 128; d++) {
                float sum = 0.f;
                for (unsigned i = 0; i < len; i++) sum += bf(x[((size_t)(start + i) * heads + h) * 128 + d]);
                out[((size_t)h * blocks + b) * 128 + d] = oracle_f32_to_bf16(sum / (float)len);
            }
        }
}

/* Key-centroid moments (cuda_sol.cu:105-109): per head and channel, fp32 sums
 * of x and x*x over the key blocks in order; mean = sum / n, var = max(sq / n -
 * mean * mean, 0), each product and sum rounded separately. out: [heads][256]
 * (128 means, then 128 variances). */
void oracle_sol_moments(float *out, const uint16_t *kc, unsigned heads, unsigned blocks) {
    for (unsigned h = 0; h < heads; h++)
        for (unsigned d = 0; d < 128; d++) {
            float sum = 0.f, sq = 0.f;
            for (unsigned b = 0; b < blocks; b++) {
                float x = bf(kc[((size_t)h * blocks + b) * 128 + d]);
                float xx = x * x;
                sum += x;
                sq += xx;
            }
            float mean = sum / (float)blocks, m2 = mean * mean, var = sq / (float)blocks - m2;
            out[h * 256 + d] = mean;
            out[h * 256 + 128 + d] = var > 0.f ? var : 0.f;
        }
}

/* Routes (cuda_sol.cu:113-139, decision rule restated with this build's fp32
 * order): a = scale * log2 e; per query block, m = sum_d q_d mean_d and
 * v = sum_d q_d^2 var_d as fmaf chains over d; threshold = m a + tau *
 * sqrt(max(v, 0) a a + 1e-6); per key block dot = (fmaf chain of q . kc) * a.
 * Exact when force_exact, either block protected, the frame windows are within
 * `radius`, the floor spreads ceil(min_exact * key_blocks) exact blocks
 * ((b+1) m / n != b m / n), dot or threshold is not finite, the key block is
 * short (< 64 rows), or dot > threshold. routes: u8 [heads][qblocks][kblocks];
 * counts[7] += exact, approximate, protected, local (unprotected), floor,
 * recovery, tail (per pair). */
void oracle_sol_route(uint8_t *routes, uint64_t *counts, const uint16_t *qc, const uint16_t *kc,
                      const float *moments, const int32_t *qmeta, const int32_t *kmeta, unsigned heads,
                      unsigned qblocks, unsigned kblocks, unsigned radius, unsigned minimum, float scale,
                      float tau, int force_exact) {
    const float a = scale * 1.4426950408889634f;
    for (unsigned h = 0; h < heads; h++)
        for (unsigned qb = 0; qb < qblocks; qb++) {
            float q[128], m = 0.f, v = 0.f;
            for (unsigned d = 0; d < 128; d++) {
                q[d] = bf(qc[((size_t)h * qblocks + qb) * 128 + d]);
                m = fmaf(q[d], moments[h * 256 + d], m);
                v = fmaf(q[d] * q[d], moments[h * 256 + 128 + d], v);
            }
            const float mean = m * a, var = (v > 0.f ? v : 0.f) * a * a;
            const float threshold = mean + tau * sqrtf(var + 1e-6f);
            const int32_t *qm = qmeta + 4 * qb;
            for (unsigned b = 0; b < kblocks; b++) {
                float dot = 0.f;
                for (unsigned d = 0; d < 128; d++) dot = fmaf(q[d], bf(kc[((size_t)h * kblocks + b) * 128 + d]), dot);
                dot *= a;
                const int32_t *km = kmeta + 4 * b;
                int protect = qm[0] || km[0];
                int local = qm[1] >= 0 && km[1] >= 0 && qm[1] <= km[2] + (int)radius && km[1] <= qm[2] + (int)radius;
                int floor_ = (uint64_t)(b + 1) * minimum / kblocks != (uint64_t)b * minimum / kblocks;
                int recovery = !isfinite(dot) || !isfinite(threshold), tail = km[3] < 64;
                int exact = force_exact || protect || local || floor_ || recovery || tail || dot > threshold;
                routes[((size_t)h * qblocks + qb) * kblocks + b] = (uint8_t)exact;
                if (counts) {
                    counts[exact ? 0 : 1]++;
                    counts[2] += protect;
                    counts[3] += local && !protect;
                    counts[4] += floor_;
                    counts[5] += recovery;
                    counts[6] += tail;
                }
            }
        }
}

/* SOL attention in float64 for rows [row0, row1) (the reference's independent
 * oracle, tests/cuda_sol_oracle.py:43-56 and tests/metal_sol.c:17-53): the
 * softmax of row r runs over every key of its query block's exact key blocks
 * (score q.k * scale) and one entry per approximate key block (score q.kc *
 * scale + ln 64, value vc). kc, vc: BF16 centroids [heads][kblocks][128].
 * out: FP32 [row1-row0][heads][128]. */
void oracle_sol_attention(float *out, const uint16_t *q, const uint16_t *k, const uint16_t *v, const uint16_t *kc,
                          const uint16_t *vc, const uint8_t *routes, unsigned seq, unsigned heads, unsigned qblock,
                          float scale, unsigned row0, unsigned row1) {
    const unsigned qblocks = (seq + qblock - 1) / qblock, kblocks = (seq + 63) / 64;
#pragma omp parallel for collapse(2)
    for (unsigned r = row0; r < row1; r++)
        for (unsigned h = 0; h < heads; h++) {
            const uint8_t *route = routes + ((size_t)h * qblocks + r / qblock) * kblocks;
            double qr[128], acc[128] = {0}, mx = -INFINITY, sum = 0;
            for (unsigned d = 0; d < 128; d++) qr[d] = bf(q[((size_t)r * heads + h) * 128 + d]);
            for (unsigned b = 0; b < kblocks; b++) {
                const unsigned rows = route[b] ? (seq - b * 64 < 64 ? seq - b * 64 : 64) : 1;
                for (unsigned j = 0; j < rows; j++) {
                    const uint16_t *kr = route[b] ? k + ((size_t)(b * 64 + j) * heads + h) * 128
                                                  : kc + ((size_t)h * kblocks + b) * 128;
                    const uint16_t *vr = route[b] ? v + ((size_t)(b * 64 + j) * heads + h) * 128
                                                  : vc + ((size_t)h * kblocks + b) * 128;
                    double s = 0;
                    for (unsigned d = 0; d < 128; d++) s += qr[d] * bf(kr[d]);
                    s *= scale;
                    if (!route[b]) s += log(64.0);
                    double next = s > mx ? s : mx, alpha = exp(mx - next), w = exp(s - next);
                    sum = sum * alpha + w;
                    for (unsigned d = 0; d < 128; d++) acc[d] = acc[d] * alpha + w * bf(vr[d]);
                    mx = next;
                }
            }
            float *o = out + ((size_t)(r - row0) * heads + h) * 128;
            for (unsigned d = 0; d < 128; d++) o[d] = sum > 0 ? (float)(acc[d] / sum) : 0.f;
        }
}
