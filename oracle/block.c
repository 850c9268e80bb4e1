/* CPU oracle — TEST INFRASTRUCTURE ONLY (see oracle.h). DiT block operators:
 * q8 packing, W8A16 / BF16 projections (FP64 accumulation), AdaLN, gates,
 * Q/K norm + RoPE, activations and the Euler update. */
#include "oracle.h"
#include <float.h>
#include <math.h>
#include <stdlib.h>

/* src/weights/q8.c:26-56 with a group parameter (64 = the reference recipe;
 * group = cols = one scale per output channel): scale = max|w|/127 (1 for an
 * all-zero group, floored at FLT_MIN), code = nearest integer to w/scale with
 * ties to even (nearbyintf in the default rounding mode), clamped to +-127. */
int oracle_q8_pack(const uint16_t *w, int8_t *codes, float *scales, unsigned rows, unsigned cols,
                   unsigned group) {
    if (!rows || !cols || !group) return 0;
    unsigned groups = (cols + group - 1) / group;
    for (unsigned r = 0; r < rows; r++)
        for (unsigned gi = 0; gi < groups; gi++) {
            unsigned b = gi * group, e = b + group < cols ? b + group : cols;
            float amax = 0.f;
            for (unsigned c = b; c < e; c++) {
                float x = oracle_bf16_to_f32(w[(size_t)r * cols + c]);
                if (isnan(x) || isinf(x)) return 0;
                amax = fmaxf(amax, fabsf(x));
            }
            float s = amax == 0.f ? 1.f : fmaxf(amax / 127.f, FLT_MIN);
            scales[(size_t)r * groups + gi] = s;
            for (unsigned c = b; c < e; c++) {
                float q = nearbyintf(oracle_bf16_to_f32(w[(size_t)r * cols + c]) / s);
                codes[(size_t)r * cols + c] = (int8_t)(q > 127.f ? 127 : q < -127.f ? -127 : (int)q);
            }
        }
    return 1;
}

static float gelu_tanh_f(float v) {
    /* src/cuda/cuda_kernels.cuh:886-895 */
    float inner = 0.7978845608028654f * (v + 0.044715f * v * v * v);
    return inner <= -10.0f ? 0.0f : inner >= 10.0f ? v : 0.5f * v * (1.0f + tanhf(inner));
}
float oracle_gelu_tanh(float x) { return gelu_tanh_f(x); }

static void linear_rows(uint16_t *y, double *y64, const uint16_t *x, const float *wrow_f, const uint16_t *bias,
                        unsigned k, unsigned n, unsigned col, int gelu, unsigned row0, unsigned row1) {
    for (unsigned r = row0; r < row1; r++) {
        double s = bias ? (double)oracle_bf16_to_f32(bias[col]) : 0.0;
        const uint16_t *xr = x + (size_t)r * k;
        for (unsigned c = 0; c < k; c++) s += (double)oracle_bf16_to_f32(xr[c]) * wrow_f[c];
        size_t at = (size_t)(r - row0) * n + col;
        uint16_t b = oracle_f32_to_bf16((float)s);
        if (gelu) b = oracle_f32_to_bf16(gelu_tanh_f(oracle_bf16_to_f32(b)));
        if (y) y[at] = b;
        if (y64) y64[at] = gelu ? (double)gelu_tanh_f((float)s) : s;
    }
}

/* W8A16 (src/metal/shaders.metal:799-855, tests/metal_q8.c:125-132): every
 * weight is reconstructed as bf16(code * scale); sums in FP64. Output rows
 * [row0, row1) into y/y64 [row1-row0, n]. */
void oracle_linear_q8(uint16_t *y, double *y64, const uint16_t *x, const int8_t *codes, const float *scales,
                      const uint16_t *bias, unsigned rows, unsigned k, unsigned n, unsigned group, int gelu,
                      unsigned row0, unsigned row1) {
    unsigned groups = (k + group - 1) / group;
#pragma omp parallel
    {
        float *wf = malloc(sizeof(float) * k);
#pragma omp for schedule(dynamic, 8)
        for (unsigned col = 0; col < n; col++) {
            for (unsigned c = 0; c < k; c++)
                wf[c] = oracle_bf16_to_f32(oracle_f32_to_bf16((float)codes[(size_t)col * k + c] *
                                                              scales[(size_t)col * groups + c / group]));
            linear_rows(y, y64, x, wf, bias, k, n, col, gelu, row0, row1);
        }
        free(wf);
    }
}

void oracle_linear_bf16(uint16_t *y, double *y64, const uint16_t *x, const uint16_t *w, const uint16_t *bias,
                        unsigned rows, unsigned k, unsigned n, int gelu, unsigned row0, unsigned row1) {
#pragma omp parallel
    {
        float *wf = malloc(sizeof(float) * k);
#pragma omp for schedule(dynamic, 8)
        for (unsigned col = 0; col < n; col++) {
            for (unsigned c = 0; c < k; c++) wf[c] = oracle_bf16_to_f32(w[(size_t)col * k + c]);
            linear_rows(y, y64, x, wf, bias, k, n, col, gelu, row0, row1);
        }
        free(wf);
    }
}

/* src/cuda/cuda_kernels.cuh:936-971: per row, sum of squares by fmaf in column
 * order, inv = 1/sqrt(mean + eps), y = bf16(fmaf(x*inv*w, 1+scale, shift)). */
void oracle_adaln(uint16_t *y, const uint16_t *x, const uint16_t *w, const uint16_t *mod, const uint32_t *row_map,
                  unsigned rows, unsigned width, unsigned slots, unsigned shift_slot, unsigned scale_slot, float eps) {
#pragma omp parallel for
    for (unsigned r = 0; r < rows; r++) {
        const uint16_t *xr = x + (size_t)r * width;
        float sum = 0.f;
        for (unsigned c = 0; c < width; c++) {
            float v = oracle_bf16_to_f32(xr[c]);
            sum = fmaf(v, v, sum);
        }
        float inv = 1.0f / sqrtf(sum / (float)width + eps);
        size_t base = (size_t)row_map[r] * slots * width;
        for (unsigned c = 0; c < width; c++) {
            float normalized = oracle_bf16_to_f32(xr[c]) * inv * oracle_bf16_to_f32(w[c]);
            float shift = oracle_bf16_to_f32(mod[base + (size_t)shift_slot * width + c]);
            float scale = oracle_bf16_to_f32(mod[base + (size_t)scale_slot * width + c]);
            y[(size_t)r * width + c] = oracle_f32_to_bf16(fmaf(normalized, 1.0f + scale, shift));
        }
    }
}

/* src/cuda/cuda_kernels.cuh:973-986 (residual + branch*gate, one rounding). */
void oracle_gate(uint16_t *y, const uint16_t *residual, const uint16_t *branch, const uint16_t *mod,
                 const uint32_t *row_map, unsigned rows, unsigned width, unsigned slots, unsigned gate_slot) {
    for (unsigned r = 0; r < rows; r++)
        for (unsigned c = 0; c < width; c++) {
            size_t i = (size_t)r * width + c;
            float gate = oracle_bf16_to_f32(mod[(size_t)row_map[r] * slots * width + (size_t)gate_slot * width + c]);
            y[i] = oracle_f32_to_bf16(fmaf(oracle_bf16_to_f32(branch[i]), gate, oracle_bf16_to_f32(residual[i])));
        }
}

/* src/cuda/cuda_kernels.cuh:988-1045 (grouped rows when grouped != 0). With
 * qw == NULL the Q/K RMSNorm is skipped (RoPE only). */
void oracle_qkv_rope(uint16_t *q, uint16_t *k, uint16_t *v, const uint16_t *qkv, const uint16_t *qw,
                     const uint16_t *kw, const uint16_t *cos_t, const uint16_t *sin_t, unsigned seq,
                     unsigned heads, unsigned dim, unsigned half, float eps, int grouped) {
    for (unsigned row = 0; row < seq; row++)
        for (unsigned h = 0; h < heads; h++) {
            size_t inner = (size_t)heads * dim, rb = (size_t)row * inner * 3;
            size_t qb = rb + (size_t)h * dim, kb = qb + inner, vb = qb + 2 * inner;
            if (grouped) { qb = rb + (size_t)h * dim * 3; kb = qb + dim; vb = kb + dim; }
            float qs = 0.f, ks = 0.f;
            for (unsigned d = 0; d < dim; d++) {
                float a = oracle_bf16_to_f32(qkv[qb + d]), b = oracle_bf16_to_f32(qkv[kb + d]);
                qs = fmaf(a, a, qs);
                ks = fmaf(b, b, ks);
            }
            float qi = qw ? 1.0f / sqrtf(qs / (float)dim + eps) : 1.f;
            float ki = qw ? 1.0f / sqrtf(ks / (float)dim + eps) : 1.f;
#define NQ(d) (qw ? oracle_bf16_to_f32(qkv[qb + (d)]) * qi * oracle_bf16_to_f32(qw[d]) : oracle_bf16_to_f32(qkv[qb + (d)]))
#define NK(d) (qw ? oracle_bf16_to_f32(qkv[kb + (d)]) * ki * oracle_bf16_to_f32(kw[d]) : oracle_bf16_to_f32(qkv[kb + (d)]))
            size_t ob = ((size_t)row * heads + h) * dim;
            for (unsigned d = 0; d < dim; d++) {
                float q0 = NQ(d), k0 = NK(d);
                if (d < half) {
                    float c = oracle_bf16_to_f32(cos_t[(size_t)row * half + d]);
                    float s = oracle_bf16_to_f32(sin_t[(size_t)row * half + d]);
                    q0 = q0 * c - NQ(d + half) * s;
                    k0 = k0 * c - NK(d + half) * s;
                } else if (d < 2 * half) {
                    unsigned p = d - half;
                    float c = oracle_bf16_to_f32(cos_t[(size_t)row * half + p]);
                    float s = oracle_bf16_to_f32(sin_t[(size_t)row * half + p]);
                    q0 = q0 * c + NQ(p) * s;
                    k0 = k0 * c + NK(p) * s;
                }
                q[ob + d] = oracle_f32_to_bf16(q0);
                k[ob + d] = oracle_f32_to_bf16(k0);
                v[ob + d] = qkv[vb + d];
            }
#undef NQ
#undef NK
        }
}

void oracle_gelu(uint16_t *y, const uint16_t *x, size_t n, int approximate) {
    for (size_t i = 0; i < n; i++) {
        float v = oracle_bf16_to_f32(x[i]), r;
        if (approximate) r = gelu_tanh_f(v);
        else r = v <= -10.0f ? 0.0f : v >= 10.0f ? v : 0.5f * v * (1.0f + erff(v * 0.7071067811865475f));
        y[i] = oracle_f32_to_bf16(r);
    }
}

/* src/cuda/cuda_kernels.cuh:1047-1059 */
void oracle_swiglu(uint16_t *y, const uint16_t *fused, unsigned rows, unsigned width) {
    for (unsigned r = 0; r < rows; r++)
        for (unsigned c = 0; c < width; c++) {
            float gate = oracle_bf16_to_f32(fused[(size_t)r * width * 2 + c]);
            float up = oracle_bf16_to_f32(fused[(size_t)r * width * 2 + width + c]);
            y[(size_t)r * width + c] = oracle_f32_to_bf16(gate / (1.0f + expf(-gate)) * up);
        }
}

/* src/cuda/cuda_kernels.cuh:1242-1254 */
void oracle_euler(float *sample, const uint16_t *last, const uint16_t *previous, size_t n, float delta, float ratio) {
    for (size_t i = 0; i < n; i++) {
        float l = oracle_bf16_to_f32(last[i]);
        float velocity = fmaf(ratio, l - oracle_bf16_to_f32(previous[i]), l);
        sample[i] = fmaf(delta, velocity, sample[i]);
    }
}

/* src/cuda/cuda_kernels.cuh:805-833: y = bf16(x * 1/sqrt(mean x^2 + eps) * w);
 * the sum of squares by fmaf in column order. */
void oracle_rms_norm(uint16_t *y, const uint16_t *x, const uint16_t *w, unsigned rows, unsigned width, float eps) {
#pragma omp parallel for
    for (unsigned r = 0; r < rows; r++) {
        const uint16_t *xr = x + (size_t)r * width;
        float sum = 0.f;
        for (unsigned c = 0; c < width; c++) {
            float v = oracle_bf16_to_f32(xr[c]);
            sum = fmaf(v, v, sum);
        }
        float inv = 1.0f / sqrtf(sum / (float)width + eps);
        for (unsigned c = 0; c < width; c++)
            y[(size_t)r * width + c] = oracle_f32_to_bf16(oracle_bf16_to_f32(xr[c]) * inv * oracle_bf16_to_f32(w[c]));
    }
}

/* src/cuda/cuda_kernels.cuh:1117-1133: the same RMSNorm per (row, head) of
 * [seq, heads, dim], in place. */
void oracle_head_rms_norm(uint16_t *t, const uint16_t *w, unsigned seq, unsigned heads, unsigned dim, float eps) {
    oracle_rms_norm(t, t, w, seq * heads, dim, eps);
}

/* src/cuda/cuda_kernels.cuh:237-265 (and the row-mapped variant :267-300):
 * y[map(r), n] = bf16(bias[n] + sum_k x[r,k] * W[n,k]) with FP32 fmaf in
 * ascending k from the bias; rows whose map entry is >= out_rows are skipped. */
void oracle_patch_linear(uint16_t *y, const float *x, const float *w, const float *bias, const uint32_t *map,
                         unsigned out_rows, unsigned m, unsigned k, unsigned n) {
#pragma omp parallel for
    for (unsigned r = 0; r < m; r++) {
        unsigned o = map ? map[r] : r;
        if (o >= out_rows) continue;
        for (unsigned c = 0; c < n; c++) {
            float acc = bias ? bias[c] : 0.f;
            for (unsigned i = 0; i < k; i++) acc = fmaf(x[(size_t)r * k + i], w[(size_t)c * k + i], acc);
            y[(size_t)o * n + c] = oracle_f32_to_bf16(acc);
        }
    }
}

/* ---- SubBlock router (reference src/cuda/cuda_subblock.cu:256-324) ---- */

/* Pooled 16-row cells: for cell c (rows 16c..16c+15, missing rows 0), the fp32
 * pairwise tree v[i] += v[i+s] for s = 8, 4, 2, 1 (cuda_subblock.cu:262-263),
 * mean = v[0] / count * scale, rounded to BF16. out: [heads][cells][128],
 * cells = ceil(seq/64) * 4 (cells past the sequence are 0). */
void oracle_sb_pool(uint16_t *out, const uint16_t *x, unsigned seq, unsigned heads, float scale) {
    const unsigned cells = (seq + 63) / 64 * 4;
#pragma omp parallel for
    for (unsigned h = 0; h < heads; h++)
        for (unsigned cell = 0; cell < cells; cell++)
            for (unsigned d = 0; d < 128; d++) {
                unsigned start = cell * 16, count = start < seq ? (seq - start < 16 ? seq - start : 16) : 0;
                float v[16];
                for (unsigned i = 0; i < 16; i++)
                    v[i] = i < count ? oracle_bf16_to_f32(x[((size_t)(start + i) * heads + h) * 128 + d]) : 0.f;
                for (unsigned s = 8; s; s >>= 1)
                    for (unsigned i = 0; i < s; i++) v[i] += v[i + s];
                float mean = count ? v[0] / (float)count * scale : 0.f;
                out[((size_t)h * cells + cell) * 128 + d] = oracle_f32_to_bf16(mean);
            }
}

/* Block scores (cuda_subblock.cu:272-297): for query block i and key block j,
 * dots of the (up to 4 x 4) valid pooled cells, each an fp32 fmaf chain over d;
 * per query cell a: lse_a = max_b + log2(sum_b exp2(dot - max_b)); score =
 * (max_a + log2(sum_a exp2(lse_a - max_a))) * ln 2. scores: [heads][B][B]. */
void oracle_sb_score(float *scores, const uint16_t *qp, const uint16_t *kp, unsigned seq, unsigned heads) {
    const unsigned blocks = (seq + 63) / 64, cells = blocks * 4;
#pragma omp parallel for collapse(2)
    for (unsigned h = 0; h < heads; h++)
        for (unsigned qb = 0; qb < blocks; qb++)
            for (unsigned kb = 0; kb < blocks; kb++) {
                unsigned nq = (seq - qb * 64 + 15) / 16, nk = (seq - kb * 64 + 15) / 16;
                if (nq > 4) nq = 4;
                if (nk > 4) nk = 4;
                float qlse[4] = {0};
                for (unsigned a = 0; a < nq; a++) {
                    float dots[4] = {0};
                    for (unsigned b = 0; b < nk; b++) {
                        const uint16_t *qr = qp + ((size_t)h * cells + qb * 4 + a) * 128;
                        const uint16_t *kr = kp + ((size_t)h * cells + kb * 4 + b) * 128;
                        float sum = 0.f;
                        for (unsigned d = 0; d < 128; d++) sum = fmaf(oracle_bf16_to_f32(qr[d]), oracle_bf16_to_f32(kr[d]), sum);
                        dots[b] = sum;
                    }
                    float largest = dots[0], sum = 0.f;
                    for (unsigned b = 1; b < nk; b++) largest = fmaxf(largest, dots[b]);
                    for (unsigned b = 0; b < nk; b++) sum += exp2f(dots[b] - largest);
                    qlse[a] = largest + log2f(sum);
                }
                float largest = qlse[0], sum = 0.f;
                for (unsigned a = 1; a < nq; a++) largest = fmaxf(largest, qlse[a]);
                for (unsigned a = 0; a < nq; a++) sum += exp2f(qlse[a] - largest);
                scores[((size_t)h * blocks + qb) * blocks + kb] = (largest + log2f(sum)) * 0.6931471805599453f;
            }
}

/* Routes (cuda_subblock.cu:300-324): key block k of query row i is kept when
 * its rank (scores greater, or equal with a lower index) is below `keep`, when
 * k is protected, or when the query block is protected. routes: [heads][B][B]. */
void oracle_sb_select(uint8_t *routes, const float *scores, unsigned heads, unsigned blocks, unsigned keep,
                      const uint8_t *q_protect, const uint8_t *k_protect) {
#pragma omp parallel for collapse(2)
    for (unsigned h = 0; h < heads; h++)
        for (unsigned qb = 0; qb < blocks; qb++) {
            const float *row = scores + ((size_t)h * blocks + qb) * blocks;
            for (unsigned k = 0; k < blocks; k++) {
                unsigned rank = 0;
                for (unsigned j = 0; j < blocks; j++) rank += row[j] > row[k] || (row[j] == row[k] && j < k);
                routes[((size_t)h * blocks + qb) * blocks + k] =
                    (uint8_t)(rank < keep || (k_protect && k_protect[k]) || (q_protect && q_protect[qb]));
            }
        }
}

/* Attention with a per-head 64 x 64 route mask (routes [heads][B][B]), rows
 * [row0, row1): the masked online softmax of oracle_attention_masked with the
 * head's own mask. out: FP32 [row1-row0, heads, 128]. */
void oracle_attention_routed(float *out, const float *q, const float *k, const float *v, unsigned seq,
                             unsigned heads, float scale, const uint8_t *routes, unsigned row0, unsigned row1) {
    const unsigned blocks = (seq + 63) / 64;
#pragma omp parallel for collapse(2)
    for (unsigned h = 0; h < heads; h++)
        for (unsigned r = row0; r < row1; r++) {
            const uint8_t *mrow = routes + ((size_t)h * blocks + r / 64) * blocks;
            const float *qr = q + ((size_t)r * heads + h) * 128;
            double m = -1e300, l = 0, acc[128] = {0};
            for (unsigned j = 0; j < seq; j++) {
                if (!mrow[j / 64]) continue;
                const float *kr = k + ((size_t)j * heads + h) * 128;
                double s = 0;
                for (unsigned d = 0; d < 128; d++) s += (double)qr[d] * kr[d];
                s *= scale;
                if (s > m) {
                    double a = exp(m - s);
                    for (unsigned d = 0; d < 128; d++) acc[d] *= a;
                    l *= a;
                    m = s;
                }
                double p = exp(s - m);
                l += p;
                const float *vr = v + ((size_t)j * heads + h) * 128;
                for (unsigned d = 0; d < 128; d++) acc[d] += p * vr[d];
            }
            float *o = out + ((size_t)(r - row0) * heads + h) * 128;
            for (unsigned d = 0; d < 128; d++) o[d] = l > 0 ? (float)(acc[d] / l) : 0.f;
        }
}
