/* CPU oracle for the DiT hot path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's algorithms (each function cites the
 * reference file:line it follows). Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, and only as the checker or the
 * timed CPU baseline — never as a product path. Built by oracle/Makefile into
 * oracle/_build/liboracle.so with -ffp-contract=off so every operation rounds
 * where the C source says it does.
 *
 * Pinning of each function (what checks it independently of its own formula)
 * is stated next to it; see tests/test_oracle.py.
 */
#ifndef H3_ORACLE_H
#define H3_ORACLE_H
#include <stddef.h>
#include <stdint.h>

/* ---- numeric helpers ---- */
float oracle_bf16_to_f32(uint16_t b);
uint16_t oracle_f32_to_bf16(float f);            /* round-to-nearest-even */
float oracle_f16_to_f32(uint16_t h);
uint8_t oracle_f32_to_e4m3(float x);             /* OCP e4m3fn, RNE, saturate 448 */
float oracle_e4m3_to_f32(uint8_t c);

/* ---- attention ----
 * Online-softmax SDPA following src/cuda/cuda_attention.cuh:7-51: per (row,
 * head), FP32 dot products (fmaf in channel order), score *= scale, running
 * max/denominator in FP32 with expf, FP32 P.V accumulation by fmaf in key order,
 * keys visited in tiles of `tile` (64 per BASELINE config 1; the reference uses
 * 16). Inputs are FP32 [seq, heads, dim] (callers widen BF16/FP16 exactly);
 * output FP32 [row1-row0, heads, dim] (callers round). Rows [row0, row1) only.
 * OpenMP over (head, row). Pinned by: FP64 brute force on every row
 * (oracle_attention_f64), constant-V and zero-input invariants, head
 * permutation symmetry. */
void oracle_attention(float *out, const float *q, const float *k, const float *v,
                      unsigned seq, unsigned heads, unsigned dim, float scale,
                      unsigned tile, unsigned row0, unsigned row1);
/* Same with a block mask: key block kb (of size `block`) is visible to query
 * block qb iff mask[qb * kblocks + kb]; rows with no visible key give 0. */
void oracle_attention_masked(float *out, const float *q, const float *k, const float *v,
                             unsigned seq, unsigned heads, unsigned dim, float scale,
                             const uint8_t *mask, unsigned block, unsigned row0, unsigned row1);
/* Direct FP64 softmax(scale q.k) v for rows [row0, row1), output [row1-row0, heads, dim]
 * (tests/metal_attention.c:55-67 recipe). */
void oracle_attention_f64(double *out, const float *q, const float *k, const float *v,
                          unsigned seq, unsigned heads, unsigned dim, double scale,
                          unsigned row0, unsigned row1);

/* ---- Sage quantization (structure of src/cuda/cuda_sage2.cu:13-51,
 * src/cuda/cuda_sage_internal.cuh:68-117). Layouts as include/h3_hip_ext.h
 * h3_hip_sage_pack. padded = ceil(seq/64)*64. */
void oracle_sage_pack(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                      unsigned seq, unsigned heads,
                      int8_t *q8, int8_t *k8, uint8_t *v8, float *q_scale, float *k_scale,
                      float *v_scale, uint16_t *k_mean);
/* K mean only, FP64 accumulation (pin for the FP32 ordered mean). */
void oracle_k_mean_f64(const uint16_t *k, unsigned seq, unsigned heads, double *mean);
unsigned oracle_sage_v_position(unsigned j);
/* Attention over the dequantized operands: s = q8.k8 * q_scale * k_scale * scale
 * (exact int32 dot), FP64 softmax, v = v8 * v_scale; rows [row0,row1). With
 * quantize_p, P is rounded as the kernel does (2^(s-m+log2 448) -> e4m3 with the
 * final max); without it P stays FP64. */
void oracle_sage_attention(double *out, const int8_t *q8, const int8_t *k8, const uint8_t *v8,
                           const float *q_scale, const float *k_scale, const float *v_scale,
                           unsigned seq, unsigned heads, float scale,
                           const uint8_t *mask, unsigned block, unsigned row0, unsigned row1);

/* ---- W8A16 (src/weights/q8.c:26-56, src/metal/shaders.metal:788-855) ---- */
int oracle_q8_pack(const uint16_t *w, int8_t *codes, float *scales, unsigned rows,
                   unsigned cols, unsigned group);
/* y = bf16(sum_k x[m,k] * bf16(code[n,k]*scale[n,k/group]) (+bias)), FP64 sum. */
void oracle_linear_q8(uint16_t *y, double *y64, const uint16_t *x, const int8_t *codes,
                      const float *scales, const uint16_t *bias, unsigned rows, unsigned k,
                      unsigned n, unsigned group, int gelu, unsigned row0, unsigned row1);
void oracle_linear_bf16(uint16_t *y, double *y64, const uint16_t *x, const uint16_t *w,
                        const uint16_t *bias, unsigned rows, unsigned k, unsigned n,
                        int gelu, unsigned row0, unsigned row1);

/* ---- elementwise (src/cuda/cuda_kernels.cuh:879-1059, 1242-1254) ---- */
void oracle_adaln(uint16_t *y, const uint16_t *x, const uint16_t *w, const uint16_t *mod,
                  const uint32_t *row_map, unsigned rows, unsigned width, unsigned slots,
                  unsigned shift_slot, unsigned scale_slot, float eps);
void oracle_gate(uint16_t *y, const uint16_t *residual, const uint16_t *branch,
                 const uint16_t *mod, const uint32_t *row_map, unsigned rows, unsigned width,
                 unsigned slots, unsigned gate_slot);
void oracle_qkv_rope(uint16_t *q, uint16_t *k, uint16_t *v, const uint16_t *qkv,
                     const uint16_t *qw, const uint16_t *kw, const uint16_t *cos_t,
                     const uint16_t *sin_t, unsigned seq, unsigned heads, unsigned dim,
                     unsigned half, float eps, int grouped);
float oracle_gelu_tanh(float x);
void oracle_gelu(uint16_t *y, const uint16_t *x, size_t n, int approximate);
void oracle_swiglu(uint16_t *y, const uint16_t *fused, unsigned rows, unsigned width);
void oracle_euler(float *sample, const uint16_t *last, const uint16_t *previous,
                  size_t n, float delta, float ratio);





/* ---- SubBlock router (src/cuda/cuda_subblock.cu:256-324); see block.c ---- */
void oracle_sb_pool(uint16_t *out, const uint16_t *x, unsigned seq, unsigned heads, float scale);
void oracle_sb_score(float *scores, const uint16_t *qp, const uint16_t *kp, unsigned seq, unsigned heads);
void oracle_sb_select(uint8_t *routes, const float *scores, unsigned heads, unsigned blocks, unsigned keep,
                      const uint8_t *q_protect, const uint8_t *k_protect);
void oracle_attention_routed(float *out, const float *q, const float *k, const float *v, unsigned seq,
                             unsigned heads, float scale, const uint8_t *routes, unsigned row0, unsigned row1);

/* ---- SOL routed attention (src/cuda/cuda_sol.cu:92-310); see sol.c ---- */
void oracle_sol_summary(uint16_t *out, const uint16_t *x, unsigned seq, unsigned heads, unsigned block);
void oracle_sol_moments(float *out, const uint16_t *kc, unsigned heads, unsigned blocks);
void oracle_sol_route(uint8_t *routes, uint64_t *counts, const uint16_t *qc, const uint16_t *kc,
                      const float *moments, const int32_t *qmeta, const int32_t *kmeta, unsigned heads,
                      unsigned qblocks, unsigned kblocks, unsigned radius, unsigned minimum, float scale,
                      float tau, int force_exact);
void oracle_sol_attention(float *out, const uint16_t *q, const uint16_t *k, const uint16_t *v, const uint16_t *kc,
                          const uint16_t *vc, const uint8_t *routes, unsigned seq, unsigned heads, unsigned qblock,
                          float scale, unsigned row0, unsigned row1);

/* ---- reference test-input generators (tests/cuda_attention.c:14-18,
 * tests/attention_native.c:20) ---- */
void oracle_xorshift_bf16(uint16_t *out, size_t count, uint32_t *seed);
void oracle_xorshift_native_bf16(uint16_t *out, size_t count, uint32_t *state);

int oracle_threads(void);

/* quant.c: FP8 W8A8 projection (cuda_quant.cuh:26-104, 339-398) */
int oracle_fp8_pack(uint8_t *codes, float *scale_out, const uint16_t *x, size_t count, size_t padded_count);
void oracle_fp8_gemm(uint16_t *y, const uint8_t *x8, float sx, const uint8_t *w8, float sw, unsigned m, unsigned n,
                     unsigned k);
float oracle_e2m1_to_f32(uint8_t c);
uint8_t oracle_f32_to_e2m1(float x);
size_t oracle_nvfp4_scale_index(unsigned row, unsigned block, unsigned k);
int oracle_nvfp4_pack(uint8_t *codes, uint8_t *scales, float *global_out, const uint16_t *x, unsigned rows,
                      unsigned padded, unsigned k, float weight_global);
void oracle_nvfp4_gemm(uint16_t *y, const uint8_t *x4, const uint8_t *xs, const uint8_t *w4, const uint8_t *ws,
                       float alpha, unsigned m, unsigned n, unsigned k);
#endif
