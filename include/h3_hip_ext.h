/* h3_hip_ext.h — entry points of the gfx950 backend with no counterpart in the
 * reference operator surface. They exist for callers that need to drive parts
 * of the DiT hot path the reference drives internally (a fixed block-sparse
 * mask instead of its learned router, pre-packed W8A16 weights instead of a
 * checkpoint file), and for measurement and parity tests. */
#ifndef H3_HIP_EXT_H
#define H3_HIP_EXT_H

#include <stddef.h>
#include <stdint.h>
#include "h3_gpu.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Library build identity ("h3hip gfx950 <version>"). */
const char *h3_hip_version(void);

/* W8A16 weight from already-packed codes: int8 [rows, columns] row-major and
 * fp32 scales [rows, ceil(columns/group)]. group = columns gives one scale per
 * output channel; group = 64 is the reference q8 recipe (src/weights/q8.h:6-12).
 * The tensor dequantizes as w = bf16(code * scale) (src/metal/shaders.metal:825-827). */
h3_gpu_tensor *h3_hip_q8_from_packed(h3_gpu *gpu, const int8_t *codes, const float *scales,
                                     uint32_t rows, uint32_t columns, uint32_t group);

/* h3_gpu_linear_bf16 followed by the tanh GELU of h3_gpu_gelu_bf16(approximate=1),
 * fused into the GEMM epilogue: y = bf16(gelu(bf16(x . W^T + bias))). The MLP
 * up-projection of the synthetic DiT block. */
int h3_hip_linear_gelu_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input,
                            const h3_gpu_tensor *weight, const h3_gpu_tensor *bias,
                            uint32_t rows, uint32_t input_dim, uint32_t output_dim);

/* An empty W8A16 weight (codes [rows, columns] and fp32 scales [rows,
 * ceil(columns/group)] allocated on the device, contents undefined). */
h3_gpu_tensor *h3_hip_q8_new(h3_gpu *gpu, uint32_t rows, uint32_t columns, uint32_t group);
/* Seeded random W8A16 contents (requires an active command): code i =
 * (splitmix64((seed << 40) + i) mod 255) - 127, scale j = lo + (hi - lo) *
 * ((splitmix64((seed << 40) + 2^39 + j) >> 11) * 2^-53). */
int h3_hip_fill_q8_random(h3_gpu *gpu, h3_gpu_tensor *weight, uint64_t seed, float lo, float hi);
/* Synchronous device -> host copy of a tensor; for a q8 weight, dst receives the
 * codes followed by the scales (the h3_hip_tensor_stream_host layout). */
int h3_hip_tensor_copy_to_host(h3_gpu_tensor *tensor, void *dst, size_t bytes);

/* Dense BF16 SDPA that allocates nothing: the computation, arguments, errors
 * and output of h3_gpu_sdpa_bf16 (head_major 0) or
 * h3_gpu_sdpa_bf16_head_major_output (head_major 1), bit for bit, with the
 * workspace (transposed V and retry bytes) in a fixed 384 MiB device array
 * instead of a device allocation. No counterpart in the reference: it is for
 * callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Workspaces above 384 MiB are
 * refused with an error (S * H up to about 1.5M rows, e.g. S = 32400 with
 * H = 40). All calls on one GPU share its array: calls that overlap on one
 * GPU race. Requires an active command (h3_gpu_begin). */
int h3_hip_sdpa_bf16_noalloc(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *query,
                             const h3_gpu_tensor *key, const h3_gpu_tensor *value, uint32_t sequence,
                             uint32_t heads, uint32_t head_dim, float scale, int head_major);

/* Interop with stream-level entry points (include/h3_sglang_flash.h): a
 * tensor's device address (NULL for host-visible storage) and the context's
 * compute stream (a hipStream_t), so such calls order with the context's
 * own work. */
void *h3_hip_tensor_device_pointer(h3_gpu_tensor *tensor);
void *h3_hip_compute_stream(h3_gpu *gpu);

/* Fixed block-sparse mask for main-DiT attention. mask is u8 [q_blocks, k_blocks]
 * (nonzero = keep) over block x block tiles; block must be 128 (or 64). While a
 * mask is bound, h3_gpu_dit_sdpa_bf16 computes softmax over the kept key tiles
 * only, in the configured precision (dense BF16 or sage2++). NULL unbinds. The
 * mask is copied; rows with no kept tile produce zeros. */
int h3_hip_dit_block_mask(h3_gpu *gpu, const uint8_t *mask, uint32_t q_blocks,
                          uint32_t k_blocks, uint32_t block);

/* Synthetic block mask of the benchmark's joint sequence (video rows first, then
 * audio): mask[qb * B + kb], B = ceil(seq/block), is 1 on the diagonal, for every
 * pair of blocks that both hold audio rows (rows >= video_rows), and otherwise
 * when splitmix64((seed << 40) + qb*B + kb) >> 11, times 2^-53, is < density.
 * Returns the number of kept blocks (0 on invalid arguments). Host only. */
unsigned h3_hip_synthetic_block_mask(uint8_t *mask, unsigned seq, unsigned video_rows,
                                     unsigned block, double density, uint64_t seed);

/* SubBlock (mode 4) bypass policy: the request's sparsity and warmup as passed
 * to h3_subblock_dense_reason (reference src/denoise/subblock.c:44-51); a call
 * for which a reason applies runs dense. Defaults: sparsity 0.75, warmup 0
 * (= 10 steps); warmup < 0 disables the warmup rule. */
int h3_hip_dit_subblock_policy(h3_gpu *gpu, float sparsity, int warmup);

/* SubBlock router capture, the counterpart of the reference's
 * h3_cuda_subblock_routes (src/cuda/cuda_subblock.cu): after a routed mode-4
 * call (a layout bound with h3_gpu_dit_sol_layout, no host mask), copies that
 * call's routes u8 [heads][B][B] and block scores f32 [heads][B][B]
 * (B = ceil(seq / 64), route_count = heads * B * B) and its pooled BF16 cells
 * [heads][4B][128] of Q (scaled by scale * log2 e) and K (pool_count =
 * heads * 4B * 128). Any output may be NULL. Waits for the compute stream. */
int h3_hip_subblock_routes(h3_gpu *gpu, uint8_t *routes, float *scores, size_t route_count,
                           uint16_t *q_pool, uint16_t *k_pool, size_t pool_count);

/* SubBlock routed calls keep their device workspace (router buffers plus the
 * transposed V of one head group) under a fixed budget, the reference's
 * attention workspace cap of 512 MiB (src/denoise/attention.h:12, plan order of
 * h3_subblock_plan_make, src/denoise/subblock.c:18-42): heads run in groups
 * (all, then halved) and 64-query blocks in slabs (all, then multiples of 32)
 * until the chunk fits. h3_hip_subblock_workspace_cap sets this context's
 * budget (0 restores 512 MiB), e.g. to force chunking in tests; a shape that
 * fits no chunk fails. h3_hip_subblock_plan_info reports the last routed
 * call's head group, query slab and workspace bytes. A chunked call keeps no
 * routes for h3_hip_subblock_routes. */
int h3_hip_subblock_workspace_cap(h3_gpu *gpu, size_t bytes);
int h3_hip_subblock_plan_info(h3_gpu *gpu, uint32_t *group, uint32_t *slab, size_t *bytes);

/* SOL (mode 3) routed calls under the same fixed 512 MiB budget (the
 * reference's h3_cuda_sol_plan_make, src/cuda/cuda_sol_policy.c): the centroids
 * of all heads, then routes, lists and the transposed V one head group at a
 * time (all heads, halved until the group fits). h3_hip_sol_workspace_cap sets
 * this context's budget (0 restores 512 MiB); h3_hip_sol_plan_info reports the
 * last routed call's head group and workspace bytes. A call that ran in head
 * groups keeps no routes for h3_hip_sol_routes. */
int h3_hip_sol_workspace_cap(h3_gpu *gpu, size_t bytes);
int h3_hip_sol_plan_info(h3_gpu *gpu, uint32_t *group, size_t *bytes);

/* SOL (mode 3) route capture, the counterpart of the reference's
 * h3_cuda_sol_routes (src/cuda/cuda_sol.cu:418-423): after a routed SOL call,
 * copies its routes u8 [heads][QB][KB] (QB = ceil(seq / q_block), KB =
 * ceil(seq / 64); route_count = heads * QB * KB) and its BF16 centroids: qc
 * [heads][QB][128] (qc_count = heads * QB * 128), kc and vc [heads][KB][128]
 * (kv_count = heads * KB * 128). Any output may be NULL. Waits for the stream. */
int h3_hip_sol_routes(h3_gpu *gpu, uint8_t *routes, size_t route_count, uint16_t *qc, size_t qc_count,
                      uint16_t *kc, uint16_t *vc, size_t kv_count);
/* SOL operator tests: route every key block exact (the reference's run-time
 * force_exact, h3_cuda_sol_run). */
int h3_hip_dit_sol_force_exact(h3_gpu *gpu, int on);
/* SOL counters, the values of the reference's "SOL counters" report at
 * synchronize (src/cuda/gpu_cuda.cu:452-460, h3_cuda_sol_stats in
 * src/cuda/cuda_sol.h:6-10): out[0] routed calls, out[1] calls the dense
 * bypass rules took, out[2..8] (query block, key block) pairs exact,
 * approximate, protected, local, floor, recovery, tail, summed over heads and
 * calls. count must be 9. Waits for the stream if calls are not yet counted. */
int h3_hip_sol_counters(h3_gpu *gpu, uint64_t *out, size_t count);

/* FP8 projections (quant.hip). SHA-256 (FIPS 180-4) of a buffer with the
 * library's own digest, the one its packed-weight caches key and verify with. */
int h3_hip_sha256(const void *data, size_t bytes, uint8_t digest[32]);
/* Tensorwide E4M3 packing of count BF16 device values (count a positive
 * multiple of 8), as a projection input is packed per call
 * (reference src/cuda/cuda_quant.cuh:26-49): codes (>= count bytes) and the
 * 16-byte global slot {scale, 1, 0, 0}. Waits for the stream. */
int h3_hip_fp8_pack(h3_gpu *gpu, const h3_gpu_tensor *x, h3_gpu_tensor *codes, h3_gpu_tensor *global,
                    size_t count);
/* A resident packed weight of the configured quantization mode (FP8 or NVFP4;
 * the h3_gpu_quant_load descriptor) from n x k BF16 device values, without a
 * file or artifact, for synthetic models and benchmarks. Requires
 * h3_gpu_quant_configure(mode 1 or 2); n, k multiples of 128. */
h3_gpu_tensor *h3_hip_quant_weight_from_bf16(h3_gpu *gpu, const h3_gpu_tensor *w, uint32_t n, uint32_t k);

/* Sage quantization of sequence-major BF16 Q, K, V [seq, heads, 128] into the
 * layouts the quantized attention kernel consumes (all head-major, rows padded
 * to a multiple of 64, padded rows zero):
 *   q8, k8   int8 [heads, padded, 128]; K is smoothed first: k' = bf16(k - mean)
 *   q_scale, k_scale fp32 [heads, padded/64]: fmaf(max|x| over the 64x128 block, 1/127, 1e-7)
 *   v8       fp8 e4m3 (OCP) [heads, 128, padded], key order permuted within each
 *            64-key tile as the kernel reads it (h3_hip_sage_v_position)
 *   v_scale  fp32 [heads, 128]: max|v| over the sequence / 448
 *   k_mean   bf16 [heads, 128]: bf16(sum / seq), sum in fp32 over rows in a fixed order:
 *            partial p sums rows [256p, 256p+256) in row order, partials summed in p order.
 * Requires an active command. Used by parity tests; the attention path calls the
 * same kernels on its own workspace. */
int h3_hip_sage_pack(h3_gpu *gpu, const h3_gpu_tensor *q, const h3_gpu_tensor *k,
                     const h3_gpu_tensor *v, uint32_t seq, uint32_t heads,
                     h3_gpu_tensor *q8, h3_gpu_tensor *k8, h3_gpu_tensor *v8,
                     h3_gpu_tensor *q_scale, h3_gpu_tensor *k_scale,
                     h3_gpu_tensor *v_scale, h3_gpu_tensor *k_mean);
/* Position of key j (0..63) of a 64-key tile inside the packed fp8 V row. */
unsigned h3_hip_sage_v_position(unsigned j);

/* Pinned host memory for streamed weights, and an asynchronous fill of a device
 * tensor from it on the copy stream (the streamed-weight path of reference
 * src/cuda/gpu_cuda.cu:761-840, with the source already in pinned memory).
 * For a q8 weight, src holds the int8 codes followed by the fp32 scales. Kernels
 * that read the tensor wait for the fill; the next fill waits for those kernels. */
void *h3_hip_host_alloc(h3_gpu *gpu, size_t bytes);
void h3_hip_host_free(h3_gpu *gpu, void *pointer, size_t bytes);
int h3_hip_tensor_stream_host(h3_gpu_tensor *tensor, const void *src, size_t bytes);

/* Raw device contents of a tensor (any dtype), for reading int8/fp8 codes. */
int h3_hip_tensor_read_bytes(const h3_gpu_tensor *tensor, void *dst, size_t bytes);
/* Fill count BF16 elements with seeded N(0,1) * scale values: the splitmix64 +
 * Box-Muller stream documented in h3cli_amd/synth.py. Requires an active command. */
int h3_hip_fill_normal_bf16(h3_gpu *gpu, h3_gpu_tensor *tensor, uint64_t seed, float scale, size_t count);

/* Kernel timing on the compute stream: record a timing event (created with
 * timing enabled) and read the elapsed milliseconds between two of them after
 * h3_gpu_submit/synchronize. */
h3_gpu_event *h3_hip_timing_event_new(h3_gpu *gpu);
int h3_hip_event_elapsed_ms(h3_gpu *gpu, h3_gpu_event *start, h3_gpu_event *end, float *ms);
/* Dominant-kernel timing: while enabled, each BF16 / Sage attention dispatch and
 * each tiled GEMM records HIP events on the compute stream around its main
 * kernel only (not the V transpose, the quantizers or small fallbacks).
 * h3_hip_kernel_timing_read (after submit) returns the summed milliseconds and
 * the number of timed launches, and clears them. Enabling or disabling also clears. */
int h3_hip_kernel_timing(h3_gpu *gpu, int enable);
int h3_hip_kernel_timing_read(h3_gpu *gpu, double *ms_total, uint64_t *launches);

#ifdef __cplusplus
}
#endif
#endif
