/* h3_gpu.h — C ABI of the MI355X (gfx950) backend for h3cli's DiT denoise hot path.
 *
 * Every declaration below has the same name, argument order and meaning as the
 * entry point it replaces in h3cli's operator surface, reference
 * `src/gpu.h` (cited per function as gpu.h:LINE). A caller written against the
 * reference header links against libh3hip.so unchanged for these symbols.
 *
 * Conventions (reference gpu.h:12-33, gpu_cuda.cu:429-477):
 *   - opaque handles; int-returning calls give 1 on success, 0 on error and
 *     pointer-returning calls give NULL on error; h3_gpu_error() holds the text;
 *   - all device work is queued on one ordered compute stream between
 *     h3_gpu_begin() and h3_gpu_submit(); asynchronous device faults (non-finite
 *     attention input, quantizer faults) are deferred and reported by submit;
 *   - bf16 values travel as uint16_t bit patterns.
 */
#ifndef H3_GPU_H
#define H3_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct h3_gpu h3_gpu;               /* gpu.h:12 */
typedef struct h3_gpu_tensor h3_gpu_tensor; /* gpu.h:13 */
typedef struct h3_gpu_event h3_gpu_event;   /* gpu.h:14 */

typedef enum {                              /* gpu.h:16-22 */
    H3_GPU_F32 = 0,
    H3_GPU_BF16,
    H3_GPU_I8,
    H3_GPU_U32,
    H3_GPU_F16
} h3_gpu_dtype;

typedef enum { H3_GPU_HOST_VISIBLE, H3_GPU_DEVICE_ONLY, H3_GPU_HOST_PINNED }
    h3_gpu_storage;                         /* gpu.h:24-25 */

/* Statistics block, field-for-field the reference layout (gpu.h:99-142) so a
 * caller's struct matches. Fields this backend does not produce stay zero. */
typedef struct {
    uint64_t q8_weights, q8_source_bytes, q8_storage_bytes, q8_dispatches;
    double q8_load_seconds;
    uint64_t layout_prepares, layout_inplace_packs, layout_scan_replaced_bytes, layout_partial_bytes;
    uint64_t allocated_bytes;
    uint64_t live_bytes;
    uint64_t peak_live_bytes;
    uint64_t tensor_allocations;
    uint64_t direct_dispatches;
    uint64_t mps_linear_dispatches;
    uint64_t mps_conv_dispatches;
    uint64_t mps_sdpa_dispatches;
    uint64_t native_attention_dispatches;
    uint64_t metal_current_allocated_bytes;
    uint64_t blit_copies;
    uint64_t submissions;
    double command_encode_seconds;
    double command_wait_seconds;
    double gpu_seconds;
    uint64_t linear_dispatches, conv_dispatches, attention_dispatches;
    uint64_t h2d_bytes, d2h_bytes, d2d_bytes, streamed_bytes;
    uint64_t resident_weight_bytes, stream_slot_bytes, resident_block_mask;
    unsigned resident_blocks, active_weight_blocks;
    uint64_t device_bytes, managed_bytes, pinned_bytes, peak_pinned_bytes;
    uint64_t stream_stalls;
    double transfer_seconds, stream_wait_seconds, linear_seconds, attention_seconds;
    double conv_seconds;
    double h2d_seconds, d2h_seconds, slot_wait_seconds, normalization_seconds;
    uint64_t weight_cache_bytes, weight_cache_hits, weight_cache_hit_bytes;
    uint64_t weight_cache_misses, weight_cache_evictions;
    double quant_conversion_seconds;
    uint64_t quant_clipped_values, quant_zeroed_values;
    uint64_t quant_projection_dispatches, quant_cache_hits, quant_cache_misses;
    uint64_t sage2_attention_dispatches, sage3_attention_dispatches, attention_workspace_bytes;
    uint64_t inflight_peak, command_retirements, bounded_waits, pressure_drains;
    uint64_t native_scratch_bytes, native_scratch_allocations, native_scratch_reuses, native_pipeline_count;
    uint64_t main_dense_calls, subblock_calls, subblock_bypass, subblock_protected_calls;
    uint64_t subblock_selected, subblock_possible, subblock_router_calls;
    uint64_t attention_timing_samples, attention_timing_missed;
    double main_attention_seconds, subblock_router_seconds, subblock_kernel_seconds;
} h3_gpu_stats;

/* ---- context ---------------------------------------------------------- */
/* gpu.h:144. shader_source_path is accepted and ignored (kernels are built
 * into the library). */
h3_gpu *h3_gpu_create(const char *shader_source_path, char *error, size_t error_size);
void h3_gpu_free(h3_gpu *gpu);                          /* gpu.h:180 */
void h3_gpu_cancel(h3_gpu *gpu);                        /* gpu.h:182 */
const char *h3_gpu_backend_name(const h3_gpu *gpu);     /* gpu.h:203 */
int h3_gpu_begin(h3_gpu *gpu);                          /* gpu.h:260 */
int h3_gpu_continue(h3_gpu *gpu);                       /* gpu.h:263 */
int h3_gpu_submit(h3_gpu *gpu);                         /* gpu.h:264 */
int h3_gpu_synchronize(h3_gpu *gpu);                    /* gpu.h:266 */
const char *h3_gpu_error(const h3_gpu *gpu);            /* gpu.h:267 */
int h3_gpu_get_stats(const h3_gpu *gpu, h3_gpu_stats *stats); /* gpu.h:268 */

/* ---- tensors ---------------------------------------------------------- */
h3_gpu_tensor *h3_gpu_tensor_alloc(h3_gpu *gpu, size_t elements,
                                   h3_gpu_dtype dtype, h3_gpu_storage storage); /* gpu.h:26 */
void *h3_gpu_tensor_contents(h3_gpu_tensor *tensor);    /* gpu.h:29 */
h3_gpu_tensor *h3_gpu_tensor_new_f32(h3_gpu *gpu, size_t elements);  /* gpu.h:209 */
h3_gpu_tensor *h3_gpu_tensor_new_bf16(h3_gpu *gpu, size_t elements); /* gpu.h:210 */
h3_gpu_tensor *h3_gpu_tensor_new_i8(h3_gpu *gpu, size_t elements);   /* gpu.h:211 */
h3_gpu_tensor *h3_gpu_tensor_from_f32(h3_gpu *gpu, const float *values, size_t elements);     /* gpu.h:212 */
h3_gpu_tensor *h3_gpu_tensor_from_bf16(h3_gpu *gpu, const uint16_t *values, size_t elements); /* gpu.h:214 */
h3_gpu_tensor *h3_gpu_tensor_from_u32(h3_gpu *gpu, const uint32_t *values, size_t elements);  /* gpu.h:216 */
/* gpu.h:228. Fill an existing BF16 tensor from a file (pread into pinned
 * bounce buffers, then asynchronous copies on the copy stream). May run on an
 * I/O thread while the compute stream uses other tensors. */
int h3_gpu_tensor_read_file_bf16(h3_gpu_tensor *tensor, const char *path,
                                 uint64_t file_offset, size_t elements,
                                 char *error, size_t error_size);
int h3_gpu_tensor_stream_file_bf16(h3_gpu_tensor *tensor, const char *path,
                                   uint64_t file_offset, size_t elements,
                                   char *error, size_t error_size); /* gpu.h:234 */
void h3_gpu_tensor_free(h3_gpu_tensor *tensor);                 /* gpu.h:237 */
size_t h3_gpu_tensor_elements(const h3_gpu_tensor *tensor);     /* gpu.h:238 */
h3_gpu_dtype h3_gpu_tensor_dtype(const h3_gpu_tensor *tensor);  /* gpu.h:239 */
int h3_gpu_tensor_read_f32(const h3_gpu_tensor *tensor, float *values, size_t elements); /* gpu.h:240 */
int h3_gpu_tensor_read_f32_range(const h3_gpu_tensor *tensor, size_t source_offset,
                                 float *values, size_t elements);                       /* gpu.h:242 */
int h3_gpu_tensor_read_bf16(const h3_gpu_tensor *tensor, uint16_t *values, size_t elements); /* gpu.h:245 */
int h3_gpu_tensor_read_u32(const h3_gpu_tensor *tensor, uint32_t *values, size_t elements);  /* gpu.h:247 */
int h3_gpu_tensor_write_f32(h3_gpu_tensor *tensor, const float *values, size_t elements);    /* gpu.h:249 */
int h3_gpu_tensor_write_f32_range(h3_gpu_tensor *tensor, size_t destination_offset,
                                  const float *values, size_t elements);                    /* gpu.h:251 */
int h3_gpu_tensor_write_bf16(h3_gpu_tensor *tensor, const uint16_t *values, size_t elements); /* gpu.h:254 */
int h3_gpu_tensor_write_bf16_range(h3_gpu_tensor *tensor, size_t destination_offset,
                                   const uint16_t *values, size_t elements);                 /* gpu.h:256 */

/* ---- events (copy-stream / compute-stream ordering) -------------------- */
h3_gpu_event *h3_gpu_event_new(h3_gpu *gpu);                    /* gpu.h:30 */
int h3_gpu_event_record(h3_gpu *gpu, h3_gpu_event *event);      /* gpu.h:31 */
int h3_gpu_event_wait(h3_gpu *gpu, h3_gpu_event *event);        /* gpu.h:32 */
void h3_gpu_event_free(h3_gpu_event *event);                    /* gpu.h:33 */

/* ---- quantized projection weights -------------------------------------- */
/* gpu.h:44 (reference src/cuda/cuda_quant.cuh:120-162). mode 0 = BF16
 * projections (no cache is touched), 1 = FP8 W8A8 (tensorwide E4M3 weights
 * and activations, FP32 accumulation, BF16 output), 2 = NVFP4 W4A4 (E2M1 with
 * UE4M3 scales per 16 values and a tensorwide scale; the same packed format,
 * multiplied as exact BF16 dequantized values). cache: artifact directory (NULL: $HOME/.cache/h3/
 * denoise-quant), created if missing. bf16_weights: BF16 bytes of whole H3
 * blocks' four projections, for the resident/streamed plan; force_stream
 * keeps packed weights in pinned host memory. */
int h3_gpu_quant_configure(h3_gpu *gpu, int mode, const char *cache,
                           uint64_t bf16_weights, uint64_t activations, int force_stream);
/* gpu.h:46 (cuda_quant.cuh:249-330). rows x columns BF16 weights at offset
 * of a file (multiples of 128), packed to the configured mode's descriptor
 * through the content-hashed H3QWT001 artifact cache (every load hashes its
 * source; the reference's H3_QUANT_VERIFY=1 behaviour). The result is passed
 * to h3_gpu_linear_bf16 like a BF16 weight (no bias). */
h3_gpu_tensor *h3_gpu_quant_load(h3_gpu *gpu, const char *path, uint64_t offset,
                                 uint32_t rows, uint32_t columns);
/* gpu.h:74. rows x columns BF16 weights from a file packed as q8 (int8
 * [rows, columns] + fp32 scale per 64-wide column group, round-half-even;
 * reference src/weights/q8.c:26-56) for W8A16 projections. */
h3_gpu_tensor *h3_gpu_q8_load(h3_gpu *gpu, const char *path, uint64_t offset,
                              uint32_t rows, uint32_t columns);

/* ---- DiT attention ---------------------------------------------------- */
/* gpu.h:52. mode: 0 default (dense BF16), 1 sage2++ (int8 QK / fp8 PV),
 * 3 sol (centroid-routed; reads the thread-current h3_cuda_sol_options as
 * gpu_cuda.cu:1553-1555 does), 4 subblock (block-sparse); 2 sage3 is
 * rejected as unsupported (reference src/denoise/attention.h:7). Once per
 * context. */
int h3_gpu_dit_attention_configure(h3_gpu *gpu, int mode);
/* gpu.h:53-55. Q,K,V sequence-major BF16 [seq,heads,dim]; out [seq,heads,dim]
 * or head-major [heads,seq,dim]. dim must be 128; heads is any value >= 1
 * (the reference fixes 56, gpu_cuda.cu:1607). The scale is rounded to BF16 as
 * the reference does (gpu_cuda.cu:1652-1654). */
int h3_gpu_dit_sdpa_bf16(h3_gpu *gpu, h3_gpu_tensor *out, const h3_gpu_tensor *q,
                         const h3_gpu_tensor *k, const h3_gpu_tensor *v, uint32_t seq,
                         uint32_t heads, uint32_t dim, float scale, int head_major,
                         unsigned block, int step);
/* gpu.h:67. Binds the absolute sampler step used by sparse modes. */
int h3_gpu_dit_attention_noise(h3_gpu *gpu, int step, float video_sigma, float audio_sigma);
/* Plain SDPA entry points (gpu.h:703 and gpu.h:709; gpu_cuda.cu:1233-1235). */
int h3_gpu_sdpa_bf16(h3_gpu *gpu, h3_gpu_tensor *out, const h3_gpu_tensor *q,
                     const h3_gpu_tensor *k, const h3_gpu_tensor *v,
                     uint32_t seq, uint32_t heads, uint32_t dim, float scale);
int h3_gpu_sdpa_bf16_head_major_output(h3_gpu *gpu, h3_gpu_tensor *out,
                     const h3_gpu_tensor *q, const h3_gpu_tensor *k, const h3_gpu_tensor *v,
                     uint32_t seq, uint32_t heads, uint32_t dim, float scale);

/* ---- DiT block operators ---------------------------------------------- */
/* gpu.h:501. y[rows,output_dim] = x[rows,input_dim] . W[output_dim,input_dim]^T (+bias),
 * FP32 accumulate, BF16 out. A q8 weight dispatches the W8A16 GEMM. */
int h3_gpu_linear_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input,
                       const h3_gpu_tensor *weight, const h3_gpu_tensor *bias,
                       uint32_t rows, uint32_t input_dim, uint32_t output_dim);
/* gpu.h:714. out[rows,width] = silu(fused[:, :width]) * fused[:, width:]. */
int h3_gpu_swiglu_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input,
                       uint32_t rows, uint32_t width);
/* gpu.h:506. fc1 (2*hidden) -> SwiGLU -> fc2 (gpu_cuda.cu:1108-1112). */
int h3_gpu_mlp_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input,
                    const h3_gpu_tensor *fc1_weight, const h3_gpu_tensor *fc2_weight,
                    uint32_t rows, uint32_t input_dim, uint32_t hidden_dim, uint32_t output_dim);
/* gpu.h:575. approximate=1: tanh form (cuda_kernels.cuh:879-902). */
int h3_gpu_gelu_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input,
                     uint32_t elements, int approximate);
/* gpu.h:586. y = bf16(fma(x*rsqrt(mean(x^2)+eps)*w, 1+scale, shift)), modulation
 * [map_rows, slots, width] BF16 indexed by row_map[row] (U32). */
int h3_gpu_adaln_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input,
                      const h3_gpu_tensor *norm_weight, const h3_gpu_tensor *modulation,
                      const h3_gpu_tensor *row_map, uint32_t rows, uint32_t width,
                      uint32_t slots, uint32_t shift_slot, uint32_t scale_slot, float epsilon);
/* gpu.h:612. out = bf16(residual + branch*gate). */
int h3_gpu_gate_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *residual,
                     const h3_gpu_tensor *branch, const h3_gpu_tensor *modulation,
                     const h3_gpu_tensor *row_map, uint32_t rows, uint32_t width,
                     uint32_t slots, uint32_t gate_slot);
/* gpu.h:618. gate then AdaLN of the gated residual, fused in one pass. */
int h3_gpu_gate_adaln_bf16(h3_gpu *gpu, h3_gpu_tensor *gated_residual, h3_gpu_tensor *output,
                           const h3_gpu_tensor *residual, const h3_gpu_tensor *branch,
                           const h3_gpu_tensor *norm_weight, const h3_gpu_tensor *gate_modulation,
                           const h3_gpu_tensor *norm_modulation, const h3_gpu_tensor *row_map,
                           uint32_t rows, uint32_t width, uint32_t slots, uint32_t gate_slot,
                           uint32_t shift_slot, uint32_t scale_slot, float epsilon);
/* gpu.h:643. qkv [seq, 3, heads, dim] -> per-head RMSNorm of Q and K (weights
 * q_norm/k_norm [dim]) then rotate-half RoPE on the first 2*rope_half dims
 * (pair d <-> d+rope_half, cos/sin [seq, rope_half]); V copied. dim <= 256.
 * Extension: q_norm = k_norm = NULL skips the Q/K RMSNorm (RoPE only). */
int h3_gpu_qkv_rope_bf16(h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key,
                         h3_gpu_tensor *value, const h3_gpu_tensor *qkv,
                         const h3_gpu_tensor *q_norm, const h3_gpu_tensor *k_norm,
                         const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin,
                         uint32_t sequence, uint32_t heads, uint32_t head_dim,
                         uint32_t rope_half, float epsilon);
/* gpu.h:654. As above with H3's grouped rows [seq, heads, 3, dim]. */
int h3_gpu_grouped_qkv_rope_bf16(h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key,
                                 h3_gpu_tensor *value, const h3_gpu_tensor *qkv,
                                 const h3_gpu_tensor *q_norm, const h3_gpu_tensor *k_norm,
                                 const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin,
                                 uint32_t sequence, uint32_t heads, uint32_t head_dim,
                                 uint32_t rope_half, float epsilon);
/* gpu.h:667. Grouped QKV projection followed by the norm/RoPE split. */
int h3_gpu_grouped_qkv_linear_rope_bf16(h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key,
                                        h3_gpu_tensor *value, h3_gpu_tensor *qkv,
                                        const h3_gpu_tensor *input, const h3_gpu_tensor *weight,
                                        const h3_gpu_tensor *q_norm, const h3_gpu_tensor *k_norm,
                                        const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin,
                                        uint32_t rows, uint32_t input_dim, uint32_t heads,
                                        uint32_t head_dim, uint32_t rope_half, float epsilon);
/* gpu.h:329 and gpu.h:331. Element casts (round-to-nearest-even to BF16). */
int h3_gpu_cast_f32_to_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, uint32_t elements);
int h3_gpu_cast_bf16_to_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, uint32_t elements);
/* gpu.h:750. out = bf16(left + right). */
int h3_gpu_add_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *left,
                    const h3_gpu_tensor *right, uint32_t elements);
/* gpu.h:564. out = bf16(x / (1 + exp(-x))). */
int h3_gpu_silu_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, uint32_t elements);
/* gpu.h:815-818. sample[offset+i] += delta*(last + ratio*(last - previous)). */
int h3_gpu_euler_bf16(h3_gpu *gpu, h3_gpu_tensor *sample, size_t sample_offset,
                      const h3_gpu_tensor *last, const h3_gpu_tensor *previous,
                      uint32_t elements, float delta, float ratio);

#ifdef __cplusplus
}
#endif
#endif
