/* h3_gpu_surface.h — the rest of the reference operator surface (src/gpu.h)
 * that a drop-in backend must link: every symbol of the reference's
 * tests/test_gpu_contract.c:152-181 (non-Apple branch) beyond include/h3_gpu.h.
 *
 * The first group is implemented on gfx950 (DiT-path helpers, weight planning,
 * profiling marks). The second group lies outside the DiT denoise path (VAE,
 * audio, text and vision encoders, SGLang-parity and Metal int8 paths): each
 * returns 0 / NULL and sets "<name>: unsupported on the HIP backend", as the
 * reference's CUDA backend does for Metal-only ops (src/cuda/gpu_cuda.cu:1358-1532).
 * Each declaration cites the src/gpu.h line it matches. */
#ifndef H3_GPU_SURFACE_H
#define H3_GPU_SURFACE_H
#include "h3_gpu.h"
#include "h3_residency.h"
#ifdef __cplusplus
extern "C" {
#endif

/* src/denoise/sol.h:7-11: block metadata ABI of the SOL / SubBlock layout. */
typedef struct { uint32_t protect; int32_t first_frame, last_frame; uint32_t rows; } h3_sol_block;
typedef struct {
    uint32_t sequence, query_blocks, key_blocks, protected_rows;
    h3_sol_block *query, *key;
} h3_sol_layout;

/* gpu.h:189-193 */
typedef enum { H3_QWEN_GQA_REFERENCE, H3_QWEN_GQA_SCALED_Q, H3_QWEN_GQA_LEGACY } h3_qwen_gqa_scale_mode;
/* Passed by pointer only (gpu.h:183-187; src/denoise/adaptive_cache.h:21). */
typedef struct h3_gqa_limits h3_gqa_limits;
typedef struct h3_adaptive_regions h3_adaptive_regions;

/* ---- implemented ---------------------------------------------------------- */
int h3_gpu_prefers_device_sampler(const h3_gpu *gpu, int continuation); /* gpu.h:204 */
int h3_gpu_should_retry_streaming(const h3_gpu *gpu); /* gpu.h:205 */
int h3_gpu_plan_weights(h3_gpu *gpu, uint64_t weights, uint64_t activations); /* gpu.h:36 */
int h3_gpu_release_weight_cache(h3_gpu *gpu); /* gpu.h:50 */
int h3_qwen_gqa_scale_parse(const char *value, h3_qwen_gqa_scale_mode *mode, char *error, size_t error_size); /* gpu.h:194 */
const char *h3_qwen_gqa_scale_name(h3_qwen_gqa_scale_mode mode); /* gpu.h:196 */
int h3_gpu_is_m5(const h3_gpu *gpu); /* gpu.h:201 */
int h3_gpu_has_nax_mlp(const h3_gpu *gpu); /* gpu.h:206 */
int h3_gpu_has_int8_mlp(const h3_gpu *gpu); /* gpu.h:207 */
int h3_gpu_tensor_is_file_mapped(const h3_gpu_tensor *tensor); /* gpu.h:220 */
h3_gpu_tensor *h3_gpu_tensor_load_bf16(h3_gpu *gpu, const char *path, uint64_t file_offset, size_t elements); /* gpu.h:221 */
h3_gpu_tensor *h3_gpu_tensor_load_f32(h3_gpu *gpu, const char *path, uint64_t file_offset, size_t elements); /* gpu.h:223 */
void h3_gpu_profile_set_label(h3_gpu *gpu, const char *label); /* gpu.h:271 */
void h3_gpu_profile_mark(h3_gpu *gpu, const char *phase); /* gpu.h:272 */
int h3_gpu_patch_linear_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t rows, uint32_t input_dim, uint32_t output_dim); /* gpu.h:307 */
int h3_gpu_patch_linear_bf16_offset(h3_gpu *gpu, h3_gpu_tensor *output, size_t output_offset, const h3_gpu_tensor *input, size_t input_offset, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t rows, uint32_t input_dim, uint32_t output_dim); /* gpu.h:312 */
int h3_gpu_patch_linear_bf16_map(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, const h3_gpu_tensor *row_map, uint32_t output_rows, uint32_t rows, uint32_t input_dim, uint32_t output_dim); /* gpu.h:319 */
int h3_gpu_copy_bf16(h3_gpu *gpu, h3_gpu_tensor *destination, size_t destination_offset, const h3_gpu_tensor *source, size_t source_offset, size_t elements); /* gpu.h:333 */
int h3_gpu_copy_f32(h3_gpu *gpu, h3_gpu_tensor *destination, size_t destination_offset, const h3_gpu_tensor *source, size_t source_offset, size_t elements); /* gpu.h:337 */
int h3_gpu_rms_norm_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, uint32_t rows, uint32_t width, float epsilon); /* gpu.h:566 */
int h3_gpu_adaln_bf16_offset(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, size_t input_offset, const h3_gpu_tensor *norm_weight, const h3_gpu_tensor *modulation, const h3_gpu_tensor *row_map, uint32_t rows, uint32_t width, uint32_t slots, uint32_t shift_slot, uint32_t scale_slot, float epsilon); /* gpu.h:593 */
int h3_gpu_head_rms_norm_bf16(h3_gpu *gpu, h3_gpu_tensor *tensor, const h3_gpu_tensor *weight, uint32_t sequence, uint32_t heads, uint32_t head_dim, float epsilon); /* gpu.h:733 */
int h3_gpu_sub_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *left, const h3_gpu_tensor *right, uint32_t elements); /* gpu.h:753 */
int h3_gpu_silu_mul_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *gate, const h3_gpu_tensor *up, uint32_t elements); /* gpu.h:845 */
int h3_gpu_plan_bf16_weights(h3_gpu *gpu, uint64_t active_mask, uint64_t block_bytes, uint64_t future_bytes, int force_stream, int retry_cap, h3_weight_plan *plan); /* gpu.h:38 */
int h3_gpu_weight_plan_compatible(h3_gpu *gpu, int force_stream); /* gpu.h:40 */
int h3_gpu_dit_sol_layout(h3_gpu *gpu, const h3_sol_layout *layout); /* gpu.h:66 */

/* ---- outside the DiT denoise path: "unsupported on the HIP backend" -------- */
int h3_gpu_gqa_causal_limits(h3_gpu *gpu, h3_gqa_limits *limits); /* gpu.h:197 */
size_t h3_gpu_gqa_causal_max_sequence(h3_gpu *gpu); /* gpu.h:198 */
int h3_gpu_gqa_causal_preflight(h3_gpu *gpu, size_t sequence, char *error, size_t error_size); /* gpu.h:199 */
int h3_gpu_linear_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t rows, uint32_t input_dim, uint32_t output_dim); /* gpu.h:303 */
int h3_gpu_silu_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, uint32_t elements); /* gpu.h:327 */
int h3_gpu_rms_norm_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, uint32_t rows, uint32_t width, float epsilon); /* gpu.h:341 */
int h3_gpu_adaln_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *norm_weight, const h3_gpu_tensor *modulation, const h3_gpu_tensor *row_map, uint32_t rows, uint32_t width, uint32_t slots, uint32_t shift_slot, uint32_t scale_slot, float epsilon); /* gpu.h:345 */
int h3_gpu_gate_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *residual, const h3_gpu_tensor *branch, const h3_gpu_tensor *modulation, const h3_gpu_tensor *row_map, uint32_t rows, uint32_t width, uint32_t slots, uint32_t gate_slot); /* gpu.h:352 */
int h3_gpu_qkv_rope_f32(h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key, h3_gpu_tensor *value, const h3_gpu_tensor *qkv, const h3_gpu_tensor *q_norm, const h3_gpu_tensor *k_norm, const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin, uint32_t sequence, uint32_t heads, uint32_t head_dim, uint32_t rope_half, float epsilon); /* gpu.h:358 */
int h3_gpu_sdpa_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *query, const h3_gpu_tensor *key, const h3_gpu_tensor *value, uint32_t sequence, uint32_t heads, uint32_t head_dim, float scale); /* gpu.h:367 */
int h3_gpu_swiglu_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *fused, uint32_t rows, uint32_t width); /* gpu.h:371 */
int h3_gpu_scale_add_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *residual, const h3_gpu_tensor *branch, const h3_gpu_tensor *scale, uint32_t rows, uint32_t width); /* gpu.h:374 */
int h3_gpu_layer_norm_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t rows, uint32_t width, float epsilon); /* gpu.h:379 */
int h3_gpu_video_qkv_rope_f32(h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key, h3_gpu_tensor *value, const h3_gpu_tensor *qkv, const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin, uint32_t sequence, uint32_t heads, uint32_t head_dim, uint32_t rope_half, float epsilon); /* gpu.h:384 */
int h3_gpu_conv1d_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t batch, uint32_t length, uint32_t input_channels, uint32_t output_channels, uint32_t kernel, uint32_t padding, uint32_t dilation); /* gpu.h:403 */
int h3_gpu_conv1d_stride_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t batch, uint32_t length, uint32_t input_channels, uint32_t output_channels, uint32_t kernel, uint32_t stride, uint32_t padding, uint32_t dilation); /* gpu.h:410 */
int h3_gpu_conv_transpose1d_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t batch, uint32_t length, uint32_t input_channels, uint32_t output_channels, uint32_t kernel, uint32_t stride, uint32_t padding); /* gpu.h:418 */
int h3_gpu_weight_norm_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *vector, const h3_gpu_tensor *magnitude, uint32_t outer, uint32_t inner); /* gpu.h:426 */
int h3_gpu_add_scaled_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *left, const h3_gpu_tensor *right, float left_scale, float right_scale, uint32_t elements); /* gpu.h:430 */
int h3_gpu_alias_free_snake_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *alpha_log, const h3_gpu_tensor *beta_log, const h3_gpu_tensor *upsample_filter, const h3_gpu_tensor *downsample_filter, uint32_t batch, uint32_t length, uint32_t channels); /* gpu.h:434 */
int h3_gpu_snake1d_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *alpha, uint32_t batch, uint32_t length, uint32_t channels); /* gpu.h:443 */
int h3_gpu_audio_qkv_split_f32(h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key, h3_gpu_tensor *value, const h3_gpu_tensor *qkv, const h3_gpu_tensor *q_bias, const h3_gpu_tensor *k_bias, const h3_gpu_tensor *v_bias, uint32_t batch, uint32_t length, uint32_t heads, uint32_t head_dim); /* gpu.h:447 */
int h3_gpu_sdpa_causal_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *query, const h3_gpu_tensor *key, const h3_gpu_tensor *value, uint32_t batch, uint32_t sequence, uint32_t heads, uint32_t head_dim, float scale); /* gpu.h:455 */
int h3_gpu_audio_attention_pool_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *attended, uint32_t batch, uint32_t length, uint32_t heads, uint32_t head_dim, uint32_t output_dim); /* gpu.h:461 */
int h3_gpu_geglu_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *gate, const h3_gpu_tensor *linear, uint32_t elements); /* gpu.h:466 */
int h3_gpu_clip_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, uint32_t elements, float minimum, float maximum); /* gpu.h:469 */
int h3_gpu_vae_encoder_pad_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, uint32_t batch, uint32_t depth, uint32_t height, uint32_t width, uint32_t channels, uint32_t depth_front, uint32_t height_before, uint32_t height_after, uint32_t width_before, uint32_t width_after); /* gpu.h:475 */
int h3_gpu_conv3d_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t batch, uint32_t depth, uint32_t height, uint32_t width, uint32_t input_channels, uint32_t output_channels, uint32_t kernel_depth, uint32_t kernel_height, uint32_t kernel_width, uint32_t stride_depth, uint32_t stride_height, uint32_t stride_width); /* gpu.h:482 */
int h3_gpu_vae_encoder_group_norm_silu_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t batch, uint32_t depth, uint32_t height, uint32_t width, uint32_t channels, uint32_t groups, float epsilon); /* gpu.h:491 */
int h3_gpu_mlp_nax_bf16(h3_gpu *gpu, h3_gpu_tensor *output, h3_gpu_tensor *activated, const h3_gpu_tensor *input, const h3_gpu_tensor *fc1_weight, const h3_gpu_tensor *fc2_weight, uint32_t rows, uint32_t input_dim, uint32_t hidden_dim, uint32_t output_dim); /* gpu.h:514 */
int h3_gpu_quantize_weight_int8(h3_gpu *gpu, h3_gpu_tensor *output, h3_gpu_tensor *scales, const h3_gpu_tensor *input, uint32_t rows, uint32_t columns); /* gpu.h:523 */
int h3_gpu_linear_int8_bf16(h3_gpu *gpu, h3_gpu_tensor *output, h3_gpu_tensor *quantized_input, h3_gpu_tensor *input_scales, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *weight_scales, uint32_t rows, uint32_t input_dim, uint32_t output_dim, int use_slower_uncached_int8_scales); /* gpu.h:527 */
int h3_gpu_linear_int8_head_major_bf16(h3_gpu *gpu, h3_gpu_tensor *output, h3_gpu_tensor *quantized_input, h3_gpu_tensor *input_scales, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *weight_scales, uint32_t rows, uint32_t heads, uint32_t head_dim, uint32_t output_dim); /* gpu.h:538 */
int h3_gpu_mlp_int8_bf16(h3_gpu *gpu, h3_gpu_tensor *output, h3_gpu_tensor *activated, h3_gpu_tensor *quantized_activation, h3_gpu_tensor *activation_scales, const h3_gpu_tensor *input, const h3_gpu_tensor *fc1_weight, const h3_gpu_tensor *fc1_scales, const h3_gpu_tensor *fc2_weight, const h3_gpu_tensor *fc2_scales, const h3_gpu_tensor *fc1_bf16, const h3_gpu_tensor *fc2_bf16, uint32_t rows, uint32_t input_dim, uint32_t hidden_dim, uint32_t output_dim, int use_slower_grouped_quantizer, int use_slower_dynamic_fc1_k, int use_int8_row_fc2, int input_is_quantized); /* gpu.h:547 */
int h3_gpu_layer_norm_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t rows, uint32_t width, float epsilon); /* gpu.h:570 */
int h3_gpu_vision_qkv_rope_bf16(h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key, h3_gpu_tensor *value, const h3_gpu_tensor *qkv, const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin, uint32_t sequence, uint32_t heads, uint32_t head_dim, uint32_t rope_half); /* gpu.h:578 */
int h3_gpu_adaln_linear_bf16(h3_gpu *gpu, h3_gpu_tensor *output, h3_gpu_tensor *inverse, const h3_gpu_tensor *input, size_t input_offset, const h3_gpu_tensor *norm_weight, const h3_gpu_tensor *modulation, const h3_gpu_tensor *row_map, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t rows, uint32_t width, uint32_t output_dim, uint32_t slots, uint32_t shift_slot, uint32_t scale_slot, float epsilon); /* gpu.h:600 */
int h3_gpu_gate_adaln_quantize_int8(h3_gpu *gpu, h3_gpu_tensor *gated_residual, h3_gpu_tensor *quantized_output, h3_gpu_tensor *quantized_scales, const h3_gpu_tensor *residual, const h3_gpu_tensor *branch, const h3_gpu_tensor *norm_weight, const h3_gpu_tensor *gate_modulation, const h3_gpu_tensor *norm_modulation, const h3_gpu_tensor *row_map, uint32_t rows, uint32_t padded_rows, uint32_t width, uint32_t slots, uint32_t gate_slot, uint32_t shift_slot, uint32_t scale_slot, float epsilon); /* gpu.h:630 */
int h3_gpu_grouped_qkv_linear_rope_int8(h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key, h3_gpu_tensor *value, h3_gpu_tensor *quantized_input, h3_gpu_tensor *input_scales, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *weight_scales, const h3_gpu_tensor *q_norm, const h3_gpu_tensor *k_norm, const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin, uint32_t rows, uint32_t input_dim, uint32_t heads, uint32_t head_dim, uint32_t rope_half, float epsilon, int input_is_quantized, int use_slower_unfused_qkv_rope, int use_slower_scalar_qkv_rms, int use_slower_uncached_int8_scales); /* gpu.h:682 */
int h3_gpu_embedding_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *weight, const h3_gpu_tensor *token_ids, uint32_t tokens, uint32_t vocab_size, uint32_t width); /* gpu.h:717 */
int h3_gpu_text_qk_rope_bf16(h3_gpu *gpu, h3_gpu_tensor *query_output, h3_gpu_tensor *key_output, const h3_gpu_tensor *query_input, const h3_gpu_tensor *key_input, const h3_gpu_tensor *q_norm, const h3_gpu_tensor *k_norm, const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin, uint32_t sequence, uint32_t query_heads, uint32_t kv_heads, uint32_t head_dim, float epsilon); /* gpu.h:721 */
int h3_gpu_rope_text_bf16(h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key, const h3_gpu_tensor *rope_cos_f32, const h3_gpu_tensor *rope_sin_f32, uint32_t sequence, uint32_t query_heads, uint32_t kv_heads, uint32_t head_dim); /* gpu.h:737 */
int h3_gpu_gqa_causal_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *query, const h3_gpu_tensor *key, const h3_gpu_tensor *value, uint32_t sequence, uint32_t query_heads, uint32_t kv_heads, uint32_t head_dim, float scale); /* gpu.h:743 */
int h3_gpu_token_pool_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, size_t input_offset, h3_gpu_tensor *original, size_t original_offset, h3_gpu_tensor *baseline, size_t baseline_offset, const h3_gpu_tensor *baseline_indices, const h3_gpu_tensor *pairs, uint32_t input_rows, uint32_t rows, uint32_t baseline_rows, uint32_t width); /* gpu.h:756 */
int h3_gpu_token_pool_adaln_bf16(h3_gpu *gpu, h3_gpu_tensor *residual, h3_gpu_tensor *output, const h3_gpu_tensor *input, size_t input_offset, h3_gpu_tensor *original, size_t original_offset, h3_gpu_tensor *baseline, size_t baseline_offset, const h3_gpu_tensor *baseline_indices, const h3_gpu_tensor *pairs, const h3_gpu_tensor *norm_weight, const h3_gpu_tensor *modulation, const h3_gpu_tensor *row_map, uint32_t input_rows, uint32_t rows, uint32_t baseline_rows, uint32_t width, uint32_t slots, uint32_t shift_slot, uint32_t scale_slot, float epsilon); /* gpu.h:767 */
int h3_gpu_token_expand_delta_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *original, size_t original_offset, const h3_gpu_tensor *reduced, const h3_gpu_tensor *baseline, size_t baseline_offset, const h3_gpu_tensor *baseline_indices, const h3_gpu_tensor *parents, uint32_t rows, uint32_t reduced_rows, uint32_t baseline_rows, uint32_t width, uint32_t exact_prefix_rows, float update_scale); /* gpu.h:782 */
int h3_gpu_token_expand_adaln_bf16(h3_gpu *gpu, h3_gpu_tensor *residual, h3_gpu_tensor *output, const h3_gpu_tensor *original, size_t original_offset, const h3_gpu_tensor *reduced, const h3_gpu_tensor *baseline, size_t baseline_offset, const h3_gpu_tensor *baseline_indices, const h3_gpu_tensor *parents, const h3_gpu_tensor *norm_weight, const h3_gpu_tensor *modulation, const h3_gpu_tensor *row_map, uint32_t rows, uint32_t reduced_rows, uint32_t baseline_rows, uint32_t width, uint32_t exact_prefix_rows, float update_scale, uint32_t slots, uint32_t shift_slot, uint32_t scale_slot, float epsilon); /* gpu.h:795 */
int h3_gpu_video_preview_bf16(h3_gpu *gpu, h3_gpu_tensor *scratch, const h3_gpu_tensor *sample, size_t sample_offset, const h3_gpu_tensor *last, const h3_gpu_tensor *previous, const h3_gpu_tensor *row_classes, const h3_gpu_tensor *strengths, uint32_t time, uint32_t height, uint32_t width, float sigma_next, float ratio); /* gpu.h:824 */
int h3_gpu_video_preview_read(const h3_gpu_tensor *scratch, float *latent, size_t elements); /* gpu.h:829 */
int h3_gpu_bridge_euler_bf16(h3_gpu *gpu, h3_gpu_tensor *sample, size_t sample_offset, const h3_gpu_tensor *last, const h3_gpu_tensor *previous, const h3_gpu_tensor *row_classes, const h3_gpu_tensor *strengths, uint32_t rows, uint32_t row_width, float delta, float ratio); /* gpu.h:834 */
int h3_gpu_bridge_check_exact(h3_gpu *gpu, const h3_gpu_tensor *sample, size_t sample_offset, const h3_gpu_tensor *initial, const h3_gpu_tensor *row_classes, const h3_gpu_tensor *strengths, h3_gpu_tensor *changed, uint32_t rows, uint32_t row_width); /* gpu.h:841 */
int h3_gpu_video_graph_abort(h3_gpu *gpu); /* gpu.h:282 */
int h3_gpu_video_graph_begin(h3_gpu *gpu); /* gpu.h:280 */
int h3_gpu_video_graph_end(h3_gpu *gpu); /* gpu.h:281 */
int h3_gpu_video_linear(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t rows, uint32_t k, uint32_t n); /* gpu.h:283 */
int h3_gpu_video_qkv(h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key, h3_gpu_tensor *value, const h3_gpu_tensor *qkv, const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin, uint32_t sequence, uint32_t heads, uint32_t head_dim, uint32_t rope_half, float epsilon); /* gpu.h:392 */
int h3_gpu_video_sdpa(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *q, const h3_gpu_tensor *k, const h3_gpu_tensor *v, uint32_t rows, uint32_t heads, uint32_t dim, float scale); /* gpu.h:286 */
int h3_gpu_video_unpack(h3_gpu *gpu, const h3_gpu_tensor *projected, float *rgb, int latent_h, int latent_w, int output_frames, int first_frame, int frames); /* gpu.h:290 */
int h3_gpu_video_vae_configure(h3_gpu *gpu, int reserved); /* gpu.h:277 */
int h3_gpu_adaptive_probe(h3_gpu *gpu, h3_gpu_tensor *probe, const h3_gpu_tensor *output, const h3_gpu_tensor *anchor, h3_gpu_tensor *scratch, unsigned rows, unsigned columns, unsigned video_start, unsigned video_rows, unsigned audio_start, unsigned audio_rows, int ready, float *scores); /* gpu.h:62 */
int h3_gpu_adaptive_continuation_probe(h3_gpu *gpu, h3_gpu_tensor *probe, const h3_gpu_tensor *output, const h3_gpu_tensor *anchor, h3_gpu_tensor *scratch, unsigned columns, const h3_adaptive_regions *regions, int ready, float *scores); /* gpu.h:59 */
int h3_gpu_sglang_audio_average(h3_gpu *gpu, h3_gpu_tensor *sum, const h3_gpu_tensor *last, uint32_t count); /* gpu.h:152 */
void h3_gpu_sglang_audio_decoder(h3_gpu *gpu); /* gpu.h:149 */
void h3_gpu_sglang_audio_encoder(h3_gpu *gpu); /* gpu.h:150 */
int h3_gpu_sglang_batch_groups(h3_gpu *gpu, const uint32_t *counts, size_t count); /* gpu.h:169 */
int h3_gpu_sglang_head_f32(h3_gpu *gpu, h3_gpu_tensor *out, const h3_gpu_tensor *in, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t rows, uint32_t k, uint32_t n, uint32_t packed_rows); /* gpu.h:177 */
int h3_gpu_sglang_posterior(h3_gpu *gpu, const float *moments, const float *epsilon, float *sample, size_t count); /* gpu.h:158 */
int h3_gpu_sglang_preload_weight(h3_gpu *gpu, const char *path, uint64_t offset, size_t elements); /* gpu.h:156 */
int h3_gpu_sglang_rope_trig(h3_gpu *gpu, h3_gpu_tensor *cosine, h3_gpu_tensor *sine, const h3_gpu_tensor *angles, uint32_t count); /* gpu.h:175 */
int h3_gpu_sglang_stitch_begin(h3_gpu *gpu, int tile_h, int tile_w, int count_y, int count_x, const int *starts_y, const int *starts_x, int first_frame, int frames); /* gpu.h:296 */
int h3_gpu_sglang_stitch_read(h3_gpu *gpu, float *rgb); /* gpu.h:300 */
int h3_gpu_sglang_stitch_tile(h3_gpu *gpu, const h3_gpu_tensor *projected, int tile); /* gpu.h:299 */
void h3_gpu_sglang_text_encoder(h3_gpu *gpu); /* gpu.h:148 */
int h3_gpu_sglang_time_features(h3_gpu *gpu, h3_gpu_tensor *out, const h3_gpu_tensor *times, uint32_t rows); /* gpu.h:174 */
int h3_gpu_sglang_vae_enabled(const h3_gpu *gpu); /* gpu.h:157 */
int h3_gpu_sglang_vae_rope(h3_gpu *gpu, h3_gpu_tensor *cosine, h3_gpu_tensor *sine, uint32_t time, uint32_t height, uint32_t width, uint32_t rows); /* gpu.h:165 */
h3_gpu_tensor *h3_gpu_sglang_vae_weight(h3_gpu *gpu, const h3_gpu_tensor *weight); /* gpu.h:164 */
void h3_gpu_sglang_video_encoder(h3_gpu *gpu); /* gpu.h:151 */
int h3_gpu_sglang_vision_groups(h3_gpu *gpu, const uint32_t *counts, size_t count); /* gpu.h:170 */
int h3_gpu_sglang_vision_patch(h3_gpu *gpu, h3_gpu_tensor *out, const h3_gpu_tensor *in, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t rows, uint32_t k, uint32_t n); /* gpu.h:162 */
int h3_gpu_sglang_vision_prepare(h3_gpu *gpu, h3_gpu_tensor *position, const h3_gpu_tensor *table, h3_gpu_tensor *cosine, h3_gpu_tensor *sine, uint32_t height, uint32_t width); /* gpu.h:160 */
int h3_gpu_sglang_vision_prepare_range(h3_gpu *gpu, h3_gpu_tensor *position, const h3_gpu_tensor *table, h3_gpu_tensor *cosine, h3_gpu_tensor *sine, uint32_t height, uint32_t width, uint32_t offset); /* gpu.h:171 */

#ifdef __cplusplus
}
#endif
#endif
