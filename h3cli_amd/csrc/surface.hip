// The remainder of the reference operator surface (src/gpu.h) that the
// reference's tests/test_gpu_contract.c:152-181 requires a backend to link:
// context queries, weight planning, profiling marks, the SOL layout hook, and
// the ops outside the DiT denoise path, which fail with an error as the
// reference's CUDA backend does for Metal-only ops (src/cuda/gpu_cuda.cu:1358-1532).
#include "common.h"
#include "internal.h"
#include "subblock.h"
#include "sol.h"
#include "../../include/h3_gpu_surface.h"
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstring>

static int unsupported(h3_gpu *g, const char *what) { return g ? h3_set_error(g, "%s", what) : 0; }

static double wall_seconds() {
    using namespace std::chrono;
    return duration<double>(steady_clock::now().time_since_epoch()).count();
}

// ---- context queries (src/cuda/gpu_cuda.cu:530-537, 641)
extern "C" int h3_gpu_is_m5(const h3_gpu *g) { (void)g; return 0; }
extern "C" int h3_gpu_has_nax_mlp(const h3_gpu *g) { (void)g; return 0; }
extern "C" int h3_gpu_has_int8_mlp(const h3_gpu *g) { (void)g; return 0; }
extern "C" int h3_gpu_prefers_device_sampler(const h3_gpu *g, int continuation) { (void)continuation; return g != nullptr; }
// Streaming is retried after a failed resident allocation in automatic weight mode.
extern "C" int h3_gpu_should_retry_streaming(const h3_gpu *g) {
    if (!g || !g->allocation_failed) return 0;
    h3_weight_options o;
    return h3_weight_options_read(&o, 0, nullptr, 0) && o.mode == H3_WEIGHTS_AUTO;
}
// No host-side weight cache is kept: streamed weights live in caller tensors.
extern "C" int h3_gpu_release_weight_cache(h3_gpu *g) { return g != nullptr; }

// ---- weight planning (src/cuda/gpu_cuda.cu:538-590)
static uint64_t reserve_bytes(size_t total) { return std::max<uint64_t>(1ull << 30, total / 10); }

static int device_memory(h3_gpu *g, size_t *available, size_t *total, const char *what) {
    return h3_hip_check(g, hipMemGetInfo(available, total), what);
}

// Packed-weight plan: 0 = resident, 1 = stream, -1 = error.
extern "C" int h3_gpu_plan_weights(h3_gpu *g, uint64_t weights, uint64_t activations) {
    if (!g) return -1;
    h3_weight_options o;
    if (!h3_weight_options_read(&o, 0, g->error, sizeof(g->error))) return -1;
    size_t available, total;
    if (!device_memory(g, &available, &total, "weight planner")) return -1;
    uint64_t free_bytes = available;
    if (o.capacity_limit) free_bytes = std::min<uint64_t>(free_bytes, o.capacity_limit > g->stats.live_bytes ? o.capacity_limit - g->stats.live_bytes : 0);
    const uint64_t reserve = reserve_bytes(total);
    if (activations > free_bytes || reserve > free_bytes - activations) {
        h3_set_error(g, "insufficient HIP capacity for streamed activations/reserve");
        return -1;
    }
    bool fit = weights <= free_bytes - activations - reserve;
    if (o.mode == H3_WEIGHTS_RESIDENT && !fit) {
        h3_set_error(g, "resident weights need %.2f GiB plus %.2f GiB activations/reserve; %.2f GiB free",
                     weights / 1073741824., (activations + reserve) / 1073741824., free_bytes / 1073741824.);
        return -1;
    }
    if (o.mode == H3_WEIGHTS_STREAM) fit = false;
    return fit ? 0 : 1;
}

extern "C" int h3_gpu_plan_bf16_weights(h3_gpu *g, uint64_t active_mask, uint64_t block_bytes, uint64_t future_bytes,
                                        int force_stream, int retry_cap, h3_weight_plan *plan) {
    if (!g || !plan) return 0;
    h3_weight_options o;
    if (!h3_weight_options_read(&o, 0, g->error, sizeof(g->error))) return 0;
    if (force_stream && o.mode == H3_WEIGHTS_RESIDENT)
        return h3_set_error(g, "--ssd-streaming conflicts with CUDA resident weight mode");
    if (force_stream) o.mode = H3_WEIGHTS_STREAM;
    if (retry_cap >= 0 && (o.max_resident < 0 || retry_cap < o.max_resident)) o.max_resident = retry_cap;
    size_t available, total;
    if (!device_memory(g, &available, &total, "BF16 weight planner")) return 0;
    int ok = h3_weight_plan_build(plan, o, active_mask, block_bytes, available, g->stats.live_bytes, future_bytes,
                                  reserve_bytes(total), g->error, sizeof(g->error));
    if (ok) {
        g->stats.resident_weight_bytes = plan->resident_bytes;
        g->stats.stream_slot_bytes = plan->slot_bytes;
        g->stats.resident_blocks = plan->resident_count;
        g->stats.active_weight_blocks = plan->active_count;
        g->stats.resident_block_mask = plan->resident_mask;
    }
    return ok;
}

// A context can be kept across requests when the weight options have not
// changed and the device still has the planner's reserve free.
extern "C" int h3_gpu_weight_plan_compatible(h3_gpu *g, int force_stream) {
    if (!g) return 0;
    h3_weight_options now;
    if (!h3_weight_options_read(&now, force_stream, nullptr, 0)) return 0;
    if (g->stats.active_weight_blocks && g->stats.resident_blocks < g->stats.active_weight_blocks &&
        now.mode == H3_WEIGHTS_AUTO)
        return 0;  // a partial automatic plan is recomputed per request
    size_t available, total;
    return hipMemGetInfo(&available, &total) == hipSuccess && available >= reserve_bytes(total);
}

// ---- SOL / SubBlock layout (gpu.h:66): bound for the SubBlock router in
// attention mode 4 and for SOL routing in mode 3; other modes check only that
// the tables are present.
extern "C" int h3_gpu_dit_sol_layout(h3_gpu *g, const h3_sol_layout *layout) {
    if (!g || !layout) return 0;
    if (!layout->sequence || !layout->query_blocks || !layout->key_blocks || !layout->query || !layout->key)
        return h3_set_error(g, "SOL layout: empty sequence or block tables");
    // SubBlock and SOL modes bind the layout for their routers (reference
    // gpu_cuda.cu:1572-1591); other modes only validate it.
    if (h3_attention_mode(g) == 4) return h3_subblock_bind(g, h3_attention_router(g), layout);
    if (h3_attention_mode(g) == 3) {
        h3_sol_router *r = h3_attention_sol(g);
        return h3_sol_bind(g, r, layout, r->options);
    }
    return 1;
}

// ---- Qwen GQA scale mode (src/cuda/gpu_cuda.cu:1235-1243): host text parse.
extern "C" int h3_qwen_gqa_scale_parse(const char *value, h3_qwen_gqa_scale_mode *mode, char *error, size_t error_size) {
    if (!mode) return 0;
    if (!value || !*value || !strcmp(value, "reference")) *mode = H3_QWEN_GQA_REFERENCE;
    else if (!strcmp(value, "scaled-q")) *mode = H3_QWEN_GQA_SCALED_Q;
    else if (!strcmp(value, "legacy")) *mode = H3_QWEN_GQA_LEGACY;
    else {
        if (error && error_size) snprintf(error, error_size, "invalid H3_QWEN_GQA_SCALE_MODE: %s", value);
        return 0;
    }
    return 1;
}
extern "C" const char *h3_qwen_gqa_scale_name(h3_qwen_gqa_scale_mode mode) {
    return mode == H3_QWEN_GQA_SCALED_Q ? "scaled-q" : mode == H3_QWEN_GQA_LEGACY ? "legacy" : "reference";
}

// ---- profiling marks (gpu.h:271-272): one stderr summary line under H3_PROFILE.
extern "C" void h3_gpu_profile_set_label(h3_gpu *g, const char *label) {
    if (g && label) snprintf(g->label, sizeof(g->label), "%s", label);
}
extern "C" void h3_gpu_profile_mark(h3_gpu *g, const char *phase) {
    if (!g || !getenv("H3_PROFILE")) return;
    const h3_gpu_stats &s = g->stats;
    fprintf(stderr,
            "h3hip: profile %s / %s: wall %.3fs, GEMM %llu attention %llu, H2D %.3f GiB streamed %.3f GiB, "
            "GEMM %.6fs attention %.6fs, bounce stalls %llu, subblock calls %llu bypass %llu\n",
            g->label, phase ? phase : "", wall_seconds() - g->created, (unsigned long long)s.linear_dispatches,
            (unsigned long long)s.attention_dispatches, s.h2d_bytes / 1073741824., s.streamed_bytes / 1073741824.,
            s.linear_seconds, s.attention_seconds, (unsigned long long)s.stream_stalls,
            (unsigned long long)s.subblock_calls, (unsigned long long)s.subblock_bypass);
}

// ---- outside the DiT denoise path
extern "C" int h3_gpu_gqa_causal_limits(h3_gpu *gpu, h3_gqa_limits *limits) { (void)limits; return unsupported(gpu, "h3_gpu_gqa_causal_limits: unsupported on the HIP backend"); }
extern "C" size_t h3_gpu_gqa_causal_max_sequence(h3_gpu *gpu) { unsupported(gpu, "h3_gpu_gqa_causal_max_sequence: unsupported on the HIP backend"); return 0; }
extern "C" int h3_gpu_gqa_causal_preflight(h3_gpu *gpu, size_t sequence, char *error, size_t error_size) { (void)sequence; (void)error; (void)error_size; return unsupported(gpu, "h3_gpu_gqa_causal_preflight: unsupported on the HIP backend"); }
extern "C" int h3_gpu_linear_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t rows, uint32_t input_dim, uint32_t output_dim) { (void)output; (void)input; (void)weight; (void)bias; (void)rows; (void)input_dim; (void)output_dim; return unsupported(gpu, "h3_gpu_linear_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_silu_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, uint32_t elements) { (void)output; (void)input; (void)elements; return unsupported(gpu, "h3_gpu_silu_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_rms_norm_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, uint32_t rows, uint32_t width, float epsilon) { (void)output; (void)input; (void)weight; (void)rows; (void)width; (void)epsilon; return unsupported(gpu, "h3_gpu_rms_norm_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_adaln_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *norm_weight, const h3_gpu_tensor *modulation, const h3_gpu_tensor *row_map, uint32_t rows, uint32_t width, uint32_t slots, uint32_t shift_slot, uint32_t scale_slot, float epsilon) { (void)output; (void)input; (void)norm_weight; (void)modulation; (void)row_map; (void)rows; (void)width; (void)slots; (void)shift_slot; (void)scale_slot; (void)epsilon; return unsupported(gpu, "h3_gpu_adaln_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_gate_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *residual, const h3_gpu_tensor *branch, const h3_gpu_tensor *modulation, const h3_gpu_tensor *row_map, uint32_t rows, uint32_t width, uint32_t slots, uint32_t gate_slot) { (void)output; (void)residual; (void)branch; (void)modulation; (void)row_map; (void)rows; (void)width; (void)slots; (void)gate_slot; return unsupported(gpu, "h3_gpu_gate_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_qkv_rope_f32(h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key, h3_gpu_tensor *value, const h3_gpu_tensor *qkv, const h3_gpu_tensor *q_norm, const h3_gpu_tensor *k_norm, const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin, uint32_t sequence, uint32_t heads, uint32_t head_dim, uint32_t rope_half, float epsilon) { (void)query; (void)key; (void)value; (void)qkv; (void)q_norm; (void)k_norm; (void)rope_cos; (void)rope_sin; (void)sequence; (void)heads; (void)head_dim; (void)rope_half; (void)epsilon; return unsupported(gpu, "h3_gpu_qkv_rope_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_sdpa_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *query, const h3_gpu_tensor *key, const h3_gpu_tensor *value, uint32_t sequence, uint32_t heads, uint32_t head_dim, float scale) { (void)output; (void)query; (void)key; (void)value; (void)sequence; (void)heads; (void)head_dim; (void)scale; return unsupported(gpu, "h3_gpu_sdpa_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_swiglu_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *fused, uint32_t rows, uint32_t width) { (void)output; (void)fused; (void)rows; (void)width; return unsupported(gpu, "h3_gpu_swiglu_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_scale_add_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *residual, const h3_gpu_tensor *branch, const h3_gpu_tensor *scale, uint32_t rows, uint32_t width) { (void)output; (void)residual; (void)branch; (void)scale; (void)rows; (void)width; return unsupported(gpu, "h3_gpu_scale_add_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_layer_norm_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t rows, uint32_t width, float epsilon) { (void)output; (void)input; (void)weight; (void)bias; (void)rows; (void)width; (void)epsilon; return unsupported(gpu, "h3_gpu_layer_norm_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_video_qkv_rope_f32(h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key, h3_gpu_tensor *value, const h3_gpu_tensor *qkv, const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin, uint32_t sequence, uint32_t heads, uint32_t head_dim, uint32_t rope_half, float epsilon) { (void)query; (void)key; (void)value; (void)qkv; (void)rope_cos; (void)rope_sin; (void)sequence; (void)heads; (void)head_dim; (void)rope_half; (void)epsilon; return unsupported(gpu, "h3_gpu_video_qkv_rope_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_conv1d_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t batch, uint32_t length, uint32_t input_channels, uint32_t output_channels, uint32_t kernel, uint32_t padding, uint32_t dilation) { (void)output; (void)input; (void)weight; (void)bias; (void)batch; (void)length; (void)input_channels; (void)output_channels; (void)kernel; (void)padding; (void)dilation; return unsupported(gpu, "h3_gpu_conv1d_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_conv1d_stride_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t batch, uint32_t length, uint32_t input_channels, uint32_t output_channels, uint32_t kernel, uint32_t stride, uint32_t padding, uint32_t dilation) { (void)output; (void)input; (void)weight; (void)bias; (void)batch; (void)length; (void)input_channels; (void)output_channels; (void)kernel; (void)stride; (void)padding; (void)dilation; return unsupported(gpu, "h3_gpu_conv1d_stride_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_conv_transpose1d_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t batch, uint32_t length, uint32_t input_channels, uint32_t output_channels, uint32_t kernel, uint32_t stride, uint32_t padding) { (void)output; (void)input; (void)weight; (void)bias; (void)batch; (void)length; (void)input_channels; (void)output_channels; (void)kernel; (void)stride; (void)padding; return unsupported(gpu, "h3_gpu_conv_transpose1d_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_weight_norm_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *vector, const h3_gpu_tensor *magnitude, uint32_t outer, uint32_t inner) { (void)output; (void)vector; (void)magnitude; (void)outer; (void)inner; return unsupported(gpu, "h3_gpu_weight_norm_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_add_scaled_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *left, const h3_gpu_tensor *right, float left_scale, float right_scale, uint32_t elements) { (void)output; (void)left; (void)right; (void)left_scale; (void)right_scale; (void)elements; return unsupported(gpu, "h3_gpu_add_scaled_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_alias_free_snake_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *alpha_log, const h3_gpu_tensor *beta_log, const h3_gpu_tensor *upsample_filter, const h3_gpu_tensor *downsample_filter, uint32_t batch, uint32_t length, uint32_t channels) { (void)output; (void)input; (void)alpha_log; (void)beta_log; (void)upsample_filter; (void)downsample_filter; (void)batch; (void)length; (void)channels; return unsupported(gpu, "h3_gpu_alias_free_snake_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_snake1d_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *alpha, uint32_t batch, uint32_t length, uint32_t channels) { (void)output; (void)input; (void)alpha; (void)batch; (void)length; (void)channels; return unsupported(gpu, "h3_gpu_snake1d_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_audio_qkv_split_f32(h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key, h3_gpu_tensor *value, const h3_gpu_tensor *qkv, const h3_gpu_tensor *q_bias, const h3_gpu_tensor *k_bias, const h3_gpu_tensor *v_bias, uint32_t batch, uint32_t length, uint32_t heads, uint32_t head_dim) { (void)query; (void)key; (void)value; (void)qkv; (void)q_bias; (void)k_bias; (void)v_bias; (void)batch; (void)length; (void)heads; (void)head_dim; return unsupported(gpu, "h3_gpu_audio_qkv_split_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_sdpa_causal_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *query, const h3_gpu_tensor *key, const h3_gpu_tensor *value, uint32_t batch, uint32_t sequence, uint32_t heads, uint32_t head_dim, float scale) { (void)output; (void)query; (void)key; (void)value; (void)batch; (void)sequence; (void)heads; (void)head_dim; (void)scale; return unsupported(gpu, "h3_gpu_sdpa_causal_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_audio_attention_pool_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *attended, uint32_t batch, uint32_t length, uint32_t heads, uint32_t head_dim, uint32_t output_dim) { (void)output; (void)attended; (void)batch; (void)length; (void)heads; (void)head_dim; (void)output_dim; return unsupported(gpu, "h3_gpu_audio_attention_pool_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_geglu_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *gate, const h3_gpu_tensor *linear, uint32_t elements) { (void)output; (void)gate; (void)linear; (void)elements; return unsupported(gpu, "h3_gpu_geglu_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_clip_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, uint32_t elements, float minimum, float maximum) { (void)output; (void)input; (void)elements; (void)minimum; (void)maximum; return unsupported(gpu, "h3_gpu_clip_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_vae_encoder_pad_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, uint32_t batch, uint32_t depth, uint32_t height, uint32_t width, uint32_t channels, uint32_t depth_front, uint32_t height_before, uint32_t height_after, uint32_t width_before, uint32_t width_after) { (void)output; (void)input; (void)batch; (void)depth; (void)height; (void)width; (void)channels; (void)depth_front; (void)height_before; (void)height_after; (void)width_before; (void)width_after; return unsupported(gpu, "h3_gpu_vae_encoder_pad_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_conv3d_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t batch, uint32_t depth, uint32_t height, uint32_t width, uint32_t input_channels, uint32_t output_channels, uint32_t kernel_depth, uint32_t kernel_height, uint32_t kernel_width, uint32_t stride_depth, uint32_t stride_height, uint32_t stride_width) { (void)output; (void)input; (void)weight; (void)bias; (void)batch; (void)depth; (void)height; (void)width; (void)input_channels; (void)output_channels; (void)kernel_depth; (void)kernel_height; (void)kernel_width; (void)stride_depth; (void)stride_height; (void)stride_width; return unsupported(gpu, "h3_gpu_conv3d_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_vae_encoder_group_norm_silu_f32(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t batch, uint32_t depth, uint32_t height, uint32_t width, uint32_t channels, uint32_t groups, float epsilon) { (void)output; (void)input; (void)weight; (void)bias; (void)batch; (void)depth; (void)height; (void)width; (void)channels; (void)groups; (void)epsilon; return unsupported(gpu, "h3_gpu_vae_encoder_group_norm_silu_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_mlp_nax_bf16(h3_gpu *gpu, h3_gpu_tensor *output, h3_gpu_tensor *activated, const h3_gpu_tensor *input, const h3_gpu_tensor *fc1_weight, const h3_gpu_tensor *fc2_weight, uint32_t rows, uint32_t input_dim, uint32_t hidden_dim, uint32_t output_dim) { (void)output; (void)activated; (void)input; (void)fc1_weight; (void)fc2_weight; (void)rows; (void)input_dim; (void)hidden_dim; (void)output_dim; return unsupported(gpu, "h3_gpu_mlp_nax_bf16: unsupported on the HIP backend"); }
extern "C" int h3_gpu_quantize_weight_int8(h3_gpu *gpu, h3_gpu_tensor *output, h3_gpu_tensor *scales, const h3_gpu_tensor *input, uint32_t rows, uint32_t columns) { (void)output; (void)scales; (void)input; (void)rows; (void)columns; return unsupported(gpu, "h3_gpu_quantize_weight_int8: unsupported on the HIP backend"); }
extern "C" int h3_gpu_linear_int8_bf16(h3_gpu *gpu, h3_gpu_tensor *output, h3_gpu_tensor *quantized_input, h3_gpu_tensor *input_scales, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *weight_scales, uint32_t rows, uint32_t input_dim, uint32_t output_dim, int use_slower_uncached_int8_scales) { (void)output; (void)quantized_input; (void)input_scales; (void)input; (void)weight; (void)weight_scales; (void)rows; (void)input_dim; (void)output_dim; (void)use_slower_uncached_int8_scales; return unsupported(gpu, "h3_gpu_linear_int8_bf16: unsupported on the HIP backend"); }
extern "C" int h3_gpu_linear_int8_head_major_bf16(h3_gpu *gpu, h3_gpu_tensor *output, h3_gpu_tensor *quantized_input, h3_gpu_tensor *input_scales, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *weight_scales, uint32_t rows, uint32_t heads, uint32_t head_dim, uint32_t output_dim) { (void)output; (void)quantized_input; (void)input_scales; (void)input; (void)weight; (void)weight_scales; (void)rows; (void)heads; (void)head_dim; (void)output_dim; return unsupported(gpu, "h3_gpu_linear_int8_head_major_bf16: unsupported on the HIP backend"); }
extern "C" int h3_gpu_mlp_int8_bf16(h3_gpu *gpu, h3_gpu_tensor *output, h3_gpu_tensor *activated, h3_gpu_tensor *quantized_activation, h3_gpu_tensor *activation_scales, const h3_gpu_tensor *input, const h3_gpu_tensor *fc1_weight, const h3_gpu_tensor *fc1_scales, const h3_gpu_tensor *fc2_weight, const h3_gpu_tensor *fc2_scales, const h3_gpu_tensor *fc1_bf16, const h3_gpu_tensor *fc2_bf16, uint32_t rows, uint32_t input_dim, uint32_t hidden_dim, uint32_t output_dim, int use_slower_grouped_quantizer, int use_slower_dynamic_fc1_k, int use_int8_row_fc2, int input_is_quantized) { (void)output; (void)activated; (void)quantized_activation; (void)activation_scales; (void)input; (void)fc1_weight; (void)fc1_scales; (void)fc2_weight; (void)fc2_scales; (void)fc1_bf16; (void)fc2_bf16; (void)rows; (void)input_dim; (void)hidden_dim; (void)output_dim; (void)use_slower_grouped_quantizer; (void)use_slower_dynamic_fc1_k; (void)use_int8_row_fc2; (void)input_is_quantized; return unsupported(gpu, "h3_gpu_mlp_int8_bf16: unsupported on the HIP backend"); }
extern "C" int h3_gpu_layer_norm_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t rows, uint32_t width, float epsilon) { (void)output; (void)input; (void)weight; (void)bias; (void)rows; (void)width; (void)epsilon; return unsupported(gpu, "h3_gpu_layer_norm_bf16: unsupported on the HIP backend"); }
extern "C" int h3_gpu_vision_qkv_rope_bf16(h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key, h3_gpu_tensor *value, const h3_gpu_tensor *qkv, const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin, uint32_t sequence, uint32_t heads, uint32_t head_dim, uint32_t rope_half) { (void)query; (void)key; (void)value; (void)qkv; (void)rope_cos; (void)rope_sin; (void)sequence; (void)heads; (void)head_dim; (void)rope_half; return unsupported(gpu, "h3_gpu_vision_qkv_rope_bf16: unsupported on the HIP backend"); }
extern "C" int h3_gpu_adaln_linear_bf16(h3_gpu *gpu, h3_gpu_tensor *output, h3_gpu_tensor *inverse, const h3_gpu_tensor *input, size_t input_offset, const h3_gpu_tensor *norm_weight, const h3_gpu_tensor *modulation, const h3_gpu_tensor *row_map, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t rows, uint32_t width, uint32_t output_dim, uint32_t slots, uint32_t shift_slot, uint32_t scale_slot, float epsilon) { (void)output; (void)inverse; (void)input; (void)input_offset; (void)norm_weight; (void)modulation; (void)row_map; (void)weight; (void)bias; (void)rows; (void)width; (void)output_dim; (void)slots; (void)shift_slot; (void)scale_slot; (void)epsilon; return unsupported(gpu, "h3_gpu_adaln_linear_bf16: unsupported on the HIP backend"); }
extern "C" int h3_gpu_gate_adaln_quantize_int8(h3_gpu *gpu, h3_gpu_tensor *gated_residual, h3_gpu_tensor *quantized_output, h3_gpu_tensor *quantized_scales, const h3_gpu_tensor *residual, const h3_gpu_tensor *branch, const h3_gpu_tensor *norm_weight, const h3_gpu_tensor *gate_modulation, const h3_gpu_tensor *norm_modulation, const h3_gpu_tensor *row_map, uint32_t rows, uint32_t padded_rows, uint32_t width, uint32_t slots, uint32_t gate_slot, uint32_t shift_slot, uint32_t scale_slot, float epsilon) { (void)gated_residual; (void)quantized_output; (void)quantized_scales; (void)residual; (void)branch; (void)norm_weight; (void)gate_modulation; (void)norm_modulation; (void)row_map; (void)rows; (void)padded_rows; (void)width; (void)slots; (void)gate_slot; (void)shift_slot; (void)scale_slot; (void)epsilon; return unsupported(gpu, "h3_gpu_gate_adaln_quantize_int8: unsupported on the HIP backend"); }
extern "C" int h3_gpu_grouped_qkv_linear_rope_int8(h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key, h3_gpu_tensor *value, h3_gpu_tensor *quantized_input, h3_gpu_tensor *input_scales, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *weight_scales, const h3_gpu_tensor *q_norm, const h3_gpu_tensor *k_norm, const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin, uint32_t rows, uint32_t input_dim, uint32_t heads, uint32_t head_dim, uint32_t rope_half, float epsilon, int input_is_quantized, int use_slower_unfused_qkv_rope, int use_slower_scalar_qkv_rms, int use_slower_uncached_int8_scales) { (void)query; (void)key; (void)value; (void)quantized_input; (void)input_scales; (void)input; (void)weight; (void)weight_scales; (void)q_norm; (void)k_norm; (void)rope_cos; (void)rope_sin; (void)rows; (void)input_dim; (void)heads; (void)head_dim; (void)rope_half; (void)epsilon; (void)input_is_quantized; (void)use_slower_unfused_qkv_rope; (void)use_slower_scalar_qkv_rms; (void)use_slower_uncached_int8_scales; return unsupported(gpu, "h3_gpu_grouped_qkv_linear_rope_int8: unsupported on the HIP backend"); }
extern "C" int h3_gpu_embedding_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *weight, const h3_gpu_tensor *token_ids, uint32_t tokens, uint32_t vocab_size, uint32_t width) { (void)output; (void)weight; (void)token_ids; (void)tokens; (void)vocab_size; (void)width; return unsupported(gpu, "h3_gpu_embedding_bf16: unsupported on the HIP backend"); }
extern "C" int h3_gpu_text_qk_rope_bf16(h3_gpu *gpu, h3_gpu_tensor *query_output, h3_gpu_tensor *key_output, const h3_gpu_tensor *query_input, const h3_gpu_tensor *key_input, const h3_gpu_tensor *q_norm, const h3_gpu_tensor *k_norm, const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin, uint32_t sequence, uint32_t query_heads, uint32_t kv_heads, uint32_t head_dim, float epsilon) { (void)query_output; (void)key_output; (void)query_input; (void)key_input; (void)q_norm; (void)k_norm; (void)rope_cos; (void)rope_sin; (void)sequence; (void)query_heads; (void)kv_heads; (void)head_dim; (void)epsilon; return unsupported(gpu, "h3_gpu_text_qk_rope_bf16: unsupported on the HIP backend"); }
extern "C" int h3_gpu_rope_text_bf16(h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key, const h3_gpu_tensor *rope_cos_f32, const h3_gpu_tensor *rope_sin_f32, uint32_t sequence, uint32_t query_heads, uint32_t kv_heads, uint32_t head_dim) { (void)query; (void)key; (void)rope_cos_f32; (void)rope_sin_f32; (void)sequence; (void)query_heads; (void)kv_heads; (void)head_dim; return unsupported(gpu, "h3_gpu_rope_text_bf16: unsupported on the HIP backend"); }
extern "C" int h3_gpu_gqa_causal_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *query, const h3_gpu_tensor *key, const h3_gpu_tensor *value, uint32_t sequence, uint32_t query_heads, uint32_t kv_heads, uint32_t head_dim, float scale) { (void)output; (void)query; (void)key; (void)value; (void)sequence; (void)query_heads; (void)kv_heads; (void)head_dim; (void)scale; return unsupported(gpu, "h3_gpu_gqa_causal_bf16: unsupported on the HIP backend"); }
extern "C" int h3_gpu_token_pool_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, size_t input_offset, h3_gpu_tensor *original, size_t original_offset, h3_gpu_tensor *baseline, size_t baseline_offset, const h3_gpu_tensor *baseline_indices, const h3_gpu_tensor *pairs, uint32_t input_rows, uint32_t rows, uint32_t baseline_rows, uint32_t width) { (void)output; (void)input; (void)input_offset; (void)original; (void)original_offset; (void)baseline; (void)baseline_offset; (void)baseline_indices; (void)pairs; (void)input_rows; (void)rows; (void)baseline_rows; (void)width; return unsupported(gpu, "h3_gpu_token_pool_bf16: unsupported on the HIP backend"); }
extern "C" int h3_gpu_token_pool_adaln_bf16(h3_gpu *gpu, h3_gpu_tensor *residual, h3_gpu_tensor *output, const h3_gpu_tensor *input, size_t input_offset, h3_gpu_tensor *original, size_t original_offset, h3_gpu_tensor *baseline, size_t baseline_offset, const h3_gpu_tensor *baseline_indices, const h3_gpu_tensor *pairs, const h3_gpu_tensor *norm_weight, const h3_gpu_tensor *modulation, const h3_gpu_tensor *row_map, uint32_t input_rows, uint32_t rows, uint32_t baseline_rows, uint32_t width, uint32_t slots, uint32_t shift_slot, uint32_t scale_slot, float epsilon) { (void)residual; (void)output; (void)input; (void)input_offset; (void)original; (void)original_offset; (void)baseline; (void)baseline_offset; (void)baseline_indices; (void)pairs; (void)norm_weight; (void)modulation; (void)row_map; (void)input_rows; (void)rows; (void)baseline_rows; (void)width; (void)slots; (void)shift_slot; (void)scale_slot; (void)epsilon; return unsupported(gpu, "h3_gpu_token_pool_adaln_bf16: unsupported on the HIP backend"); }
extern "C" int h3_gpu_token_expand_delta_bf16(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *original, size_t original_offset, const h3_gpu_tensor *reduced, const h3_gpu_tensor *baseline, size_t baseline_offset, const h3_gpu_tensor *baseline_indices, const h3_gpu_tensor *parents, uint32_t rows, uint32_t reduced_rows, uint32_t baseline_rows, uint32_t width, uint32_t exact_prefix_rows, float update_scale) { (void)output; (void)original; (void)original_offset; (void)reduced; (void)baseline; (void)baseline_offset; (void)baseline_indices; (void)parents; (void)rows; (void)reduced_rows; (void)baseline_rows; (void)width; (void)exact_prefix_rows; (void)update_scale; return unsupported(gpu, "h3_gpu_token_expand_delta_bf16: unsupported on the HIP backend"); }
extern "C" int h3_gpu_token_expand_adaln_bf16(h3_gpu *gpu, h3_gpu_tensor *residual, h3_gpu_tensor *output, const h3_gpu_tensor *original, size_t original_offset, const h3_gpu_tensor *reduced, const h3_gpu_tensor *baseline, size_t baseline_offset, const h3_gpu_tensor *baseline_indices, const h3_gpu_tensor *parents, const h3_gpu_tensor *norm_weight, const h3_gpu_tensor *modulation, const h3_gpu_tensor *row_map, uint32_t rows, uint32_t reduced_rows, uint32_t baseline_rows, uint32_t width, uint32_t exact_prefix_rows, float update_scale, uint32_t slots, uint32_t shift_slot, uint32_t scale_slot, float epsilon) { (void)residual; (void)output; (void)original; (void)original_offset; (void)reduced; (void)baseline; (void)baseline_offset; (void)baseline_indices; (void)parents; (void)norm_weight; (void)modulation; (void)row_map; (void)rows; (void)reduced_rows; (void)baseline_rows; (void)width; (void)exact_prefix_rows; (void)update_scale; (void)slots; (void)shift_slot; (void)scale_slot; (void)epsilon; return unsupported(gpu, "h3_gpu_token_expand_adaln_bf16: unsupported on the HIP backend"); }
extern "C" int h3_gpu_video_preview_bf16(h3_gpu *gpu, h3_gpu_tensor *scratch, const h3_gpu_tensor *sample, size_t sample_offset, const h3_gpu_tensor *last, const h3_gpu_tensor *previous, const h3_gpu_tensor *row_classes, const h3_gpu_tensor *strengths, uint32_t time, uint32_t height, uint32_t width, float sigma_next, float ratio) { (void)scratch; (void)sample; (void)sample_offset; (void)last; (void)previous; (void)row_classes; (void)strengths; (void)time; (void)height; (void)width; (void)sigma_next; (void)ratio; return unsupported(gpu, "h3_gpu_video_preview_bf16: unsupported on the HIP backend"); }
extern "C" int h3_gpu_video_preview_read(const h3_gpu_tensor *scratch, float *latent, size_t elements) { (void)scratch; (void)latent; (void)elements; return 0; }
extern "C" int h3_gpu_bridge_euler_bf16(h3_gpu *gpu, h3_gpu_tensor *sample, size_t sample_offset, const h3_gpu_tensor *last, const h3_gpu_tensor *previous, const h3_gpu_tensor *row_classes, const h3_gpu_tensor *strengths, uint32_t rows, uint32_t row_width, float delta, float ratio) { (void)sample; (void)sample_offset; (void)last; (void)previous; (void)row_classes; (void)strengths; (void)rows; (void)row_width; (void)delta; (void)ratio; return unsupported(gpu, "h3_gpu_bridge_euler_bf16: unsupported on the HIP backend"); }
extern "C" int h3_gpu_bridge_check_exact(h3_gpu *gpu, const h3_gpu_tensor *sample, size_t sample_offset, const h3_gpu_tensor *initial, const h3_gpu_tensor *row_classes, const h3_gpu_tensor *strengths, h3_gpu_tensor *changed, uint32_t rows, uint32_t row_width) { (void)sample; (void)sample_offset; (void)initial; (void)row_classes; (void)strengths; (void)changed; (void)rows; (void)row_width; return unsupported(gpu, "h3_gpu_bridge_check_exact: unsupported on the HIP backend"); }
extern "C" int h3_gpu_video_graph_abort(h3_gpu *gpu) { return unsupported(gpu, "h3_gpu_video_graph_abort: unsupported on the HIP backend"); }
extern "C" int h3_gpu_video_graph_begin(h3_gpu *gpu) { return unsupported(gpu, "h3_gpu_video_graph_begin: unsupported on the HIP backend"); }
extern "C" int h3_gpu_video_graph_end(h3_gpu *gpu) { return unsupported(gpu, "h3_gpu_video_graph_end: unsupported on the HIP backend"); }
extern "C" int h3_gpu_video_linear(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *input, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t rows, uint32_t k, uint32_t n) { (void)output; (void)input; (void)weight; (void)bias; (void)rows; (void)k; (void)n; return unsupported(gpu, "h3_gpu_video_linear: unsupported on the HIP backend"); }
extern "C" int h3_gpu_video_qkv(h3_gpu *gpu, h3_gpu_tensor *query, h3_gpu_tensor *key, h3_gpu_tensor *value, const h3_gpu_tensor *qkv, const h3_gpu_tensor *rope_cos, const h3_gpu_tensor *rope_sin, uint32_t sequence, uint32_t heads, uint32_t head_dim, uint32_t rope_half, float epsilon) { (void)query; (void)key; (void)value; (void)qkv; (void)rope_cos; (void)rope_sin; (void)sequence; (void)heads; (void)head_dim; (void)rope_half; (void)epsilon; return unsupported(gpu, "h3_gpu_video_qkv: unsupported on the HIP backend"); }
extern "C" int h3_gpu_video_sdpa(h3_gpu *gpu, h3_gpu_tensor *output, const h3_gpu_tensor *q, const h3_gpu_tensor *k, const h3_gpu_tensor *v, uint32_t rows, uint32_t heads, uint32_t dim, float scale) { (void)output; (void)q; (void)k; (void)v; (void)rows; (void)heads; (void)dim; (void)scale; return unsupported(gpu, "h3_gpu_video_sdpa: unsupported on the HIP backend"); }
extern "C" int h3_gpu_video_unpack(h3_gpu *gpu, const h3_gpu_tensor *projected, float *rgb, int latent_h, int latent_w, int output_frames, int first_frame, int frames) { (void)projected; (void)rgb; (void)latent_h; (void)latent_w; (void)output_frames; (void)first_frame; (void)frames; return unsupported(gpu, "h3_gpu_video_unpack: unsupported on the HIP backend"); }
extern "C" int h3_gpu_video_vae_configure(h3_gpu *gpu, int reserved) { (void)reserved; return unsupported(gpu, "h3_gpu_video_vae_configure: unsupported on the HIP backend"); }
extern "C" int h3_gpu_adaptive_probe(h3_gpu *gpu, h3_gpu_tensor *probe, const h3_gpu_tensor *output, const h3_gpu_tensor *anchor, h3_gpu_tensor *scratch, unsigned rows, unsigned columns, unsigned video_start, unsigned video_rows, unsigned audio_start, unsigned audio_rows, int ready, float *scores) { (void)probe; (void)output; (void)anchor; (void)scratch; (void)rows; (void)columns; (void)video_start; (void)video_rows; (void)audio_start; (void)audio_rows; (void)ready; (void)scores; return unsupported(gpu, "h3_gpu_adaptive_probe: unsupported on the HIP backend"); }
extern "C" int h3_gpu_adaptive_continuation_probe(h3_gpu *gpu, h3_gpu_tensor *probe, const h3_gpu_tensor *output, const h3_gpu_tensor *anchor, h3_gpu_tensor *scratch, unsigned columns, const h3_adaptive_regions *regions, int ready, float *scores) { (void)probe; (void)output; (void)anchor; (void)scratch; (void)columns; (void)regions; (void)ready; (void)scores; return unsupported(gpu, "h3_gpu_adaptive_continuation_probe: unsupported on the HIP backend"); }
extern "C" int h3_gpu_sglang_audio_average(h3_gpu *gpu, h3_gpu_tensor *sum, const h3_gpu_tensor *last, uint32_t count) { (void)sum; (void)last; (void)count; return unsupported(gpu, "h3_gpu_sglang_audio_average: unsupported on the HIP backend"); }
extern "C" void h3_gpu_sglang_audio_decoder(h3_gpu *gpu) {  }
extern "C" void h3_gpu_sglang_audio_encoder(h3_gpu *gpu) {  }
extern "C" int h3_gpu_sglang_batch_groups(h3_gpu *gpu, const uint32_t *counts, size_t count) { (void)counts; (void)count; return unsupported(gpu, "h3_gpu_sglang_batch_groups: unsupported on the HIP backend"); }
extern "C" int h3_gpu_sglang_head_f32(h3_gpu *gpu, h3_gpu_tensor *out, const h3_gpu_tensor *in, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t rows, uint32_t k, uint32_t n, uint32_t packed_rows) { (void)out; (void)in; (void)weight; (void)bias; (void)rows; (void)k; (void)n; (void)packed_rows; return unsupported(gpu, "h3_gpu_sglang_head_f32: unsupported on the HIP backend"); }
extern "C" int h3_gpu_sglang_posterior(h3_gpu *gpu, const float *moments, const float *epsilon, float *sample, size_t count) { (void)moments; (void)epsilon; (void)sample; (void)count; return unsupported(gpu, "h3_gpu_sglang_posterior: unsupported on the HIP backend"); }
extern "C" int h3_gpu_sglang_preload_weight(h3_gpu *gpu, const char *path, uint64_t offset, size_t elements) { (void)path; (void)offset; (void)elements; return unsupported(gpu, "h3_gpu_sglang_preload_weight: unsupported on the HIP backend"); }
extern "C" int h3_gpu_sglang_rope_trig(h3_gpu *gpu, h3_gpu_tensor *cosine, h3_gpu_tensor *sine, const h3_gpu_tensor *angles, uint32_t count) { (void)cosine; (void)sine; (void)angles; (void)count; return unsupported(gpu, "h3_gpu_sglang_rope_trig: unsupported on the HIP backend"); }
extern "C" int h3_gpu_sglang_stitch_begin(h3_gpu *gpu, int tile_h, int tile_w, int count_y, int count_x, const int *starts_y, const int *starts_x, int first_frame, int frames) { (void)tile_h; (void)tile_w; (void)count_y; (void)count_x; (void)starts_y; (void)starts_x; (void)first_frame; (void)frames; return unsupported(gpu, "h3_gpu_sglang_stitch_begin: unsupported on the HIP backend"); }
extern "C" int h3_gpu_sglang_stitch_read(h3_gpu *gpu, float *rgb) { (void)rgb; return unsupported(gpu, "h3_gpu_sglang_stitch_read: unsupported on the HIP backend"); }
extern "C" int h3_gpu_sglang_stitch_tile(h3_gpu *gpu, const h3_gpu_tensor *projected, int tile) { (void)projected; (void)tile; return unsupported(gpu, "h3_gpu_sglang_stitch_tile: unsupported on the HIP backend"); }
extern "C" void h3_gpu_sglang_text_encoder(h3_gpu *gpu) {  }
extern "C" int h3_gpu_sglang_time_features(h3_gpu *gpu, h3_gpu_tensor *out, const h3_gpu_tensor *times, uint32_t rows) { (void)out; (void)times; (void)rows; return unsupported(gpu, "h3_gpu_sglang_time_features: unsupported on the HIP backend"); }
extern "C" int h3_gpu_sglang_vae_enabled(const h3_gpu *gpu) { return 0; }
extern "C" int h3_gpu_sglang_vae_rope(h3_gpu *gpu, h3_gpu_tensor *cosine, h3_gpu_tensor *sine, uint32_t time, uint32_t height, uint32_t width, uint32_t rows) { (void)cosine; (void)sine; (void)time; (void)height; (void)width; (void)rows; return unsupported(gpu, "h3_gpu_sglang_vae_rope: unsupported on the HIP backend"); }
extern "C" h3_gpu_tensor *h3_gpu_sglang_vae_weight(h3_gpu *gpu, const h3_gpu_tensor *weight) { (void)weight; unsupported(gpu, "h3_gpu_sglang_vae_weight: unsupported on the HIP backend"); return nullptr; }
extern "C" void h3_gpu_sglang_video_encoder(h3_gpu *gpu) {  }
extern "C" int h3_gpu_sglang_vision_groups(h3_gpu *gpu, const uint32_t *counts, size_t count) { (void)counts; (void)count; return unsupported(gpu, "h3_gpu_sglang_vision_groups: unsupported on the HIP backend"); }
extern "C" int h3_gpu_sglang_vision_patch(h3_gpu *gpu, h3_gpu_tensor *out, const h3_gpu_tensor *in, const h3_gpu_tensor *weight, const h3_gpu_tensor *bias, uint32_t rows, uint32_t k, uint32_t n) { (void)out; (void)in; (void)weight; (void)bias; (void)rows; (void)k; (void)n; return unsupported(gpu, "h3_gpu_sglang_vision_patch: unsupported on the HIP backend"); }
extern "C" int h3_gpu_sglang_vision_prepare(h3_gpu *gpu, h3_gpu_tensor *position, const h3_gpu_tensor *table, h3_gpu_tensor *cosine, h3_gpu_tensor *sine, uint32_t height, uint32_t width) { (void)position; (void)table; (void)cosine; (void)sine; (void)height; (void)width; return unsupported(gpu, "h3_gpu_sglang_vision_prepare: unsupported on the HIP backend"); }
extern "C" int h3_gpu_sglang_vision_prepare_range(h3_gpu *gpu, h3_gpu_tensor *position, const h3_gpu_tensor *table, h3_gpu_tensor *cosine, h3_gpu_tensor *sine, uint32_t height, uint32_t width, uint32_t offset) { (void)position; (void)table; (void)cosine; (void)sine; (void)height; (void)width; (void)offset; return unsupported(gpu, "h3_gpu_sglang_vision_prepare_range: unsupported on the HIP backend"); }
