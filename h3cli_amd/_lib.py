"""ctypes binding of libh3hip.so (the C ABI declared in include/h3_gpu.h and
include/h3_hip_ext.h). Loading fails loudly when the library has not been built:
there is no fallback path."""
import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libh3hip.so"

F32, BF16, I8, U32, F16 = 0, 1, 2, 3, 4
HOST_VISIBLE, DEVICE_ONLY, HOST_PINNED = 0, 1, 2

_p = C.c_void_p
_u32 = C.c_uint32
_i = C.c_int
_f = C.c_float
_sz = C.c_size_t

# name: (restype, [argtypes])
_SIGNATURES = {
    # context
    "h3_gpu_create": (_p, [C.c_char_p, C.c_char_p, _sz]),
    "h3_gpu_free": (None, [_p]),
    "h3_gpu_cancel": (None, [_p]),
    "h3_gpu_backend_name": (C.c_char_p, [_p]),
    "h3_gpu_begin": (_i, [_p]),
    "h3_gpu_continue": (_i, [_p]),
    "h3_gpu_submit": (_i, [_p]),
    "h3_gpu_synchronize": (_i, [_p]),
    "h3_gpu_error": (C.c_char_p, [_p]),
    "h3_gpu_get_stats": (_i, [_p, _p]),
    # tensors
    "h3_gpu_tensor_alloc": (_p, [_p, _sz, _i, _i]),
    "h3_gpu_tensor_contents": (_p, [_p]),
    "h3_gpu_tensor_new_f32": (_p, [_p, _sz]),
    "h3_gpu_tensor_new_bf16": (_p, [_p, _sz]),
    "h3_gpu_tensor_new_i8": (_p, [_p, _sz]),
    "h3_gpu_tensor_from_f32": (_p, [_p, _p, _sz]),
    "h3_gpu_tensor_from_bf16": (_p, [_p, _p, _sz]),
    "h3_gpu_tensor_from_u32": (_p, [_p, _p, _sz]),
    "h3_gpu_tensor_read_file_bf16": (_i, [_p, C.c_char_p, C.c_uint64, _sz, C.c_char_p, _sz]),
    "h3_gpu_tensor_stream_file_bf16": (_i, [_p, C.c_char_p, C.c_uint64, _sz, C.c_char_p, _sz]),
    "h3_gpu_tensor_free": (None, [_p]),
    "h3_gpu_tensor_elements": (_sz, [_p]),
    "h3_gpu_tensor_dtype": (_i, [_p]),
    "h3_gpu_tensor_read_f32": (_i, [_p, _p, _sz]),
    "h3_gpu_tensor_read_f32_range": (_i, [_p, _sz, _p, _sz]),
    "h3_gpu_tensor_read_bf16": (_i, [_p, _p, _sz]),
    "h3_gpu_tensor_read_u32": (_i, [_p, _p, _sz]),
    "h3_gpu_tensor_write_f32": (_i, [_p, _p, _sz]),
    "h3_gpu_tensor_write_f32_range": (_i, [_p, _sz, _p, _sz]),
    "h3_gpu_tensor_write_bf16": (_i, [_p, _p, _sz]),
    "h3_gpu_tensor_write_bf16_range": (_i, [_p, _sz, _p, _sz]),
    # events
    "h3_gpu_event_new": (_p, [_p]),
    "h3_gpu_event_record": (_i, [_p, _p]),
    "h3_gpu_event_wait": (_i, [_p, _p]),
    "h3_gpu_event_free": (None, [_p]),
    # attention
    "h3_gpu_dit_attention_configure": (_i, [_p, _i]),
    "h3_gpu_dit_sdpa_bf16": (_i, [_p, _p, _p, _p, _p, _u32, _u32, _u32, _f, _i, C.c_uint, _i]),
    "h3_gpu_dit_attention_noise": (_i, [_p, _i, _f, _f]),
    "h3_gpu_sdpa_bf16": (_i, [_p, _p, _p, _p, _p, _u32, _u32, _u32, _f]),
    "h3_gpu_sdpa_bf16_head_major_output": (_i, [_p, _p, _p, _p, _p, _u32, _u32, _u32, _f]),
    # DiT block operators
    "h3_gpu_linear_bf16": (_i, [_p, _p, _p, _p, _p, _u32, _u32, _u32]),
    "h3_gpu_mlp_bf16": (_i, [_p, _p, _p, _p, _p, _u32, _u32, _u32, _u32]),
    "h3_gpu_swiglu_bf16": (_i, [_p, _p, _p, _u32, _u32]),
    "h3_gpu_gelu_bf16": (_i, [_p, _p, _p, _u32, _i]),
    "h3_gpu_adaln_bf16": (_i, [_p, _p, _p, _p, _p, _p, _u32, _u32, _u32, _u32, _u32, _f]),
    "h3_gpu_gate_bf16": (_i, [_p, _p, _p, _p, _p, _p, _u32, _u32, _u32, _u32]),
    "h3_gpu_gate_adaln_bf16": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _u32, _u32, _u32, _u32, _u32, _u32, _f]),
    "h3_gpu_qkv_rope_bf16": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _u32, _u32, _u32, _u32, _f]),
    "h3_gpu_grouped_qkv_rope_bf16": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _u32, _u32, _u32, _u32, _f]),
    "h3_gpu_grouped_qkv_linear_rope_bf16": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _u32, _u32, _u32, _u32,
                                                 _u32, _f]),
    "h3_gpu_euler_bf16": (_i, [_p, _p, _sz, _p, _p, _u32, _f, _f]),
    "h3_gpu_quant_configure": (_i, [_p, _i, C.c_char_p, C.c_uint64, C.c_uint64, _i]),
    "h3_gpu_quant_load": (_p, [_p, C.c_char_p, C.c_uint64, _u32, _u32]),
    "h3_gpu_q8_load": (_p, [_p, C.c_char_p, C.c_uint64, _u32, _u32]),
    # extensions
    "h3_hip_q8_from_packed": (_p, [_p, _p, _p, _u32, _u32, _u32]),
    "h3_hip_linear_gelu_bf16": (_i, [_p, _p, _p, _p, _p, _u32, _u32, _u32]),
    "h3_hip_version": (C.c_char_p, []),
    "h3_hip_dit_block_mask": (_i, [_p, _p, _u32, _u32, _u32]),
    "h3_hip_sage_pack": (_i, [_p, _p, _p, _p, _u32, _u32, _p, _p, _p, _p, _p, _p, _p]),
    "h3_hip_sage_v_position": (C.c_uint, [C.c_uint]),
    "h3_hip_timing_event_new": (_p, [_p]),
    "h3_hip_event_elapsed_ms": (_i, [_p, _p, _p, C.POINTER(_f)]),
    "h3_hip_host_alloc": (_p, [_p, _sz]),
    "h3_hip_host_free": (None, [_p, _p, _sz]),
    "h3_hip_tensor_stream_host": (_i, [_p, _p, _sz]),
    "h3_hip_tensor_read_bytes": (_i, [_p, _p, _sz]),
    "h3_hip_fill_normal_bf16": (_i, [_p, _p, C.c_uint64, _f, _sz]),
    "h3_hip_synthetic_block_mask": (C.c_uint, [_p, C.c_uint, C.c_uint, C.c_uint, C.c_double, C.c_uint64]),
}



class SolBlock(C.Structure):
    """h3_sol_block (include/h3_gpu_surface.h; reference src/denoise/sol.h:7)."""
    _fields_ = [("protect", C.c_uint32), ("first_frame", C.c_int32), ("last_frame", C.c_int32), ("rows", C.c_uint32)]


class SolLayout(C.Structure):
    """h3_sol_layout (include/h3_gpu_surface.h; reference src/denoise/sol.h:8-11)."""
    _fields_ = [("sequence", C.c_uint32), ("query_blocks", C.c_uint32), ("key_blocks", C.c_uint32),
                ("protected_rows", C.c_uint32), ("query", C.POINTER(SolBlock)), ("key", C.POINTER(SolBlock))]

class GpuStats(C.Structure):
    """h3_gpu_stats (include/h3_gpu.h), field for field."""
    _fields_ = [("q8_weights", C.c_uint64), ("q8_source_bytes", C.c_uint64), ("q8_storage_bytes", C.c_uint64), ("q8_dispatches", C.c_uint64), ("q8_load_seconds", C.c_double), ("layout_prepares", C.c_uint64), ("layout_inplace_packs", C.c_uint64), ("layout_scan_replaced_bytes", C.c_uint64), ("layout_partial_bytes", C.c_uint64), ("allocated_bytes", C.c_uint64), ("live_bytes", C.c_uint64), ("peak_live_bytes", C.c_uint64), ("tensor_allocations", C.c_uint64), ("direct_dispatches", C.c_uint64), ("mps_linear_dispatches", C.c_uint64), ("mps_conv_dispatches", C.c_uint64), ("mps_sdpa_dispatches", C.c_uint64), ("native_attention_dispatches", C.c_uint64), ("metal_current_allocated_bytes", C.c_uint64), ("blit_copies", C.c_uint64), ("submissions", C.c_uint64), ("command_encode_seconds", C.c_double), ("command_wait_seconds", C.c_double), ("gpu_seconds", C.c_double), ("linear_dispatches", C.c_uint64), ("conv_dispatches", C.c_uint64), ("attention_dispatches", C.c_uint64), ("h2d_bytes", C.c_uint64), ("d2h_bytes", C.c_uint64), ("d2d_bytes", C.c_uint64), ("streamed_bytes", C.c_uint64), ("resident_weight_bytes", C.c_uint64), ("stream_slot_bytes", C.c_uint64), ("resident_block_mask", C.c_uint64), ("resident_blocks", C.c_uint32), ("active_weight_blocks", C.c_uint32), ("device_bytes", C.c_uint64), ("managed_bytes", C.c_uint64), ("pinned_bytes", C.c_uint64), ("peak_pinned_bytes", C.c_uint64), ("stream_stalls", C.c_uint64), ("transfer_seconds", C.c_double), ("stream_wait_seconds", C.c_double), ("linear_seconds", C.c_double), ("attention_seconds", C.c_double), ("conv_seconds", C.c_double), ("h2d_seconds", C.c_double), ("d2h_seconds", C.c_double), ("slot_wait_seconds", C.c_double), ("normalization_seconds", C.c_double), ("weight_cache_bytes", C.c_uint64), ("weight_cache_hits", C.c_uint64), ("weight_cache_hit_bytes", C.c_uint64), ("weight_cache_misses", C.c_uint64), ("weight_cache_evictions", C.c_uint64), ("quant_conversion_seconds", C.c_double), ("quant_clipped_values", C.c_uint64), ("quant_zeroed_values", C.c_uint64), ("quant_projection_dispatches", C.c_uint64), ("quant_cache_hits", C.c_uint64), ("quant_cache_misses", C.c_uint64), ("sage2_attention_dispatches", C.c_uint64), ("sage3_attention_dispatches", C.c_uint64), ("attention_workspace_bytes", C.c_uint64), ("inflight_peak", C.c_uint64), ("command_retirements", C.c_uint64), ("bounded_waits", C.c_uint64), ("pressure_drains", C.c_uint64), ("native_scratch_bytes", C.c_uint64), ("native_scratch_allocations", C.c_uint64), ("native_scratch_reuses", C.c_uint64), ("native_pipeline_count", C.c_uint64), ("main_dense_calls", C.c_uint64), ("subblock_calls", C.c_uint64), ("subblock_bypass", C.c_uint64), ("subblock_protected_calls", C.c_uint64), ("subblock_selected", C.c_uint64), ("subblock_possible", C.c_uint64), ("subblock_router_calls", C.c_uint64), ("attention_timing_samples", C.c_uint64), ("attention_timing_missed", C.c_uint64), ("main_attention_seconds", C.c_double), ("subblock_router_seconds", C.c_double), ("subblock_kernel_seconds", C.c_double)]

class DitSynthConfig(C.Structure):
    """include/h3_dit_synth.h h3_hip_dit_synth_config."""
    _fields_ = [("blocks", _u32), ("hidden", _u32), ("heads", _u32), ("mlp", _u32),
                ("frames", _u32), ("height", _u32), ("width", _u32), ("audio_rows", _u32),
                ("latent", _u32), ("streamed_first", _u32), ("mask_density", _f),
                ("attention_mode", _i), ("eps", _f), ("time", _f), ("seed", C.c_uint64),
                ("rope_half", _u32), ("swiglu", _i), ("qk_norm", _i), ("grouped_qkv", _i),
                ("subblock_sparsity", _f), ("projection_quant", _i), ("trace_block", _u32)]


_SIGNATURES.update({
    "h3_hip_dit_synth_default": (DitSynthConfig, []),
    "h3_hip_dit_synth_h3": (DitSynthConfig, []),
    "h3_hip_dit_synth_create": (_p, [_p, C.POINTER(DitSynthConfig), C.c_char_p, _sz]),
    "h3_hip_dit_synth_free": (None, [_p]),
    "h3_hip_sdpa_bf16_noalloc": (_i, [_p, _p, _p, _p, _p, _u32, _u32, _u32, _f, _i]),
    "h3_sglang_flash": (_i, [_p, _p, _p, _p, _p, _u32, _u32, _u32, _u32, _u32, _f, _i, _i, _p, C.c_char_p, _sz]),
    "h3_sglang_flash_query_range": (_i, [_p, _p, _p, _p, _p, _u32, _u32, _u32, _u32, _f, _i, _p, C.c_char_p, _sz]),
    "h3_hip_tensor_device_pointer": (_p, [_p]),
    "h3_hip_compute_stream": (_p, [_p]),
    "h3_hip_dit_time_features": (None, [_p, _u32, _p]),
    "h3_hip_dit_rope_tables": (_i, [_u32, _u32, _u32, _u32, _u32, _p, _p]),
    "h3_hip_dit_synth_load": (_i, [_p, C.c_char_p, C.c_char_p, _sz]),
    "h3_hip_dit_synth_step": (_i, [_p, _i, _f]),
    "h3_hip_dit_synth_tensor": (_p, [_p, C.c_char_p]),
    "h3_hip_dit_synth_rows": (_u32, [_p]),
    "h3_hip_dit_synth_kept_blocks": (C.c_uint64, [_p, C.POINTER(C.c_uint64)]),
    "h3_gpu_add_bf16": (_i, [_p, _p, _p, _p, _u32]),
    "h3_gpu_silu_bf16": (_i, [_p, _p, _p, _u32]),
    "h3_gpu_cast_f32_to_bf16": (_i, [_p, _p, _p, _u32]),
    "h3_gpu_cast_bf16_to_f32": (_i, [_p, _p, _p, _u32]),
    "h3_hip_q8_new": (_p, [_p, _u32, _u32, _u32]),
    "h3_hip_fill_q8_random": (_i, [_p, _p, C.c_uint64, _f, _f]),
    "h3_hip_tensor_copy_to_host": (_i, [_p, _p, _sz]),
    "h3_hip_dit_subblock_policy": (_i, [_p, _f, _i]),
    "h3_hip_subblock_routes": (_i, [_p, _p, _p, C.c_size_t, _p, _p, C.c_size_t]),
    "h3_hip_subblock_workspace_cap": (_i, [_p, _sz]),
    "h3_hip_subblock_plan_info": (_i, [_p, _p, _p, _p]),
    "h3_hip_sol_workspace_cap": (_i, [_p, _sz]),
    "h3_hip_sol_plan_info": (_i, [_p, _p, _p]),
    "h3_hip_sol_routes": (_i, [_p, _p, C.c_size_t, _p, C.c_size_t, _p, _p, C.c_size_t]),
    "h3_hip_dit_sol_force_exact": (_i, [_p, _i]),
    "h3_hip_sol_counters": (_i, [_p, _p, C.c_size_t]),
    "h3_hip_sha256": (_i, [_p, C.c_size_t, _p]),
    "h3_hip_fp8_pack": (_i, [_p, _p, _p, _p, C.c_size_t]),
    "h3_hip_quant_weight_from_bf16": (_p, [_p, _p, _u32, _u32]),
    # the rest of the reference surface implemented here (include/h3_gpu_surface.h)
    "h3_gpu_adaln_bf16_offset": (_i, [_p, _p, _p, _sz, _p, _p, _p, _u32, _u32, _u32, _u32, _u32, _f]),
    "h3_gpu_rms_norm_bf16": (_i, [_p, _p, _p, _p, _u32, _u32, _f]),
    "h3_gpu_head_rms_norm_bf16": (_i, [_p, _p, _p, _u32, _u32, _u32, _f]),
    "h3_gpu_sub_bf16": (_i, [_p, _p, _p, _p, _u32]),
    "h3_gpu_silu_mul_bf16": (_i, [_p, _p, _p, _p, _u32]),
    "h3_gpu_patch_linear_bf16": (_i, [_p, _p, _p, _p, _p, _u32, _u32, _u32]),
    "h3_gpu_patch_linear_bf16_offset": (_i, [_p, _p, _sz, _p, _sz, _p, _p, _u32, _u32, _u32]),
    "h3_gpu_patch_linear_bf16_map": (_i, [_p, _p, _p, _p, _p, _p, _u32, _u32, _u32, _u32]),
    "h3_gpu_copy_bf16": (_i, [_p, _p, _sz, _p, _sz, _sz]),
    "h3_gpu_copy_f32": (_i, [_p, _p, _sz, _p, _sz, _sz]),
    "h3_gpu_tensor_load_bf16": (_p, [_p, C.c_char_p, C.c_uint64, _sz]),
    "h3_gpu_tensor_load_f32": (_p, [_p, C.c_char_p, C.c_uint64, _sz]),
    "h3_gpu_plan_weights": (_i, [_p, C.c_uint64, C.c_uint64]),
    "h3_gpu_plan_bf16_weights": (_i, [_p, C.c_uint64, C.c_uint64, C.c_uint64, _i, _i, _p]),
    "h3_gpu_weight_plan_compatible": (_i, [_p, _i]),
    "h3_gpu_dit_sol_layout": (_i, [_p, _p]),
    "h3_gpu_profile_set_label": (None, [_p, C.c_char_p]),
    "h3_gpu_profile_mark": (None, [_p, C.c_char_p]),
    "h3_device_query": (_i, [_p, C.c_char_p, _sz]),
    "h3_hip_kernel_timing": (_i, [_p, _i]),
    "h3_hip_kernel_timing_read": (_i, [_p, C.POINTER(C.c_double), C.POINTER(C.c_uint64)]),
    "h3_device_configure": (_i, [C.c_char_p, C.c_char_p, C.c_char_p, _sz]),
    "h3_device_memory_fits": (_i, [C.c_uint64]),
    "h3_subblock_budget": (C.c_uint, [C.c_uint, _f]),
    "h3_subblock_warmup": (_i, [_i]),
    "h3_subblock_dense_reason": (C.c_char_p, [C.c_uint, C.c_uint, _i, _f, _i]),
    "h3_attention_name": (C.c_char_p, [_i]),
    "h3_attention_parse": (_i, [C.c_char_p, C.POINTER(_i)]),
    "h3_attention_options": (_i, [_i, C.c_char_p, _sz]),
    "h3_attention_preflight": (_i, [_i, C.c_char_p, _sz]),
})

# Declared in include/*.h but optional for this module's loader (added as the
# backend grows); listed so the export test can check them when present.
_OPTIONAL = set()

_lib = None


def load():
    """Load libh3hip.so and bind every known signature. Raises if not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is not built: run `python -m h3cli_amd.build` "
                           "(the HIP backend has no fallback)")
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name, None)
        if fn is None:
            if name in _OPTIONAL:
                continue
            raise RuntimeError(f"libh3hip.so does not export {name}")
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def signatures():
    return dict(_SIGNATURES)
