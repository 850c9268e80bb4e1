// Internal definitions shared by the gfx950 backend translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstddef>
#include <cstdio>
#include <cstdarg>
#include <cstring>
#include <mutex>
#include <utility>
#include <vector>
#include "../../include/h3_gpu.h"
#include "../../include/h3_hip_ext.h"

// ---------------------------------------------------------------- vector types
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- bf16 helpers
__host__ __device__ inline float bf16_to_f32(uint16_t b) {
    return __builtin_bit_cast(float, (uint32_t)b << 16);
}
// Round-to-nearest-even; NaN stays a quiet NaN.
// Round-to-nearest-even FP32 -> BF16. On the device this is one
// v_cvt_pk_bf16_f32 (same result for every non-NaN input; NaN becomes a quiet
// NaN); the host keeps the bit-level rounding.
__host__ __device__ inline uint16_t f32_to_bf16(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_bit_cast(uint16_t, (__bf16)f);
#else
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
#endif
}

// Finite test on the bit pattern. The library is built with relaxed NaN
// semantics, so the bits pass through an opaque step that keeps the compiler
// from turning the test back into a floating-point compare it may fold.
__host__ __device__ inline bool finite_f32(float x) {
    uint32_t u = __builtin_bit_cast(uint32_t, x);
#ifdef __HIP_DEVICE_COMPILE__
    asm volatile("" : "+v"(u));
#else
    volatile uint32_t opaque = u;
    u = opaque;
#endif
    return (u & 0x7f800000u) != 0x7f800000u;
}

// Non-finite test on raw BF16 bits (exponent all ones = Inf or NaN), two
// values per 32-bit word. Integer-only, so it holds under any FP assumptions.
__host__ __device__ inline bool bf16x2_nonfinite(uint32_t w) {
    return ((w & 0x7f80u) == 0x7f80u) | ((w & 0x7f800000u) == 0x7f800000u);
}
template <class V>
__device__ inline bool bf16_vec_nonfinite(const V &v) {
    static_assert(sizeof(V) % 4 == 0, "vector of BF16 pairs");
    bool bad = false;
#pragma unroll
    for (unsigned i = 0; i < sizeof(V) / 4; i++)
        bad |= bf16x2_nonfinite(reinterpret_cast<const uint32_t *>(&v)[i]);
    return bad;
}

// A wave-uniform load from memory no kernel writes while this one runs,
// through the constant address space: hipcc then issues a scalar load
// (s_load, counted by lgkmcnt). A vector load of the same value is counted by
// vmcnt, and the wait for it also waits for every earlier direct global->LDS
// tile load, which ends the prefetch of the next tile early.
template <typename T> __device__ inline T load_uniform(const T *p) {
    return *(const __attribute__((address_space(4))) T *)p;
}
// Wait for this wave's outstanding vector-memory loads, including direct
// global->LDS loads, before a barrier publishes their LDS contents.
__device__ inline void wait_vm_loads() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// Raw buffer loads return zeros for a per-lane (VGPR) offset past the
// descriptor's size. The kernels rely on that check only, not on one covering
// the uniform (SGPR) offset: a row past a tensor's end that the SGPR offset
// reaches is masked with this VGPR offset instead. It is past every size below
// 4 GiB, and even as a 32-bit sum with an SGPR offset it addresses no byte
// outside the tensor's own 4 GiB window.
constexpr uint32_t BUFFER_OOB = 0xFFFFFFF0u;

// ---------------------------------------------------------------- objects
struct h3_gpu_tensor {
    h3_gpu *owner;
    void *data;             // device (or pinned host) pointer
    size_t elements;
    size_t bytes;           // logical bytes (elements * item size)
    size_t bytes_alloc;     // allocated bytes (with tail slack)
    h3_gpu_dtype dtype;
    h3_gpu_storage storage;
    // W8A16 weight: data holds int8 codes [rows, cols]; scales fp32 [rows, groups].
    int q8;
    uint32_t q8_rows, q8_cols, q8_group;
    float *q8_scales;
    // FP8 packed projection weight (h3_gpu_quant_load): data holds the packed
    // descriptor (codes [quant_n, quant_k], scale at quant_scale, global slot at
    // quant_global), in device memory or, for streamed weights, pinned host memory.
    int quant_mode;
    uint32_t quant_n, quant_k;
    size_t quant_scale, quant_global;
    void *quant_dequant;    // NVFP4 resident weight: BF16 code * block scale [quant_n, quant_k]
    // Streaming fences (copy stream fills, compute stream reads).
    hipEvent_t ready, released;
    bool ready_pending, release_recorded;
};

struct h3_gpu_event { hipEvent_t event; };

struct h3_attention_state;  // attention.hip
struct h3_stream_state;     // context.hip (weight streaming bounce buffers)

struct h3_gpu {
    int device;
    hipStream_t compute, copy;
    bool active, deferred_error;
    char error[1024];
    h3_gpu_stats stats;
    unsigned *fault;        // device flags: [0] nonfinite attention, [1] Sage quantizer, [2] FP8 projection input
    int quant_mode;
    struct h3_quant_state *quant;   // quant.hip: artifact cache and FP8 workspaces (mode 1)
    h3_attention_state *attention;
    h3_stream_state *streaming;
    std::mutex copy_mutex;
    // optional event timing of attention / linear dispatches (H3_PROFILE)
    bool profiling;
    // Kernel-shape selector for measurement (H3_HIP_ATTENTION_VARIANT): 0 is the
    // default shape, other values pick the alternatives each kernel documents.
    int attention_variant;
    int gemm_variant;
    char label[64];         // h3_gpu_profile_set_label
    double created;         // wall clock at creation (profile marks)
    bool allocation_failed; // a device allocation ran out of memory
    // Opt-in timing of the dominant kernel of each dispatch (h3_hip_kernel_timing):
    // event pairs on the compute stream, summed when read.
    bool kernel_timing;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> *kernel_events;
    // gemm.hip: BF16 values of the W8A16 weight of the current projection
    // (grow-only; reused by every projection on the compute stream).
    void *gemm_weights;
    size_t gemm_weights_bytes;
};

// ---------------------------------------------------------------- helpers
int h3_set_error(h3_gpu *g, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int h3_hip_check(h3_gpu *g, hipError_t e, const char *what);
int h3_launch_ready(h3_gpu *g);
int h3_launch_status(h3_gpu *g, const char *what);
int h3_require(h3_gpu *g, const h3_gpu_tensor *t, h3_gpu_dtype dtype, size_t elements, const char *name);
void h3_stats_track_alloc(h3_gpu *g, size_t bytes, int sign);

// Number of XCDs on MI355X; workgroups are dispatched round-robin across them.
constexpr int kXcds = 8;

// Bijective remap of a linear workgroup id so that consecutive logical ids land
// on the same XCD (and its L2): hardware id i runs on XCD i % 8.
__device__ inline unsigned xcd_remap(unsigned pid, unsigned total) {
    unsigned per = (total + kXcds - 1) / kXcds;
    unsigned tall = total % kXcds; if (tall == 0) tall = kXcds;
    unsigned xcd = pid % kXcds, local = pid / kXcds;
    if (xcd < tall) return xcd * per + local;
    return tall * per + (xcd - tall) * (per - 1) + local;
}
