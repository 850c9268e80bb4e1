// Device generator of the seeded synthetic inputs: the same splitmix64 +
// Box-Muller stream as h3cli_amd/synth.py (float64 math, then float32 * scale,
// then BF16 round-to-nearest-even), so full-size benchmark inputs need no host
// generation or PCIe upload.
#include "common.h"
#include "internal.h"

__device__ inline uint64_t splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void fill_normal_bf16(uint16_t *out, size_t count, uint64_t seed, float scale) {
    size_t j = (size_t)blockIdx.x * 256 + threadIdx.x;  // pair index
    if (2 * j >= count) return;
    uint64_t base = seed << 40;
    uint64_t a = splitmix64(base + 2 * j), b = splitmix64(base + 2 * j + 1);
    double u1 = ((double)(a >> 11) + 1.0) * 0x1.0p-53;
    double u2 = (double)(b >> 11) * 0x1.0p-53;
    double r = sqrt(-2.0 * log(u1));
    double s, c;
    sincos(2.0 * 3.14159265358979323846 * u2, &s, &c);
    out[2 * j] = f32_to_bf16((float)(r * c) * scale);
    if (2 * j + 1 < count) out[2 * j + 1] = f32_to_bf16((float)(r * s) * scale);
}

extern "C" int h3_hip_fill_normal_bf16(h3_gpu *g, h3_gpu_tensor *t, uint64_t seed, float scale, size_t count) {
    if (!h3_launch_ready(g) || !h3_require(g, t, H3_GPU_BF16, count, "fill")) return 0;
    if (!count) return 1;
    size_t pairs = (count + 1) / 2;
    hipLaunchKernelGGL(fill_normal_bf16, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, g->compute,
                       (uint16_t *)t->data, count, seed, scale);
    return h3_launch_status(g, "normal fill");
}

// Seeded random W8A16 weights: code = (u % 255) - 127 with u = splitmix64((seed << 40) + i)
// over the codes, and scale = lo + (hi - lo) * ((v >> 11) * 2^-53) with
// v = splitmix64((seed << 40) + (1 << 39) + j) over the scales.
__global__ __launch_bounds__(256) void fill_q8(int8_t *codes, size_t n, float *scales, size_t ns, uint64_t seed,
                                              float lo, float hi) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    uint64_t base = seed << 40;
    if (i < n) codes[i] = (int8_t)((int)(splitmix64(base + i) % 255u) - 127);
    if (i < ns) {
        double u = (double)(splitmix64(base + (1ull << 39) + i) >> 11) * 0x1.0p-53;
        scales[i] = lo + (hi - lo) * (float)u;
    }
}

extern "C" int h3_hip_fill_q8_random(h3_gpu *g, h3_gpu_tensor *t, uint64_t seed, float lo, float hi) {
    if (!h3_launch_ready(g) || !t || !t->q8) return h3_set_error(g, "q8 fill: needs a q8 weight and an active command");
    size_t n = t->elements, ns = (size_t)t->q8_rows * ((t->q8_cols + t->q8_group - 1) / t->q8_group);
    size_t total = n > ns ? n : ns;
    hipLaunchKernelGGL(fill_q8, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, g->compute, (int8_t *)t->data, n,
                       t->q8_scales, ns, seed, lo, hi);
    return h3_launch_status(g, "q8 fill");
}

// Device -> host copy of a tensor (q8: codes then scales, the stream_host layout).
extern "C" int h3_hip_tensor_copy_to_host(h3_gpu_tensor *t, void *dst, size_t bytes) {
    if (!t || !dst) return 0;
    h3_gpu *g = t->owner;
    size_t code_bytes = t->bytes, scale_bytes = 0;
    if (t->q8) scale_bytes = (size_t)t->q8_rows * ((t->q8_cols + t->q8_group - 1) / t->q8_group) * 4;
    if (bytes != code_bytes + scale_bytes) return h3_set_error(g, "copy to host: %zu bytes, tensor holds %zu", bytes, code_bytes + scale_bytes);
    return h3_hip_check(g, hipStreamSynchronize(g->compute), "copy fence") &&
           h3_hip_check(g, hipMemcpy(dst, t->data, code_bytes, hipMemcpyDeviceToHost), "copy codes") &&
           (!scale_bytes || h3_hip_check(g, hipMemcpy((char *)dst + code_bytes, t->q8_scales, scale_bytes, hipMemcpyDeviceToHost), "copy scales"));
}
