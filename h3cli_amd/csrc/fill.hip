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
