// Projection GEMMs of the DiT block for gfx950: y[M,N] = x[M,K] . W[N,K]^T (+bias)
// (+GELU-tanh), BF16 activations and output, FP32 accumulation.
//
// Weights are either BF16 (reference h3_gpu_linear_bf16, src/cuda/gpu_cuda.cu:927-1011)
// or W8A16 q8: int8 codes [N,K] with fp32 scales per (row, K-group); the group is
// 64 in the reference q8 recipe (src/weights/q8.c:26-56) or K for one scale per
// output channel. The q8 arithmetic is the reference's Metal kernel
// (src/metal/shaders.metal:799-855): every weight is reconstructed as
// w = bf16(code * scale) and multiplied in FP32 accumulation, bf16 output (+bias).
//
// MI355X design:
//  * C^T = W . X^T on v_mfma_f32_32x32x16_bf16, so a lane owns one output row and
//    four consecutive columns per register group (8-byte row-major stores);
//  * 256 x 256 output tile per workgroup of 4 waves (each 128 x 128, 16
//    accumulator blocks), K staged 64 at a time, double buffered in LDS;
//  * X tiles go global -> LDS directly (global_load_lds_dwordx4, XOR-swizzled
//    16-byte chunks); int8 weight tiles are loaded into registers one tile ahead,
//    dequantized in registers (w = bf16(code * scale)) and written to LDS as BF16,
//    so each weight is converted once per workgroup, not per wave;
//  * tile ids are XCD-remapped and grouped along M so that the workgroups an XCD
//    runs together share weight columns in its L2.
#include "common.h"
#include "internal.h"
#include <cmath>

namespace {

constexpr int TM = 256, TN = 256, TK = 64;
constexpr int ROW_BYTES = TK * 2;               // 128 B per BF16 tile row
constexpr int TILE_BYTES = 256 * ROW_BYTES;     // 32 KB per operand tile
constexpr int STAGE = 2 * TILE_BYTES;           // X tile + W tile
constexpr int GROUP_M = 8;                      // tile rows per grouped band

__device__ inline unsigned swz(unsigned row, unsigned ch) { return ch ^ ((row >> 1) & 7); }

struct GemmArgs {
    uint16_t *y;
    const uint16_t *x;
    const void *w;            // bf16 [N,K] or int8 [N,K]
    const float *scales;      // q8: [N, groups]
    const uint16_t *bias;     // optional [N]
    unsigned m, n, k, group, groups;
    int gelu;
};

__device__ inline float gelu_tanh(float v) {
    // Reference h3_gelu_bf16, approximate form (src/cuda/cuda_kernels.cuh:879-902).
    float inner = 0.7978845608028654f * (v + 0.044715f * v * v * v);
    return inner <= -10.0f ? 0.0f : inner >= 10.0f ? v : 0.5f * v * (1.0f + tanhf(inner));
}

template <bool Q8>
__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void gemm_kernel(GemmArgs a) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    const unsigned tid = threadIdx.x, wave = tid / 64, lane = tid % 64, n32 = lane % 32, hf = lane / 32;
    const unsigned tiles_m = (a.m + TM - 1) / TM, tiles_n = a.n / TN;
    // XCD-aware id, then grouped ordering: GROUP_M tile rows sweep the columns together.
    const unsigned pid = xcd_remap(blockIdx.x, gridDim.x);
    const unsigned band = pid / (GROUP_M * tiles_n), first_m = band * GROUP_M;
    const unsigned rows_in_band = min(tiles_m - first_m, (unsigned)GROUP_M);
    const unsigned tm = first_m + (pid % (GROUP_M * tiles_n)) % rows_in_band;
    const unsigned tn = (pid % (GROUP_M * tiles_n)) / rows_in_band;
    const unsigned m0 = tm * TM, n0 = tn * TN;
    // Wave (wm, wn) owns output rows m0 + wm*128 .. +128 and columns n0 + wn*128 .. +128.
    const unsigned wm = wave / 2, wn = wave % 2;
    const unsigned ksteps = a.k / TK;

    f32x16 acc[4][4];   // [n block][m block], C^T layout: lane = output row, regs = columns
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f32x16{};

    // Weight staging (q8): 256 rows x 64 int8 = 1024 16-byte chunks, 4 per thread.
    i32x4 wq[4];
    float wscale[4];
    auto load_w = [&](unsigned kt) {
        if constexpr (Q8) {
            const int8_t *w8 = reinterpret_cast<const int8_t *>(a.w);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                unsigned c = tid + 256 * j, row = c / 4, part = c % 4;
                size_t off = (size_t)(n0 + row) * a.k + kt * TK + part * 16;
                wq[j] = *reinterpret_cast<const i32x4 *>(w8 + off);
                wscale[j] = a.scales[(size_t)(n0 + row) * a.groups + (kt * TK + part * 16) / a.group];
            }
        }
    };
    auto store_w = [&](int stage) {
        if constexpr (Q8) {
            uint8_t *ws = lds + stage * STAGE + TILE_BYTES;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                unsigned c = tid + 256 * j, row = c / 4, part = c % 4;
                bf16x8 lo, hi;
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    int q = (int)(int8_t)((wq[j][e / 4] >> (8 * (e % 4))) & 0xff);
                    __bf16 v = (__bf16)((float)q * wscale[j]);
                    if (e < 8) lo[e] = v; else hi[e - 8] = v;
                }
                *reinterpret_cast<bf16x8 *>(ws + row * ROW_BYTES + swz(row, part * 2) * 16) = lo;
                *reinterpret_cast<bf16x8 *>(ws + row * ROW_BYTES + swz(row, part * 2 + 1) * 16) = hi;
            }
        }
    };
    // Direct global -> LDS loads: X rows (clamped at M) and, for BF16 weights, W rows.
    auto load_direct = [&](unsigned kt, int stage) {
        uint8_t *xs = lds + stage * STAGE;
#pragma unroll
        for (unsigned b = wave; b < 32; b += 4) {
            unsigned row = 8 * b + lane / 8, ph = lane % 8;
            unsigned gm = min(m0 + row, a.m - 1);
            const uint16_t *src = a.x + (size_t)gm * a.k + kt * TK + swz(row, ph) * 8;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                             (__attribute__((address_space(3))) void *)(xs + b * 1024), 16, 0, 0);
            if constexpr (!Q8) {
                const uint16_t *wsrc = reinterpret_cast<const uint16_t *>(a.w) + (size_t)(n0 + row) * a.k + kt * TK + swz(row, ph) * 8;
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)wsrc,
                                                 (__attribute__((address_space(3))) void *)(xs + TILE_BYTES + b * 1024), 16, 0, 0);
            }
        }
    };

    load_direct(0, 0);
    load_w(0);
    store_w(0);
    wait_vm_loads();
    __syncthreads();

    for (unsigned kt = 0; kt < ksteps; kt++) {
        const int cur = kt & 1;
        const bool more = kt + 1 < ksteps;
        if (more) { load_direct(kt + 1, cur ^ 1); load_w(kt + 1); }
        const uint8_t *xs = lds + cur * STAGE;
        const uint8_t *ws = xs + TILE_BYTES;
#pragma unroll
        for (int ks = 0; ks < TK / 16; ks++) {
            bf16x8 wf[4], xf[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                unsigned wr = wn * 128 + i * 32 + n32, xr = wm * 128 + i * 32 + n32;
                wf[i] = *reinterpret_cast<const bf16x8 *>(ws + wr * ROW_BYTES + swz(wr, ks * 2 + hf) * 16);
                xf[i] = *reinterpret_cast<const bf16x8 *>(xs + xr * ROW_BYTES + swz(xr, ks * 2 + hf) * 16);
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[i], xf[j], acc[i][j], 0, 0, 0);
        }
        if (more) store_w(cur ^ 1);
        wait_vm_loads();
        __syncthreads();
    }

    // Epilogue: lane holds output row m = m0 + wm*128 + j*32 + n32 and columns
    // n0 + wn*128 + i*32 + g*8 + hf*4 + 0..3 for register group g.
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const unsigned row = m0 + wm * 128 + j * 32 + n32;
        if (row >= a.m) continue;
        uint16_t *dst = a.y + (size_t)row * a.n;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const unsigned col = n0 + wn * 128 + i * 32 + g4 * 8 + hf * 4;
                u16x4 out;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float v = acc[i][j][g4 * 4 + e];
                    if (a.bias) v += bf16_to_f32(a.bias[col + e]);
                    uint16_t b = f32_to_bf16(v);
                    if (a.gelu) b = f32_to_bf16(gelu_tanh(bf16_to_f32(b)));
                    out[e] = b;
                }
                *reinterpret_cast<u16x4 *>(dst + col) = out;
            }
    }
}

// Any-shape fallback (small or unaligned projections): one thread per output,
// FP32 accumulation in k order. Same weight reconstruction as the tiled kernel.
__global__ __launch_bounds__(256) void gemm_small(GemmArgs a, int q8) {
    size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)a.m * a.n) return;
    unsigned row = idx / a.n, col = idx % a.n;
    const uint16_t *xr = a.x + (size_t)row * a.k;
    float acc = 0.f;
    for (unsigned kk = 0; kk < a.k; kk++) {
        float w;
        if (q8) {
            int q = reinterpret_cast<const int8_t *>(a.w)[(size_t)col * a.k + kk];
            w = bf16_to_f32(f32_to_bf16((float)q * a.scales[(size_t)col * a.groups + kk / a.group]));
        } else {
            w = bf16_to_f32(reinterpret_cast<const uint16_t *>(a.w)[(size_t)col * a.k + kk]);
        }
        acc = fmaf(bf16_to_f32(xr[kk]), w, acc);
    }
    if (a.bias) acc += bf16_to_f32(a.bias[col]);
    uint16_t b = f32_to_bf16(acc);
    if (a.gelu) b = f32_to_bf16(gelu_tanh(bf16_to_f32(b)));
    a.y[idx] = b;
}

template <bool Q8>
int launch_tiled(h3_gpu *g, const GemmArgs &a) {
    constexpr size_t shared = 2 * STAGE;
    static bool configured = false;
    if (!configured) {
        if (!h3_hip_check(g, hipFuncSetAttribute((const void *)gemm_kernel<Q8>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)shared), "GEMM shared memory"))
            return 0;
        configured = true;
    }
    unsigned tiles = (a.m + TM - 1) / TM * (a.n / TN);
    hipLaunchKernelGGL(gemm_kernel<Q8>, dim3(tiles), dim3(256), shared, g->compute, a);
    return h3_launch_status(g, Q8 ? "W8A16 GEMM" : "BF16 GEMM");
}

}  // namespace

int h3_gemm(h3_gpu *g, uint16_t *y, const uint16_t *x, const h3_gpu_tensor *w, const uint16_t *bias, uint32_t m,
            uint32_t k, uint32_t n, int gelu) {
    GemmArgs a;
    a.y = y; a.x = x; a.w = w->data; a.bias = bias; a.m = m; a.n = n; a.k = k; a.gelu = gelu;
    a.scales = w->q8 ? w->q8_scales : nullptr;
    a.group = w->q8 ? w->q8_group : 1;
    a.groups = w->q8 ? (k + a.group - 1) / a.group : 1;
    if (!h3_tensor_acquire(g, w)) return 0;
    int ok;
    const bool tiled = n % TN == 0 && k % TK == 0 && m >= 32 && (!w->q8 || a.group % 16 == 0);
    if (tiled) ok = w->q8 ? launch_tiled<true>(g, a) : launch_tiled<false>(g, a);
    else {
        size_t total = (size_t)m * n;
        hipLaunchKernelGGL(gemm_small, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, g->compute, a, w->q8 ? 1 : 0);
        ok = h3_launch_status(g, "small GEMM");
    }
    if (ok) {
        g->stats.linear_dispatches++;
        if (w->q8) { g->stats.q8_dispatches++; g->stats.quant_projection_dispatches++; }
    }
    return ok && h3_tensor_release(g, w);
}
