// FP8 W8A8 DiT projections (reference src/cuda/cuda_quant.cuh): tensorwide
// E4M3 packing of weights and activations, the content-hashed packed-weight
// artifacts (H3QWT001), and an FP8 GEMM on gfx950's v_mfma_f32_32x32x64_f8f6f4
// in place of cuBLASLt.
//
// Arithmetic contract (cuda_quant.cuh:26-49, 362-394):
//   scale = max(max|x| / 448, 1e-20), code = E4M3(x / scale), RNE, saturating;
//   y = bf16(sx * sw * sum_k x8[m,k] * w8[n,k]), FP32 accumulation.
// Packed weight descriptor (src/weights/residency.c:39-51): n*k codes, the
// 4-byte scale at the 256-aligned `scale` offset, and a 16-byte global slot
// {scale, 1, 0, 0} at the 256-aligned `global` offset, zero elsewhere; this is
// the artifact payload, so caches written by either build are interchangeable.
//
// MI355X design:
//  * packing is HBM-bound: a max pass (16-byte loads, per-workgroup maxima),
//    a one-workgroup finish, and an encode pass (16-byte loads, 8-byte stores);
//  * the GEMM computes C^T = W . X^T with 256 x 256 output tiles, 8 waves (two
//    per SIMD, 128 x 64 each), 128-byte K stages of both operands loaded
//    global -> LDS directly (XOR-swizzled 16-byte chunks), double buffered;
//    each K stage is two 32x32x64 FP8 MFMA steps per accumulator block, the
//    fragments of the next step read during the current one; workgroup ids are
//    XCD-remapped and grouped along M, as in the BF16 GEMM.
#include "common.h"
#include "internal.h"
#include "sage.h"
#include "../../include/h3_quant.h"
#include "../../include/h3_residency.h"
#include "../../include/h3_gpu_surface.h"
#include "../host/sha256.h"
#include <algorithm>
#include <atomic>
#include <memory>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fcntl.h>
#include <string>
#include <sys/file.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <vector>

struct h3_quant_state {
    std::string cache;                 // artifact directory
    bool streaming = false;            // packed weights stay in pinned host memory
    h3_device_buffer activation;       // packed activation codes + maxima + global slot
    h3_device_buffer streamed;         // device copy of a streamed packed weight
    h3_device_buffer dequant_x;        // NVFP4: the activation's dequantized BF16 values
    h3_device_buffer dequant_w;        // NVFP4: a streamed weight's dequantized BF16 values
};

namespace {

constexpr unsigned MAX_PARTIALS = 1024;
constexpr unsigned FAULT_QUANT = 2;    // g->fault index: nonfinite projection input

// Mode names as they appear in artifact names and messages ("fp8", "nvfp4").
const char *mode_name(int mode) { return mode == H3_QUANT_FP8 ? "fp8" : mode == H3_QUANT_NVFP4 ? "nvfp4" : "off"; }

// ---------------------------------------------------------------- packing
// Maximum |x| of BF16 values as the integer maximum of their magnitude bits
// (equal to the float maximum for finite values); a non-finite value sets the
// fault flag and is left out.
__global__ __launch_bounds__(256) void fp8_amax(const uint16_t *x, size_t chunks, unsigned *partials,
                                                unsigned *fault) {
    unsigned best = 0;
    bool bad = false;
    for (size_t c = (size_t)blockIdx.x * 256 + threadIdx.x; c < chunks; c += (size_t)gridDim.x * 256) {
        const u16x8 v = *reinterpret_cast<const u16x8 *>(x + c * 8);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const unsigned mag = v[j] & 0x7fffu;
            if (mag >= 0x7f80u) bad = true;
            else best = max(best, mag);
        }
    }
    if (bad) fault[FAULT_QUANT] = 1u;
    for (int off = 32; off; off >>= 1) best = max(best, (unsigned)__shfl_xor((int)best, off, 64));
    __shared__ unsigned waves[4];
    if (threadIdx.x % 64 == 0) waves[threadIdx.x / 64] = best;
    __syncthreads();
    if (threadIdx.x == 0) partials[blockIdx.x] = max(max(waves[0], waves[1]), max(waves[2], waves[3]));
}

// scale = max(amax / divisor, 1e-20) (IEEE division; 448 for FP8, 2688 for
// NVFP4); global slot {scale, scale * weight_global[0] (an NVFP4 activation)
// or 1, 0, 0} and, for FP8 weights, the scale plane's single value
// (cuda_quant.cuh:36-39, 43).
__global__ __launch_bounds__(256) void fp8_finish(const unsigned *partials, unsigned count, float *global,
                                                  float *scale_slot, float divisor, const float *weight_global) {
    unsigned best = 0;
    for (unsigned i = threadIdx.x; i < count; i += 256) best = max(best, partials[i]);
    for (int off = 32; off; off >>= 1) best = max(best, (unsigned)__shfl_xor((int)best, off, 64));
    __shared__ unsigned waves[4];
    if (threadIdx.x % 64 == 0) waves[threadIdx.x / 64] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        const float amax = bf16_to_f32((uint16_t)max(max(waves[0], waves[1]), max(waves[2], waves[3])));
        const float scale = fmaxf(__fdiv_rn(amax, divisor), 1e-20f);
        global[0] = scale; global[1] = weight_global ? __fmul_rn(scale, weight_global[0]) : 1.f;
        global[2] = 0.f; global[3] = 0.f;
        if (scale_slot) scale_slot[0] = scale;
    }
}

// code = E4M3(x / scale), eight values per thread. The quotient is the IEEE
// one; the encode is v_cvt_pk_fp8_f32 (OCP E4M3, round to nearest even). Its
// saturation differs from the reference's only above 464, and |x| / scale <=
// amax / RN(amax / 448) < 449 here (or x / 1e-20 < 448 when the floor applies).
__global__ __launch_bounds__(256) void fp8_encode(const uint16_t *x, size_t chunks, const float *global,
                                                  uint8_t *codes) {
    const float scale = global[0];
    for (size_t c = (size_t)blockIdx.x * 256 + threadIdx.x; c < chunks; c += (size_t)gridDim.x * 256) {
        const u16x8 v = *reinterpret_cast<const u16x8 *>(x + c * 8);
        float q[8];
#pragma unroll
        for (int j = 0; j < 8; j++) q[j] = __fdiv_rn(bf16_to_f32(v[j]), scale);
        int lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
        lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], lo, true);
        int hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[4], q[5], 0, false);
        hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[6], q[7], hi, true);
        *reinterpret_cast<uint2 *>(codes + c * 8) = make_uint2((unsigned)lo, (unsigned)hi);
    }
}

unsigned pack_grid(size_t chunks) {
    return (unsigned)std::min<size_t>(MAX_PARTIALS, std::max<size_t>(1, (chunks + 255) / 256));
}

// Packs count BF16 values (count % 8 == 0) into codes, with the global slot at
// global and, for weights, the scale plane at scale_slot. partials: MAX_PARTIALS.
int fp8_pack(h3_gpu *g, const uint16_t *x, size_t count, uint8_t *codes, unsigned *partials, float *global,
             float *scale_slot) {
    const size_t chunks = count / 8;
    const unsigned grid = pack_grid(chunks);
    hipLaunchKernelGGL(fp8_amax, dim3(grid), dim3(256), 0, g->compute, x, chunks, partials, g->fault);
    hipLaunchKernelGGL(fp8_finish, dim3(1), dim3(256), 0, g->compute, partials, grid, global, scale_slot, 448.f,
                       (const float *)nullptr);
    hipLaunchKernelGGL(fp8_encode, dim3(grid), dim3(256), 0, g->compute, x, chunks, global, codes);
    return h3_launch_status(g, "FP8 packing");
}

// ---------------------------------------------------------------- NVFP4
// NVFP4 (cuda_quant.cuh:50-72): per 16-column block a UE4M3 scale
// sf = E4M3(max(blockmax / (6 g), 2^-9)) and E2M1 codes of x / (sf g), both
// round to nearest even; scales in cuBLASLt's VEC16 tiled layout. MI355X has no
// NVFP4 matrix path (its FP4 MFMAs take E8M0 scales per 32 values), so the
// projection dequantizes: a code times its block scale has at most 6
// significant bits and is exact in BF16, and y = bf16(gx gw sum (x4 sfx)(w4 sfw))
// runs on the BF16 GEMM with gx gw as its alpha.
__host__ __device__ inline size_t nvfp4_scale_index(unsigned row, unsigned block, unsigned k) {
    const unsigned tiles = (k / 16 + 3) / 4;
    return ((size_t)(row / 128) * tiles + block / 4) * 512 + (row % 32) * 16 + ((row % 128) / 32) * 4 + block % 4;
}

// E2M1 code of |x| (ties to the even code, saturating at 6) with x's sign.
__device__ inline uint8_t f32_to_e2m1(float x) {
    const float a = fabsf(x);
    uint8_t c;
    if (a <= 0.25f) c = 0;
    else if (a < 0.75f) c = 1;
    else if (a <= 1.25f) c = 2;
    else if (a < 1.75f) c = 3;
    else if (a <= 2.5f) c = 4;
    else if (a < 3.5f) c = 5;
    else if (a <= 5.f) c = 6;
    else c = 7;
    return (__builtin_bit_cast(uint32_t, x) >> 28 & 8u) | c;
}

__device__ inline float e2m1_value(unsigned c) {
    const float mag = (c & 7) < 2 ? (c & 7) * 0.5f : __builtin_ldexpf(1.f + ((c & 1) ? 0.5f : 0.f), (int)((c & 6) >> 1) - 1);
    return (c & 8) ? -mag : mag;
}

__device__ inline float e4m3_value(uint8_t c) {
    const unsigned e = (c >> 3) & 15u, m = c & 7u;
    const float mag = e ? __builtin_ldexpf(1.f + m * 0.125f, (int)e - 7) : m * 0.001953125f;
    return (c & 0x80u) ? -mag : mag;
}

// One thread per (row, 16-column block). With codes/scales: the packed
// descriptor (weights at load). With deq: the dequantized BF16 values code * sf
// (activations per call; the global scale goes into the GEMM's alpha).
__global__ __launch_bounds__(256) void nvfp4_pack(const uint16_t *x, unsigned rows, unsigned k, const float *global,
                                                  uint8_t *codes, uint8_t *scales, uint16_t *deq) {
    const size_t b = (size_t)blockIdx.x * 256 + threadIdx.x;
    const unsigned blocks = k / 16;
    if (b >= (size_t)rows * blocks) return;
    const unsigned row = (unsigned)(b / blocks), col = (unsigned)(b % blocks);
    const u16x8 *src = reinterpret_cast<const u16x8 *>(x + (size_t)row * k + col * 16);
    const u16x8 lo = src[0], hi = src[1];
    float v[16], m = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) { v[j] = bf16_to_f32(lo[j]); v[j + 8] = bf16_to_f32(hi[j]); }
#pragma unroll
    for (int j = 0; j < 16; j++) m = fmaxf(m, fabsf(v[j]));
    const float g = global[0];
    const uint8_t sf = f32_to_e4m3(fmaxf(__fdiv_rn(m, __fmul_rn(6.f, g)), 0.001953125f));
    const float sv = e4m3_value(sf), r = __fdiv_rn(1.f, __fmul_rn(sv, g));
    uint8_t c[16];
#pragma unroll
    for (int j = 0; j < 16; j++) c[j] = f32_to_e2m1(__fmul_rn(v[j], r));
    if (codes) {
        uint32_t w0 = 0, w1 = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            w0 |= (uint32_t)(c[2 * j] | c[2 * j + 1] << 4) << (8 * j);
            w1 |= (uint32_t)(c[8 + 2 * j] | c[8 + 2 * j + 1] << 4) << (8 * j);
        }
        *reinterpret_cast<uint2 *>(codes + b * 8) = make_uint2(w0, w1);
        scales[nvfp4_scale_index(row, col, k)] = sf;
    }
    if (deq) {
        u16x8 o0, o1;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            o0[j] = f32_to_bf16(e2m1_value(c[j]) * sv);
            o1[j] = f32_to_bf16(e2m1_value(c[j + 8]) * sv);
        }
        u16x8 *dst = reinterpret_cast<u16x8 *>(deq + (size_t)row * k + col * 16);
        dst[0] = o0; dst[1] = o1;
    }
}

// BF16 values code * sf of a packed NVFP4 descriptor [n, k] (weights).
__global__ __launch_bounds__(256) void nvfp4_dequant(const uint8_t *codes, const uint8_t *scales, unsigned n,
                                                     unsigned k, uint16_t *out) {
    const size_t b = (size_t)blockIdx.x * 256 + threadIdx.x;
    const unsigned blocks = k / 16;
    if (b >= (size_t)n * blocks) return;
    const unsigned row = (unsigned)(b / blocks), col = (unsigned)(b % blocks);
    const float sv = e4m3_value(scales[nvfp4_scale_index(row, col, k)]);
    const uint2 w = *reinterpret_cast<const uint2 *>(codes + b * 8);
    u16x8 o0, o1;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        o0[j] = f32_to_bf16(e2m1_value((w.x >> (4 * j)) & 15u) * sv);
        o1[j] = f32_to_bf16(e2m1_value((w.y >> (4 * j)) & 15u) * sv);
    }
    u16x8 *dst = reinterpret_cast<u16x8 *>(out + (size_t)row * k + col * 16);
    dst[0] = o0; dst[1] = o1;
}

// NVFP4-packs count = rows * k BF16 values: global g from the tensor's max,
// then codes and tiled scales (weights, weight_global null) or the dequantized
// BF16 values (activations, alpha = g * weight_global[0] in global[1]).
int nvfp4_pack_all(h3_gpu *g, const uint16_t *x, unsigned rows, unsigned k, unsigned *partials, float *global,
                   const float *weight_global, uint8_t *codes, uint8_t *scales, uint16_t *deq) {
    const size_t count = (size_t)rows * k, chunks = count / 8;
    const unsigned grid = pack_grid(chunks);
    hipLaunchKernelGGL(fp8_amax, dim3(grid), dim3(256), 0, g->compute, x, chunks, partials, g->fault);
    hipLaunchKernelGGL(fp8_finish, dim3(1), dim3(256), 0, g->compute, partials, grid, global, (float *)nullptr,
                       2688.f, weight_global);
    const size_t blocks = count / 16;
    hipLaunchKernelGGL(nvfp4_pack, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0, g->compute, x, rows, k,
                       (const float *)global, codes, scales, deq);
    return h3_launch_status(g, "NVFP4 packing");
}

// ---------------------------------------------------------------- GEMM
constexpr int TM = 256, TN = 256, TK = 128;          // TK in FP8 bytes
constexpr int ROW = TK;                              // 128 B per LDS row
constexpr int TILE = 256 * ROW;                      // 32 KB per operand tile
constexpr int STAGE = 2 * TILE;
constexpr int GROUP_M = 8;

__device__ inline unsigned swz(unsigned row, unsigned ch) { return ch ^ ((row >> 1) & 7); }

struct Fp8Args {
    uint16_t *y;
    const uint8_t *x, *w;
    const float *sx, *sw;     // device scalars: activation and weight scales
    unsigned m, n, k;
};

__global__ __attribute__((amdgpu_flat_work_group_size(512, 512), amdgpu_waves_per_eu(2, 2)))
void fp8_gemm(Fp8Args a) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    const unsigned tid = threadIdx.x, wave = tid / 64, lane = tid % 64, n32 = lane % 32, hf = lane / 32;
    const unsigned tiles_m = (a.m + TM - 1) / TM, tiles_n = (a.n + TN - 1) / TN;
    const unsigned pid = xcd_remap(blockIdx.x, gridDim.x);
    const unsigned band = pid / (GROUP_M * tiles_n), first_m = band * GROUP_M;
    const unsigned rows_in_band = min(tiles_m - first_m, (unsigned)GROUP_M);
    const unsigned tm = first_m + (pid % (GROUP_M * tiles_n)) % rows_in_band;
    const unsigned tn = (pid % (GROUP_M * tiles_n)) / rows_in_band;
    const unsigned m0 = tm * TM, n0 = tn * TN;
    const unsigned wm = wave / 4, wn = wave % 4;   // rows m0 + wm*128, columns n0 + wn*64
    const unsigned ksteps = a.k / TK;

    f32x16 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f32x16{};

    // 256 rows x 128 B of each operand: 32 groups of 8 rows, 16 B per lane.
    auto load = [&](unsigned kt, int stage) {
        uint8_t *xs = lds + stage * STAGE;
#pragma unroll
        for (unsigned b = wave; b < 32; b += 8) {
            const unsigned row = 8 * b + lane / 8, ph = lane % 8;
            const unsigned gm = min(m0 + row, a.m - 1);
            const uint8_t *xsrc = a.x + (size_t)gm * a.k + kt * TK + swz(row, ph) * 16;
            const uint8_t *wsrc = a.w + (size_t)min(n0 + row, a.n - 1) * a.k + kt * TK + swz(row, ph) * 16;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)xsrc,
                                             (__attribute__((address_space(3))) void *)(xs + b * 1024), 16, 0, 0);
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)wsrc,
                                             (__attribute__((address_space(3))) void *)(xs + TILE + b * 1024), 16, 0, 0);
        }
    };
    // MFMA step s (64 K bytes): lane half hf supplies bytes 32 hf .. 32 hf + 31,
    // chunks 4 s + 2 hf and 4 s + 2 hf + 1 of its row.
    auto fragment = [&](const uint8_t *tile, unsigned row, int s) -> i32x8 {
        const unsigned c0 = 4 * s + 2 * hf;
        const i32x4 lo = *reinterpret_cast<const i32x4 *>(tile + row * ROW + swz(row, c0) * 16);
        const i32x4 hi = *reinterpret_cast<const i32x4 *>(tile + row * ROW + swz(row, c0 + 1) * 16);
        return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };

    load(0, 0);
    wait_vm_loads();
    __syncthreads();
    for (unsigned kt = 0; kt < ksteps; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < ksteps) load(kt + 1, cur ^ 1);
        const uint8_t *xs = lds + cur * STAGE, *ws = xs + TILE;
        i32x8 wf[2][2], xf[2][4];
#pragma unroll
        for (int s = 0; s < 2; s++) {
#pragma unroll
            for (int i = 0; i < 2; i++) wf[s][i] = fragment(ws, wn * 64 + i * 32 + n32, s);
#pragma unroll
            for (int j = 0; j < 4; j++) xf[s][j] = fragment(xs, wm * 128 + j * 32 + n32, s);
        }
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[s][i], xf[s][j], acc[i][j], 0, 0,
                                                                                0, 0, 0, 0);
        wait_vm_loads();
        __syncthreads();
    }

    const float scale = a.sx[0] * a.sw[0];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const unsigned row = m0 + wm * 128 + j * 32 + n32;
        if (row >= a.m) continue;
        uint16_t *dst = a.y + (size_t)row * a.n;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const unsigned col = n0 + wn * 64 + i * 32 + g4 * 8 + hf * 4;
                if (col >= a.n) continue;     // N is a multiple of 128: the last tile may be half full
                u16x4 out;
#pragma unroll
                for (int e = 0; e < 4; e++) out[e] = f32_to_bf16(acc[i][j][g4 * 4 + e] * scale);
                *reinterpret_cast<u16x4 *>(dst + col) = out;
            }
    }
}

// Packed weights have N and K multiples of 128 (h3_gpu_quant_load); any M.
int launch_gemm(h3_gpu *g, const Fp8Args &a) {
    static bool configured = false;
    if (!configured) {
        if (!h3_hip_check(g, hipFuncSetAttribute((const void *)fp8_gemm, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 2 * STAGE), "FP8 GEMM shared memory"))
            return 0;
        configured = true;
    }
    const unsigned tiles = (a.m + TM - 1) / TM * ((a.n + TN - 1) / TN);
    hipEvent_t timing = h3_kernel_timing_begin(g);
    hipLaunchKernelGGL(fp8_gemm, dim3(tiles), dim3(512), 2 * STAGE, g->compute, a);
    h3_kernel_timing_end(g, timing);
    return h3_launch_status(g, "native fp8 projection");
}

// ---------------------------------------------------------------- host helpers
void sha256_of(const void *data, size_t bytes, unsigned char out[32]) {
    h3hip_sha256 s;
    h3hip_sha256_init(&s);
    h3hip_sha256_update(&s, data, bytes);
    h3hip_sha256_final(&s, out);
}

// Little-endian field cursors over a fixed header image.
class HeaderWriter {
public:
    explicit HeaderWriter(unsigned char *p) : p_(p) {}
    HeaderWriter &raw(const void *v, size_t n) { memcpy(p_ + at_, v, n); at_ += n; return *this; }
    HeaderWriter &u32(uint32_t v) { return le(v, 4); }
    HeaderWriter &u64(uint64_t v) { return le(v, 8); }
private:
    HeaderWriter &le(uint64_t v, unsigned n) {
        for (unsigned b = 0; b < n; b++) p_[at_ + b] = (unsigned char)(v >> (8 * b));
        at_ += n;
        return *this;
    }
    unsigned char *p_;
    size_t at_ = 0;
};
class HeaderReader {
public:
    explicit HeaderReader(const unsigned char *p) : p_(p) {}
    HeaderReader &raw(void *v, size_t n) { memcpy(v, p_ + at_, n); at_ += n; return *this; }
    HeaderReader &u32(uint32_t &v) { v = (uint32_t)le(4); return *this; }
    HeaderReader &u64(uint64_t &v) { v = le(8); return *this; }
private:
    uint64_t le(unsigned n) {
        uint64_t v = 0;
        for (unsigned b = n; b-- > 0;) v = v << 8 | p_[at_ + b];
        at_ += n;
        return v;
    }
    const unsigned char *p_;
    size_t at_ = 0;
};

// The H3QWT001 artifact header (the reference's strict format,
// cuda_quant.cuh:169-248): 128 bytes, "H3QWT001", recipe u32, mode u32, n u32,
// k u32, payload bytes u64, scale offset u64, global offset u64, SHA-256 of the
// BF16 source, SHA-256 of the payload, 16 zero bytes.
struct ArtifactHeader {
    static constexpr size_t kSize = 128;
    static constexpr char kMagic[9] = "H3QWT001";
    uint32_t recipe = 0, mode = 0, n = 0, k = 0;
    uint64_t bytes = 0, scale = 0, global = 0;
    unsigned char source_sha[32] = {}, payload_sha[32] = {};

    void encode(unsigned char out[kSize]) const {
        memset(out, 0, kSize);
        HeaderWriter(out).raw(kMagic, 8).u32(recipe).u32(mode).u32(n).u32(k).u64(bytes).u64(scale).u64(global)
            .raw(source_sha, 32).raw(payload_sha, 32);
    }
    // False when the magic or the reserved tail is wrong.
    bool decode(const unsigned char in[kSize]) {
        char magic[8];
        HeaderReader(in).raw(magic, 8).u32(recipe).u32(mode).u32(n).u32(k).u64(bytes).u64(scale).u64(global)
            .raw(source_sha, 32).raw(payload_sha, 32);
        static const unsigned char zero[16] = {};
        return memcmp(magic, kMagic, 8) == 0 && memcmp(in + 112, zero, 16) == 0;
    }
    // Same weight, same packing: every field but the payload digest.
    bool describes_same(const ArtifactHeader &o) const {
        return recipe == o.recipe && mode == o.mode && n == o.n && k == o.k && bytes == o.bytes &&
               scale == o.scale && global == o.global && memcmp(source_sha, o.source_sha, 32) == 0;
    }
};
constexpr char ArtifactHeader::kMagic[9];

// What identifies a source file's contents without reading them: a file whose
// identity differs from an earlier one may have changed since.
struct FileIdentity {
    dev_t dev = 0;
    ino_t ino = 0;
    off_t size = 0;
    struct timespec mtime = {}, ctime = {};

    static FileIdentity of(const struct stat &st) {
        FileIdentity id;
        id.dev = st.st_dev; id.ino = st.st_ino; id.size = st.st_size;
        id.mtime = st.st_mtim; id.ctime = st.st_ctim;
        return id;
    }
    bool still_matches(const char *path) const {
        struct stat st;
        if (stat(path, &st) != 0) return false;
        const FileIdentity now = of(st);
        auto same = [](const timespec &a, const timespec &b) { return a.tv_sec == b.tv_sec && a.tv_nsec == b.tv_nsec; };
        return now.dev == dev && now.ino == ino && now.size == size && same(now.mtime, mtime) && same(now.ctime, ctime);
    }
};

// A read-only mapping of the n x k BF16 source of one packed weight, with the
// identity the file had when it was opened.
class SourceWeight {
public:
    ~SourceWeight() { if (base_ != MAP_FAILED) munmap(base_, length_); }

    bool open(h3_gpu *g, const char *path, uint64_t offset, size_t bytes) {
        const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
        struct stat st;
        const bool in_range = fd >= 0 && fstat(fd, &st) == 0 && offset <= (uint64_t)st.st_size &&
                              bytes <= (uint64_t)st.st_size - offset;
        if (!in_range) {
            if (fd >= 0) close(fd);
            return h3_set_error(g, "invalid quantized source range: %s", path);
        }
        identity_ = FileIdentity::of(st);
        const size_t page = (size_t)sysconf(_SC_PAGESIZE);
        skip_ = (size_t)(offset % page);
        length_ = bytes + skip_;
        base_ = mmap(nullptr, length_, PROT_READ, MAP_PRIVATE, fd, (off_t)(offset - skip_));
        const int map_errno = errno;
        close(fd);
        if (base_ == MAP_FAILED) return h3_set_error(g, "cannot map quantized source: %s", strerror(map_errno));
        bytes_ = bytes;
        return true;
    }
    const uint16_t *values() const { return (const uint16_t *)((const char *)base_ + skip_); }
    void digest(unsigned char out[32]) const { sha256_of(values(), bytes_, out); }
    const FileIdentity &identity() const { return identity_; }

private:
    void *base_ = MAP_FAILED;
    size_t length_ = 0, skip_ = 0, bytes_ = 0;
    FileIdentity identity_;
};

// An exclusive advisory lock on <artifact>.lock, held for one lookup/publish.
class ArtifactLock {
public:
    ~ArtifactLock() { if (fd_ >= 0) { flock(fd_, LOCK_UN); close(fd_); } }
    bool take(const std::string &artifact) {
        fd_ = ::open((artifact + ".lock").c_str(), O_CREAT | O_RDWR | O_CLOEXEC, 0600);
        if (fd_ < 0) return false;
        if (flock(fd_, LOCK_EX) == 0) return true;
        const int e = errno;
        close(fd_);
        fd_ = -1;
        errno = e;
        return false;
    }
private:
    int fd_ = -1;
};

// All of [p, p + n) read from, or written to, fd.
bool read_all(int fd, void *p, size_t n) {
    for (auto *c = (unsigned char *)p; n;) {
        const ssize_t r = read(fd, c, n);
        if (r > 0) { c += r; n -= (size_t)r; }
        else if (r == 0 || errno != EINTR) return false;
    }
    return true;
}
bool write_all(int fd, const void *p, size_t n) {
    for (auto *c = (const unsigned char *)p; n;) {
        const ssize_t r = write(fd, c, n);
        if (r > 0) { c += r; n -= (size_t)r; }
        else if (r == 0 || errno != EINTR) return false;
    }
    return true;
}

// The artifact directory: <cache>/v<recipe>-<mode>-<n>x<k>-<sha256(source) hex>.h3q.
class ArtifactStore {
public:
    enum class Lookup { Absent, Hit, Corrupt, Unreadable };

    explicit ArtifactStore(std::string dir) : dir_(std::move(dir)) {}

    std::string path_for(const ArtifactHeader &h) const {
        char hex[65];
        for (int i = 0; i < 32; i++) snprintf(hex + 2 * i, 3, "%02x", h.source_sha[i]);
        return dir_ + "/v" + std::to_string(h.recipe) + "-" + mode_name((int)h.mode) + "-" + std::to_string(h.n) + "x" +
               std::to_string(h.k) + "-" + hex + ".h3q";
    }

    // Reads the artifact at path into payload (payload.size() bytes) when it
    // holds exactly the weight `want` describes and its payload digest checks.
    Lookup fetch(const std::string &path, const ArtifactHeader &want, std::vector<unsigned char> &payload) const {
        const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd < 0) return errno == ENOENT ? Lookup::Absent : Lookup::Unreadable;
        unsigned char image[ArtifactHeader::kSize];
        ArtifactHeader found;
        struct stat st;
        bool good = fstat(fd, &st) == 0 && (uint64_t)st.st_size == ArtifactHeader::kSize + payload.size() &&
                    read_all(fd, image, sizeof(image)) && found.decode(image) && found.describes_same(want) &&
                    read_all(fd, payload.data(), payload.size());
        close(fd);
        if (good) {
            unsigned char digest[32];
            sha256_of(payload.data(), payload.size(), digest);
            good = memcmp(digest, found.payload_sha, 32) == 0;
        }
        return good ? Lookup::Hit : Lookup::Corrupt;
    }

    // Writes header + payload to a private file beside path, flushes it, and
    // renames it over path, so readers see a whole artifact or none.
    bool publish(const std::string &path, const ArtifactHeader &h, const std::vector<unsigned char> &payload) const {
        unsigned char image[ArtifactHeader::kSize];
        h.encode(image);
        static std::atomic<unsigned> serial{0};
        const std::string part = path + ".part-" + std::to_string((long)getpid()) + "-" + std::to_string(serial++);
        const int fd = ::open(part.c_str(), O_CREAT | O_EXCL | O_WRONLY | O_CLOEXEC, 0644);
        if (fd < 0) return false;
        bool ok = write_all(fd, image, sizeof(image)) && write_all(fd, payload.data(), payload.size()) && fsync(fd) == 0;
        ok = close(fd) == 0 && ok;
        ok = ok && rename(part.c_str(), path.c_str()) == 0;
        if (!ok) {
            const int e = errno;
            unlink(part.c_str());
            errno = e;
        }
        return ok;
    }

private:
    std::string dir_;
};

// Creates dir and its missing parents (mode 0755); true if it is a directory.
bool ensure_directory(const std::string &dir) {
    if (dir.empty()) return false;
    struct stat st;
    if (stat(dir.c_str(), &st) == 0) {
        if (S_ISDIR(st.st_mode)) return true;
        errno = ENOTDIR;
        return false;
    }
    const size_t cut = dir.find_last_of('/');
    if (cut != std::string::npos && cut > 0 && !ensure_directory(dir.substr(0, cut))) return false;
    if (mkdir(dir.c_str(), 0755) == 0 || errno == EEXIST) return stat(dir.c_str(), &st) == 0 && S_ISDIR(st.st_mode);
    return false;
}

// Packs n x k BF16 weights (host) into the descriptor layout on the device and
// copies it back: packed receives `bytes` bytes.
int prepare_packed(h3_gpu *g, const uint16_t *source, uint32_t n, uint32_t k, size_t bytes, size_t scale,
                   size_t global, unsigned char *packed) {
    const int mode = g->quant_mode;
    const size_t count = (size_t)n * k, partial_bytes = MAX_PARTIALS * 4;
    void *staging = nullptr, *device = nullptr, *partials = nullptr;
    int ok = h3_hip_check(g, hipMalloc(&staging, count * 2), "quantization source upload") &&
             h3_hip_check(g, hipMalloc(&device, bytes), "packed weight") &&
             h3_hip_check(g, hipMalloc(&partials, partial_bytes), "packed weight maxima") &&
             h3_hip_check(g, hipMemcpyAsync(staging, source, count * 2, hipMemcpyHostToDevice, g->compute),
                          "quantization source upload") &&
             h3_hip_check(g, hipMemsetAsync(device, 0, bytes, g->compute), "packed weight initialization") &&
             (mode == H3_QUANT_FP8
                  ? fp8_pack(g, (const uint16_t *)staging, count, (uint8_t *)device, (unsigned *)partials,
                             (float *)((char *)device + global), (float *)((char *)device + scale))
                  : nvfp4_pack_all(g, (const uint16_t *)staging, n, k, (unsigned *)partials,
                                   (float *)((char *)device + global), nullptr, (uint8_t *)device,
                                   (uint8_t *)device + scale, nullptr)) &&
             h3_hip_check(g, hipStreamSynchronize(g->compute), "prepare quantized weight") &&
             h3_hip_check(g, hipMemcpy(packed, device, bytes, hipMemcpyDeviceToHost), "download packed artifact");
    if (staging) hipFree(staging);
    if (device) hipFree(device);
    if (partials) hipFree(partials);
    g->stats.h2d_bytes += count * 2;
    g->stats.d2h_bytes += bytes;
    // A non-finite weight raised the quantizer fault: report it now.
    return ok && h3_gpu_synchronize(g);
}

// The BF16 values code * sf of a resident NVFP4 weight, kept beside its
// descriptor for the GEMM.
int nvfp4_resident_dequant(h3_gpu *g, h3_gpu_tensor *t) {
    const size_t count = (size_t)t->quant_n * t->quant_k;
    if (!h3_hip_check(g, hipMalloc(&t->quant_dequant, count * 2 + 256), "NVFP4 dequantized weight")) {
        t->quant_dequant = nullptr;
        return 0;
    }
    const size_t blocks = count / 16;
    hipLaunchKernelGGL(nvfp4_dequant, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0, g->compute,
                       (const uint8_t *)t->data, (const uint8_t *)t->data + t->quant_scale, t->quant_n, t->quant_k,
                       (uint16_t *)t->quant_dequant);
    return h3_launch_status(g, "NVFP4 dequantization") && h3_hip_check(g, hipStreamSynchronize(g->compute), "NVFP4 dequantization");
}

// Why a packed payload cannot be used, or nullptr. FP8: the global slot and
// the scale agree, positive and finite, and no code is an E4M3 NaN (0x7f, 0xff);
// NVFP4: a positive finite global scale and every UE4M3 block scale in 1..126.
const char *payload_defect(int mode, const std::vector<unsigned char> &p, const ArtifactHeader &h) {
    float global_scale;
    memcpy(&global_scale, p.data() + h.global, 4);
    if (!(global_scale > 0.f) || !std::isfinite(global_scale)) return "invalid quantized weight global scale";
    if (mode == H3_QUANT_FP8) {
        float weight_scale;
        memcpy(&weight_scale, p.data() + h.scale, 4);
        if (weight_scale != global_scale) return "invalid FP8 weight scale";
        const unsigned char *codes = p.data();
        const unsigned char *end = codes + (size_t)h.n * h.k;
        return std::any_of(codes, end, [](unsigned char c) { return (c | 0x80) == 0xff; }) ? "nonfinite FP8 weight"
                                                                                           : nullptr;
    }
    const size_t plane = (size_t)(h.n + 127) / 128 * 128 * ((h.k / 16 + 3) / 4 * 4);
    const unsigned char *sf = p.data() + h.scale;
    return std::all_of(sf, sf + plane, [](unsigned char s) { return s >= 1 && s <= 126; })
               ? nullptr
               : "invalid NVFP4 weight block scale";
}

// A packed weight tensor from a checked payload: device-resident, or kept in
// pinned host memory when the context streams its packed weights.
h3_gpu_tensor *packed_tensor(h3_gpu *g, const std::vector<unsigned char> &payload, const ArtifactHeader &h) {
    const h3_gpu_storage storage = g->quant->streaming ? H3_GPU_HOST_PINNED : H3_GPU_DEVICE_ONLY;
    h3_gpu_tensor *t = h3_gpu_tensor_alloc(g, payload.size(), H3_GPU_I8, storage);
    if (!t) return nullptr;
    if (storage == H3_GPU_HOST_PINNED) {
        memcpy(t->data, payload.data(), payload.size());
    } else if (!h3_hip_check(g, hipMemcpy(t->data, payload.data(), payload.size(), hipMemcpyHostToDevice),
                             "packed weight upload")) {
        h3_gpu_tensor_free(t);
        return nullptr;
    } else {
        g->stats.h2d_bytes += payload.size();
    }
    t->elements = (size_t)h.n * h.k;
    t->quant_mode = (int)h.mode; t->quant_n = h.n; t->quant_k = h.k;
    t->quant_scale = h.scale; t->quant_global = h.global;
    if (t->quant_mode == H3_QUANT_NVFP4 && storage == H3_GPU_DEVICE_ONLY && !nvfp4_resident_dequant(g, t)) {
        h3_gpu_tensor_free(t);
        return nullptr;
    }
    return t;
}

// One packed weight through the content-hashed artifact cache. Every load
// hashes its source; the artifact is reused when its header names the same
// source digest and packing and its payload digest checks, and otherwise
// packed on the GPU and published. A corrupt artifact is an error, never
// silently replaced. The source must not change while it is packed or checked.
h3_gpu_tensor *load_through_artifact(h3_gpu *g, const char *path, uint64_t offset, const ArtifactHeader &shape) {
    SourceWeight source;
    if (!source.open(g, path, offset, (size_t)shape.n * shape.k * 2)) return nullptr;
    ArtifactHeader want = shape;
    source.digest(want.source_sha);
    const ArtifactStore store(g->quant->cache);
    const std::string artifact = store.path_for(want);
    std::vector<unsigned char> payload(want.bytes);
    bool hit = false;
    {
        ArtifactLock lock;
        if (!lock.take(artifact)) {
            h3_set_error(g, "cannot lock quantization artifact: %s", strerror(errno));
            return nullptr;
        }
        switch (store.fetch(artifact, want, payload)) {
        case ArtifactStore::Lookup::Hit:
            hit = true;
            break;
        case ArtifactStore::Lookup::Corrupt:
            h3_set_error(g, "corrupt/incompatible quantization artifact %s; remove it and prepare again", artifact.c_str());
            return nullptr;
        case ArtifactStore::Lookup::Unreadable:
            h3_set_error(g, "cannot read quantization artifact: %s", strerror(errno));
            return nullptr;
        case ArtifactStore::Lookup::Absent: {
            if (!prepare_packed(g, source.values(), want.n, want.k, want.bytes, want.scale, want.global, payload.data()))
                return nullptr;
            if (!source.identity().still_matches(path)) {
                h3_set_error(g, "source weight changed during quantization; retry with immutable model files");
                return nullptr;
            }
            ArtifactHeader done = want;
            sha256_of(payload.data(), payload.size(), done.payload_sha);
            if (!store.publish(artifact, done, payload)) {
                h3_set_error(g, "cannot commit quantization artifact: %s", strerror(errno));
                return nullptr;
            }
            break;
        }
        }
    }
    if (!source.identity().still_matches(path)) {
        h3_set_error(g, "source weight changed during artifact verification; retry with immutable model files");
        return nullptr;
    }
    if (const char *defect = payload_defect((int)want.mode, payload, want)) {
        h3_set_error(g, "%s", defect);
        return nullptr;
    }
    h3_gpu_tensor *t = packed_tensor(g, payload, want);
    if (t) (hit ? g->stats.quant_cache_hits : g->stats.quant_cache_misses)++;
    return t;
}

// The four projections of one H3 DiT block, as admission counts them
// (qkv 3 x 7168 x 5376, out 5376 x 7168, fc1 2 x 14336 x 5376, fc2 5376 x 14336).
struct ProjectionShape { uint32_t n, k; };
constexpr ProjectionShape kH3BlockProjections[4] = {{3 * 7168, 5376}, {5376, 7168}, {2 * 14336, 5376}, {5376, 14336}};
// Admission headroom beyond the packed weights and activations: the largest
// conversion operand plus the packed stream buffer, and the activation/output
// scratch (the reference's figures, cuda_quant.cuh:150-151).
constexpr uint64_t kWeightHeadroom = 1ull << 30, kActivationHeadroom = 2ull << 30;

}  // namespace

void h3_quant_destroy(h3_gpu *g) {
    if (!g->quant) return;
    h3_buffer_free(&g->quant->activation);
    h3_buffer_free(&g->quant->streamed);
    h3_buffer_free(&g->quant->dequant_x);
    h3_buffer_free(&g->quant->dequant_w);
    delete g->quant;
    g->quant = nullptr;
}

extern "C" int h3_quant_preflight(int mode, char *error, size_t size) {
    if (!mode) return 1;
    hipDeviceProp_t prop;
    int device = 0;
    if (mode < 1 || mode > 2 || hipGetDevice(&device) != hipSuccess ||
        hipGetDeviceProperties(&prop, device) != hipSuccess) {
        if (error && size) snprintf(error, size, "cannot query HIP quantization device");
        return 0;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        if (error && size)
            snprintf(error, size, "cuda-denoise-quant %s requires gfx950 (MI355X) (device %s)", mode_name(mode),
                     prop.gcnArchName);
        return 0;
    }
    return 1;
}

// gpu.h:44-45 (behaviour of the reference's cuda_quant.cuh:120-162). Admission
// counts whole H3 blocks: `weights` must be a multiple of one block's BF16
// projection bytes, and the packed equivalent plus headroom goes to the
// residency planner, whose answer decides whether packed weights stream.
extern "C" int h3_gpu_quant_configure(h3_gpu *g, int mode, const char *cache, uint64_t weights, uint64_t activations,
                                      int force_stream) {
    if (!g || !h3_quant_preflight(mode, g->error, sizeof(g->error))) return 0;
    if (!mode) return 1;      // BF16 projections never touch packed-weight caches
    if (g->quant_mode) return h3_set_error(g, "quantized GPU context already configured");
    std::string dir;
    if (cache) {
        dir = cache;
    } else {
        const char *home = getenv("HOME");
        dir = std::string(home ? home : ".") + "/.cache/h3/denoise-quant";
    }
    if (!ensure_directory(dir)) return h3_set_error(g, "cannot create quantization cache %s: %s", dir.c_str(), strerror(errno));
    uint64_t source_per_block = 0, packed_per_block = 0;
    for (const ProjectionShape &p : kH3BlockProjections) {
        uint64_t scale, global, bytes;
        h3_weight_packed_size(p.n, p.k, mode, &scale, &global, &bytes);
        source_per_block += 2ull * p.n * p.k;
        packed_per_block += bytes;
    }
    if (weights % source_per_block) return h3_set_error(g, "invalid packed DiT core geometry");
    h3_weight_options o;
    if (!h3_weight_options_read(&o, 0, g->error, sizeof(g->error))) return 0;
    if (force_stream && o.mode == H3_WEIGHTS_RESIDENT)
        return h3_set_error(g, "--ssd-streaming conflicts with CUDA resident weight mode");
    const uint64_t packed_total = weights / source_per_block * packed_per_block;
    const int planned = h3_gpu_plan_weights(g, packed_total + kWeightHeadroom, activations + kActivationHeadroom);
    if (planned < 0) return 0;
    std::unique_ptr<h3_quant_state> state(new (std::nothrow) h3_quant_state());
    if (!state) return h3_set_error(g, "quantization: out of host memory");
    state->cache = std::move(dir);
    state->streaming = planned != 0 || force_stream;
    g->quant = state.release();
    g->quant_mode = mode;
    return 1;
}

// gpu.h:46-47 (behaviour of the reference's cuda_quant.cuh:249-330): a packed
// weight of the configured mode from rows x columns BF16 values at offset of a
// file, through the artifact cache.
extern "C" h3_gpu_tensor *h3_gpu_quant_load(h3_gpu *g, const char *path, uint64_t offset, uint32_t n, uint32_t k) {
    if (!g) return nullptr;
    if (!g->quant_mode || !n || !k || n % 128 || k % 128 || (uint64_t)n * k > UINT32_MAX) {
        h3_set_error(g, "quantized weight shape must be nonzero and a multiple of 128");
        return nullptr;
    }
    if (!path) { h3_set_error(g, "invalid quantized source range: (null)"); return nullptr; }
    ArtifactHeader shape;
    shape.recipe = H3_QUANT_VERSION;
    shape.mode = (uint32_t)g->quant_mode;
    shape.n = n;
    shape.k = k;
    h3_weight_packed_size(n, k, g->quant_mode, &shape.scale, &shape.global, &shape.bytes);
    return load_through_artifact(g, path, offset, shape);
}

// y[rows, n] = FP8 projection of x[rows, k] with a packed weight (reference
// quant_gemm, cuda_quant.cuh:339-398): the activation is packed per call with
// its own tensorwide scale.
int h3_quant_gemm(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in, const h3_gpu_tensor *w, uint32_t rows,
                  uint32_t k, uint32_t n) {
    if (!g->quant || w->quant_k != k || w->quant_n != n || !rows)
        return h3_set_error(g, "quantized projection %ux%ux%u does not match its %ux%u weight", rows, n, k, w->quant_n,
                            w->quant_k);
    const size_t count = (size_t)rows * k;
    const size_t codes = (count + 255) / 256 * 256;
    if (!h3_buffer_reserve(g, &g->quant->activation, codes + MAX_PARTIALS * 4 + 16, "quantized activation"))
        return 0;
    auto *base = (uint8_t *)g->quant->activation.ptr;
    auto *partials = (unsigned *)(base + codes);
    auto *global = (float *)(base + codes + MAX_PARTIALS * 4);
    const uint8_t *weight = (const uint8_t *)w->data;
    if (w->storage != H3_GPU_DEVICE_ONLY) {
        if (!h3_buffer_reserve(g, &g->quant->streamed, w->bytes, "packed weight stream") ||
            !h3_hip_check(g, hipMemcpyAsync(g->quant->streamed.ptr, w->data, w->bytes, hipMemcpyHostToDevice, g->compute),
                          "packed weight stream"))
            return 0;
        g->stats.h2d_bytes += w->bytes;
        g->stats.streamed_bytes += w->bytes;
        weight = (const uint8_t *)g->quant->streamed.ptr;
    }
    if (w->quant_mode == H3_QUANT_NVFP4) {
        // Activation quantized and dequantized in one pass (BF16 code * sf), the
        // weight's BF16 values (resident, or dequantized from the streamed
        // copy), alpha = gx * gw.
        if (!h3_buffer_reserve(g, &g->quant->dequant_x, count * 2 + 256, "NVFP4 activation")) return 0;
        const uint16_t *wdeq = (const uint16_t *)w->quant_dequant;
        if (!wdeq) {
            const size_t wcount = (size_t)n * k;
            if (!h3_buffer_reserve(g, &g->quant->dequant_w, wcount * 2 + 256, "NVFP4 streamed weight")) return 0;
            hipLaunchKernelGGL(nvfp4_dequant, dim3((unsigned)((wcount / 16 + 255) / 256)), dim3(256), 0, g->compute,
                               weight, weight + w->quant_scale, n, k, (uint16_t *)g->quant->dequant_w.ptr);
            if (!h3_launch_status(g, "NVFP4 dequantization")) return 0;
            wdeq = (const uint16_t *)g->quant->dequant_w.ptr;
        }
        if (!nvfp4_pack_all(g, (const uint16_t *)in->data, rows, k, partials, global,
                            (const float *)(weight + w->quant_global), nullptr, nullptr,
                            (uint16_t *)g->quant->dequant_x.ptr) ||
            !h3_gemm_bf16_alpha(g, (uint16_t *)out->data, (const uint16_t *)g->quant->dequant_x.ptr, wdeq, global + 1,
                                rows, k, n))
            return 0;
        g->stats.quant_projection_dispatches++;
        g->stats.linear_dispatches++;
        return 1;
    }
    if (!fp8_pack(g, (const uint16_t *)in->data, count, base, partials, global, nullptr)) return 0;
    Fp8Args a;
    a.y = (uint16_t *)out->data; a.x = base; a.w = weight;
    a.sx = global; a.sw = (const float *)(weight + w->quant_scale);
    a.m = rows; a.n = n; a.k = k;
    if (!launch_gemm(g, a)) return 0;
    g->stats.quant_projection_dispatches++;
    g->stats.linear_dispatches++;
    return 1;
}

// A resident packed weight of the configured mode (FP8 or NVFP4) from n x k
// BF16 device values: the descriptor h3_gpu_quant_load builds, without a file
// or an artifact, for synthetic models and benchmarks.
extern "C" h3_gpu_tensor *h3_hip_quant_weight_from_bf16(h3_gpu *g, const h3_gpu_tensor *w, uint32_t n, uint32_t k) {
    if (!g) return nullptr;
    const int mode = g->quant_mode;
    if (!mode || !n || !k || n % 128 || k % 128 || (uint64_t)n * k > UINT32_MAX) {
        h3_set_error(g, "quantized weight shape must be nonzero and a multiple of 128");
        return nullptr;
    }
    if (!h3_require(g, w, H3_GPU_BF16, (size_t)n * k, "quantized weight source")) return nullptr;
    uint64_t scale, global, bytes;
    h3_weight_packed_size(n, k, mode, &scale, &global, &bytes);
    h3_gpu_tensor *t = h3_gpu_tensor_alloc(g, bytes, H3_GPU_I8, H3_GPU_DEVICE_ONLY);
    if (!t) return nullptr;
    void *partials = nullptr;
    uint8_t *base = (uint8_t *)t->data;
    int ok = h3_hip_check(g, hipMalloc(&partials, MAX_PARTIALS * 4), "quantized weight maxima") &&
             h3_hip_check(g, hipMemsetAsync(t->data, 0, bytes, g->compute), "packed weight initialization") &&
             (mode == H3_QUANT_FP8
                  ? fp8_pack(g, (const uint16_t *)w->data, (size_t)n * k, base, (unsigned *)partials,
                             (float *)(base + global), (float *)(base + scale))
                  : nvfp4_pack_all(g, (const uint16_t *)w->data, n, k, (unsigned *)partials, (float *)(base + global),
                                   nullptr, base, base + scale, nullptr)) &&
             h3_hip_check(g, hipStreamSynchronize(g->compute), "quantized weight");
    if (partials) hipFree(partials);
    if (!ok) { h3_gpu_tensor_free(t); return nullptr; }
    t->elements = (size_t)n * k;
    t->quant_mode = mode; t->quant_n = n; t->quant_k = k; t->quant_scale = scale; t->quant_global = global;
    if (mode == H3_QUANT_NVFP4 && !nvfp4_resident_dequant(g, t)) { h3_gpu_tensor_free(t); return nullptr; }
    return t;
}

// Test entry: SHA-256 of a buffer with the library's own digest.
extern "C" int h3_hip_sha256(const void *data, size_t bytes, uint8_t digest[32]) {
    if ((!data && bytes) || !digest) return 0;
    sha256_of(data, bytes, digest);
    return 1;
}

// Test entry: FP8-pack count BF16 device values (count % 8 == 0) into codes
// (count bytes) and the global slot (4 floats), as a projection input is packed.
extern "C" int h3_hip_fp8_pack(h3_gpu *g, const h3_gpu_tensor *x, h3_gpu_tensor *codes, h3_gpu_tensor *global,
                               size_t count) {
    if (!g || !x || !codes || !global) return 0;
    if (!count || count % 8) return h3_set_error(g, "FP8 pack: count must be a positive multiple of 8");
    if (!h3_require(g, x, H3_GPU_BF16, count, "FP8 pack input") || codes->bytes < count || global->bytes < 16)
        return h3_set_error(g, "FP8 pack: tensors too small");
    void *partials = nullptr;
    int ok = h3_hip_check(g, hipMalloc(&partials, MAX_PARTIALS * 4), "FP8 pack maxima") &&
             fp8_pack(g, (const uint16_t *)x->data, count, (uint8_t *)codes->data, (unsigned *)partials,
                      (float *)global->data, nullptr) &&
             h3_hip_check(g, hipStreamSynchronize(g->compute), "FP8 pack");
    if (partials) hipFree(partials);
    return ok;
}
