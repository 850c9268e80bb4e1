// DiT block elementwise operators for gfx950: AdaLN-modulated RMSNorm, gates,
// Q/K RMSNorm + rotate-half RoPE split, GELU, SwiGLU and the Euler update.
// Arithmetic follows the reference kernels (src/cuda/cuda_kernels.cuh:879-1059,
// 1242-1254); these are HBM-bound, so every kernel moves 16-byte vectors and
// keeps a row (or a head) in registers between its reduction and its output.
#include "common.h"
#include "internal.h"
#include <cmath>

namespace {

constexpr int MAX_CHUNKS = 16;  // 8-element chunks per lane: rows up to 64*16*8 = 8192 wide

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ inline void unpack8(const u16x8 &r, float *f) {
#pragma unroll
    for (int e = 0; e < 8; e++) f[e] = bf16_to_f32(r[e]);
}

struct AdaLNArgs {
    uint16_t *out;          // AdaLN output
    uint16_t *gated;        // gate_adaln: gated residual output (nullptr for plain AdaLN)
    const uint16_t *x;      // AdaLN input, or the residual for gate_adaln
    const uint16_t *branch; // gate_adaln branch
    const uint16_t *weight, *mod, *gate_mod;
    const uint32_t *row_map;
    unsigned rows, width, slots, shift_slot, scale_slot, gate_slot;
    float eps;
};

// One wave per row. MODE 0: AdaLN. MODE 1 (gate_adaln): the row is first gated (residual + branch * gate,
// rounded to BF16 and stored) and the AdaLN then normalizes that BF16 row, as the
// reference's two-kernel composition does (src/cuda/gpu_cuda.cu:1118-1120).
// MODE 2: plain RMSNorm y = bf16(x * rsqrt(mean x^2 + eps) * w), no modulation
// (src/cuda/cuda_kernels.cuh:805-833).
enum { ADALN = 0, GATE_ADALN = 1, RMS_NORM = 2 };
// CH: 16-byte chunks per lane (width <= 512 * CH); the row stays in registers
// as packed BF16 between the reduction and the output pass (exact: the value
// normalized is the BF16 input, or the BF16-rounded gated row).
template <int MODE, int CH>
__global__ __launch_bounds__(256) void adaln_kernel(AdaLNArgs a) {
    constexpr bool GATE = MODE == GATE_ADALN;
    const unsigned wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const unsigned row = blockIdx.x * 4 + wave;
    if (row >= a.rows) return;
    const unsigned chunks = a.width / 8;
    const size_t base = (size_t)row * a.width;
    const size_t mbase = MODE == RMS_NORM ? 0 : (size_t)a.row_map[row] * a.slots * a.width;
    u16x8 raw[CH];
    float sumsq = 0.f;
#pragma unroll
    for (int i = 0; i < CH; i++) {
        const unsigned c = lane + 64 * i;
        if (c >= chunks) break;
        raw[i] = *reinterpret_cast<const u16x8 *>(a.x + base + c * 8);
    }
#pragma unroll
    for (int i = 0; i < CH; i++) {
        const unsigned c = lane + 64 * i;
        if (c >= chunks) break;
        if constexpr (GATE) {
            u16x8 br = *reinterpret_cast<const u16x8 *>(a.branch + base + c * 8);
            u16x8 gr = *reinterpret_cast<const u16x8 *>(a.gate_mod + mbase + (size_t)a.gate_slot * a.width + c * 8);
#pragma unroll
            for (int e = 0; e < 8; e++)
                raw[i][e] = f32_to_bf16(fmaf(bf16_to_f32(br[e]), bf16_to_f32(gr[e]), bf16_to_f32(raw[i][e])));
            *reinterpret_cast<u16x8 *>(a.gated + base + c * 8) = raw[i];
        }
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float v = bf16_to_f32(raw[i][e]);
            sumsq = fmaf(v, v, sumsq);
        }
    }
    const float inv = rsqrtf(wave_sum(sumsq) / (float)a.width + a.eps);
#pragma unroll
    for (int i = 0; i < CH; i++) {
        const unsigned c = lane + 64 * i;
        if (c >= chunks) break;
        u16x8 wr = *reinterpret_cast<const u16x8 *>(a.weight + c * 8);
        u16x8 o;
        if constexpr (MODE == RMS_NORM) {
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = f32_to_bf16(bf16_to_f32(raw[i][e]) * inv * bf16_to_f32(wr[e]));
        } else {
            u16x8 sh = *reinterpret_cast<const u16x8 *>(a.mod + mbase + (size_t)a.shift_slot * a.width + c * 8);
            u16x8 sc = *reinterpret_cast<const u16x8 *>(a.mod + mbase + (size_t)a.scale_slot * a.width + c * 8);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                float normalized = bf16_to_f32(raw[i][e]) * inv * bf16_to_f32(wr[e]);
                o[e] = f32_to_bf16(fmaf(normalized, 1.0f + bf16_to_f32(sc[e]), bf16_to_f32(sh[e])));
            }
        }
        *reinterpret_cast<u16x8 *>(a.out + base + c * 8) = o;
    }
}

// Launch with the smallest chunk count that covers the row.
template <int MODE>
void launch_adaln(h3_gpu *g, const AdaLNArgs &a) {
    const unsigned per_lane = (a.width / 8 + 63) / 64;
    const dim3 grid((a.rows + 3) / 4), block(256);
#define H3_ADALN_CASE(n) case n: hipLaunchKernelGGL((adaln_kernel<MODE, n>), grid, block, 0, g->compute, a); break;
    switch (per_lane) {
        H3_ADALN_CASE(1) H3_ADALN_CASE(2) H3_ADALN_CASE(3) H3_ADALN_CASE(4) H3_ADALN_CASE(5) H3_ADALN_CASE(6)
        H3_ADALN_CASE(7) H3_ADALN_CASE(8) H3_ADALN_CASE(9) H3_ADALN_CASE(10) H3_ADALN_CASE(11) H3_ADALN_CASE(12)
        H3_ADALN_CASE(13) H3_ADALN_CASE(14) H3_ADALN_CASE(15) default: H3_ADALN_CASE(16)
    }
#undef H3_ADALN_CASE
}

// out = bf16(residual + branch * gate), 8 elements per thread.
__global__ __launch_bounds__(256) void gate_kernel(uint16_t *out, const uint16_t *res, const uint16_t *branch,
                                                  const uint16_t *mod, const uint32_t *row_map, unsigned rows,
                                                  unsigned width, unsigned slots, unsigned gate_slot) {
    const size_t chunk = (size_t)blockIdx.x * 256 + threadIdx.x, chunks = (size_t)rows * width / 8;
    if (chunk >= chunks) return;
    const size_t at = chunk * 8;
    const unsigned row = at / width, col = at % width;
    const size_t g = (size_t)row_map[row] * slots * width + (size_t)gate_slot * width + col;
    u16x8 r = *reinterpret_cast<const u16x8 *>(res + at), b = *reinterpret_cast<const u16x8 *>(branch + at);
    u16x8 gv = *reinterpret_cast<const u16x8 *>(mod + g), o;
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = f32_to_bf16(fmaf(bf16_to_f32(b[e]), bf16_to_f32(gv[e]), bf16_to_f32(r[e])));
    *reinterpret_cast<u16x8 *>(out + at) = o;
}

struct QkvArgs {
    uint16_t *q, *k, *v;
    const uint16_t *qkv, *qw, *kw, *cos_t, *sin_t;
    unsigned seq, heads, dim, half;
    float eps;
    int grouped;
};

// One wave per (row, head): optional per-head RMSNorm of Q and K (weights
// qw/kw; null skips the norm), rotate-half RoPE on the first 2*half channels
// (pair d <-> d + half, cos/sin [seq, half]), V copied.
__global__ __launch_bounds__(256) void qkv_rope_kernel(QkvArgs a) {
    __shared__ float stage[4][2][256];
    const unsigned wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const size_t items = (size_t)a.seq * a.heads;
    const size_t item = min((size_t)blockIdx.x * 4 + wave, items - 1);  // tail waves redo the last item
    const bool store = (size_t)blockIdx.x * 4 + wave < items;
    const unsigned row = item / a.heads, head = item % a.heads;
    const size_t inner = (size_t)a.heads * a.dim, row_base = (size_t)row * inner * 3;
    size_t qb = row_base + (size_t)head * a.dim, kb = qb + inner, vb = qb + 2 * inner;
    if (a.grouped) { qb = row_base + (size_t)head * a.dim * 3; kb = qb + a.dim; vb = kb + a.dim; }
    float qv[4], kv[4];
    float qs = 0.f, ks = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        unsigned d = lane + 64 * i;
        qv[i] = kv[i] = 0.f;
        if (d < a.dim) {
            qv[i] = bf16_to_f32(a.qkv[qb + d]);
            kv[i] = bf16_to_f32(a.qkv[kb + d]);
            qs = fmaf(qv[i], qv[i], qs);
            ks = fmaf(kv[i], kv[i], ks);
        }
    }
    float qi = 1.f, ki = 1.f;
    if (a.qw) {
        qi = rsqrtf(wave_sum(qs) / (float)a.dim + a.eps);
        ki = rsqrtf(wave_sum(ks) / (float)a.dim + a.eps);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        unsigned d = lane + 64 * i;
        if (d < a.dim) {
            float wq = a.qw ? bf16_to_f32(a.qw[d]) : 1.f, wk = a.kw ? bf16_to_f32(a.kw[d]) : 1.f;
            qv[i] = a.qw ? qv[i] * qi * wq : qv[i];
            kv[i] = a.qw ? kv[i] * ki * wk : kv[i];
            stage[wave][0][d] = qv[i];
            stage[wave][1][d] = kv[i];
        }
    }
    __syncthreads();  // partner channels come from other lanes through LDS
    if (!store) return;
    const size_t out_base = ((size_t)row * a.heads + head) * a.dim;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        unsigned d = lane + 64 * i;
        if (d >= a.dim) continue;
        float q0 = qv[i], k0 = kv[i];
        if (d < a.half) {
            float c = bf16_to_f32(a.cos_t[(size_t)row * a.half + d]), s = bf16_to_f32(a.sin_t[(size_t)row * a.half + d]);
            float q1 = stage[wave][0][d + a.half], k1 = stage[wave][1][d + a.half];
            q0 = q0 * c - q1 * s;
            k0 = k0 * c - k1 * s;
        } else if (d < 2 * a.half) {
            unsigned p = d - a.half;
            float c = bf16_to_f32(a.cos_t[(size_t)row * a.half + p]), s = bf16_to_f32(a.sin_t[(size_t)row * a.half + p]);
            float q1 = stage[wave][0][p], k1 = stage[wave][1][p];
            q0 = q0 * c + q1 * s;
            k0 = k0 * c + k1 * s;
        }
        a.q[out_base + d] = f32_to_bf16(q0);
        a.k[out_base + d] = f32_to_bf16(k0);
        a.v[out_base + d] = a.qkv[vb + d];
    }
}

// D = 128 with 2 * half <= 128 and half % 8 == 0 (the DiT shapes): 16 lanes per
// (row, head), each owning one 16-byte chunk of Q, K and V. A lane rotating
// chunk c < half/8 pairs it with chunk c + half/8 (and vice versa), loading the
// partner chunk itself (the partner lane loads it at the same time, so the
// second read hits L1); chunks past 2*half pass through. The per-head RMSNorm
// reduces over the 16 lanes with xor shuffles.
__device__ inline float sum16(float v) {
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__global__ __launch_bounds__(256) void qkv_rope_vec(QkvArgs a) {
    const size_t items = (size_t)a.seq * a.heads;
    const size_t item = (size_t)blockIdx.x * 16 + threadIdx.x / 16;
    if (item >= items) return;   // whole 16-lane groups exit together (no barriers here)
    const unsigned c = threadIdx.x % 16;              // chunk: channels 8c .. 8c+7
    const unsigned row = item / a.heads, head = item % a.heads;
    const unsigned hc = a.half / 8;
    const size_t inner = (size_t)a.heads * 128, row_base = (size_t)row * inner * 3;
    size_t qb = row_base + (size_t)head * 128, kb = qb + inner, vb = qb + 2 * inner;
    if (a.grouped) { qb = row_base + (size_t)head * 384; kb = qb + 128; vb = kb + 128; }
    const size_t out = ((size_t)row * a.heads + head) * 128 + c * 8;

    const bool rot = c < 2 * hc;
    const unsigned pc = c < hc ? c + hc : c - hc;     // partner chunk (rotating lanes)
    u16x8 qr = *reinterpret_cast<const u16x8 *>(a.qkv + qb + c * 8);
    u16x8 kr = *reinterpret_cast<const u16x8 *>(a.qkv + kb + c * 8);
    u16x8 vr = *reinterpret_cast<const u16x8 *>(a.qkv + vb + c * 8);
    u16x8 qp = {}, kp = {}, cs = {}, sn = {};
    if (rot) {
        qp = *reinterpret_cast<const u16x8 *>(a.qkv + qb + pc * 8);
        kp = *reinterpret_cast<const u16x8 *>(a.qkv + kb + pc * 8);
        const unsigned pos = (c < hc ? c : pc) * 8;   // pair index of this chunk
        cs = *reinterpret_cast<const u16x8 *>(a.cos_t + (size_t)row * a.half + pos);
        sn = *reinterpret_cast<const u16x8 *>(a.sin_t + (size_t)row * a.half + pos);
    }
    *reinterpret_cast<u16x8 *>(a.v + out) = vr;

    float q[8], k[8], q2[8], k2[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        q[e] = bf16_to_f32(qr[e]); k[e] = bf16_to_f32(kr[e]);
        q2[e] = bf16_to_f32(qp[e]); k2[e] = bf16_to_f32(kp[e]);
    }
    if (a.qw) {
        float qs = 0.f, ks = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) { qs = fmaf(q[e], q[e], qs); ks = fmaf(k[e], k[e], ks); }
        const float qi = rsqrtf(sum16(qs) / 128.0f + a.eps), ki = rsqrtf(sum16(ks) / 128.0f + a.eps);
        u16x8 wq = *reinterpret_cast<const u16x8 *>(a.qw + c * 8), wk = *reinterpret_cast<const u16x8 *>(a.kw + c * 8);
        u16x8 wq2 = {}, wk2 = {};
        if (rot) { wq2 = *reinterpret_cast<const u16x8 *>(a.qw + pc * 8); wk2 = *reinterpret_cast<const u16x8 *>(a.kw + pc * 8); }
#pragma unroll
        for (int e = 0; e < 8; e++) {
            q[e] = q[e] * qi * bf16_to_f32(wq[e]);
            k[e] = k[e] * ki * bf16_to_f32(wk[e]);
            q2[e] = q2[e] * qi * bf16_to_f32(wq2[e]);
            k2[e] = k2[e] * ki * bf16_to_f32(wk2[e]);
        }
    }
    u16x8 qo, ko;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        float qv = q[e], kv = k[e];
        if (rot) {
            const float cv = bf16_to_f32(cs[e]), sv = bf16_to_f32(sn[e]);
            if (c < hc) { qv = q[e] * cv - q2[e] * sv; kv = k[e] * cv - k2[e] * sv; }
            else { qv = q[e] * cv + q2[e] * sv; kv = k[e] * cv + k2[e] * sv; }
        }
        qo[e] = f32_to_bf16(qv);
        ko[e] = f32_to_bf16(kv);
    }
    *reinterpret_cast<u16x8 *>(a.q + out) = qo;
    *reinterpret_cast<u16x8 *>(a.k + out) = ko;
}

__device__ inline float gelu_value(float v, int approximate) {
    if (approximate) {
        float inner = 0.7978845608028654f * (v + 0.044715f * v * v * v);
        return inner <= -10.0f ? 0.0f : inner >= 10.0f ? v : 0.5f * v * (1.0f + tanhf(inner));
    }
    return v <= -10.0f ? 0.0f : v >= 10.0f ? v : 0.5f * v * (1.0f + erff(v * 0.7071067811865475f));
}

__global__ __launch_bounds__(256) void gelu_kernel(uint16_t *out, const uint16_t *in, size_t n, int approximate) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = f32_to_bf16(gelu_value(bf16_to_f32(in[i]), approximate));
}

__global__ __launch_bounds__(256) void swiglu_kernel(uint16_t *out, const uint16_t *fused, unsigned rows, unsigned width) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)rows * width) return;
    size_t row = i / width, col = i % width, base = row * width * 2;
    float gate = bf16_to_f32(fused[base + col]), up = bf16_to_f32(fused[base + width + col]);
    out[i] = f32_to_bf16(gate / (1.0f + expf(-gate)) * up);
}

__global__ __launch_bounds__(256) void euler_kernel(float *sample, const uint16_t *last, const uint16_t *prev, unsigned n,
                                                   float delta, float ratio) {
    unsigned i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float l = bf16_to_f32(last[i]);
    float velocity = fmaf(ratio, l - bf16_to_f32(prev[i]), l);
    sample[i] = fmaf(delta, velocity, sample[i]);
}

unsigned blocks_for(size_t n, unsigned per) { return (unsigned)((n + per - 1) / per); }

int check_map(h3_gpu *g, const h3_gpu_tensor *map, uint32_t rows, const char *what) {
    if (!map || map->dtype != H3_GPU_U32 || map->elements < rows) return h3_set_error(g, "%s row map: need %u U32 entries", what, rows);
    return 1;
}

}  // namespace

// gpu.h:593 (src/cuda/cuda_reference_wrappers.cuh:604): AdaLN of rows starting at
// element `offset` of the input (a multiple of 8 here, for 16-byte rows).
extern "C" int h3_gpu_adaln_bf16_offset(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in, size_t offset,
                                        const h3_gpu_tensor *w, const h3_gpu_tensor *mod, const h3_gpu_tensor *map,
                                        uint32_t rows, uint32_t width, uint32_t slots, uint32_t shift, uint32_t scale,
                                        float eps) {
    size_t n = (size_t)rows * width;
    if (!h3_launch_ready(g)) return 0;
    if (!rows || !width || width % 8 || width > 64 * MAX_CHUNKS * 8 || shift >= slots || scale >= slots || offset % 8)
        return h3_set_error(g, "AdaLN: width and input offset must be multiples of 8, width up to 8192, slots valid");
    if (!in || offset > in->elements) return h3_set_error(g, "AdaLN input offset out of range");
    if (!h3_require(g, in, H3_GPU_BF16, offset + n, "AdaLN input") || !h3_require(g, w, H3_GPU_BF16, width, "AdaLN norm") ||
        !h3_require(g, mod, H3_GPU_BF16, (size_t)slots * width, "AdaLN modulation") || !check_map(g, map, rows, "AdaLN") ||
        !h3_require(g, out, H3_GPU_BF16, n, "AdaLN output"))
        return 0;
    AdaLNArgs a{(uint16_t *)out->data, nullptr, (const uint16_t *)in->data + offset, nullptr, (const uint16_t *)w->data,
                (const uint16_t *)mod->data, nullptr, (const uint32_t *)map->data, rows, width, slots, shift, scale, 0, eps};
    launch_adaln<ADALN>(g, a);
    return h3_launch_status(g, "AdaLN");
}

extern "C" int h3_gpu_adaln_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in, const h3_gpu_tensor *w,
                                 const h3_gpu_tensor *mod, const h3_gpu_tensor *map, uint32_t rows, uint32_t width,
                                 uint32_t slots, uint32_t shift, uint32_t scale, float eps) {
    return h3_gpu_adaln_bf16_offset(g, out, in, 0, w, mod, map, rows, width, slots, shift, scale, eps);
}

// gpu.h:566 (src/cuda/cuda_reference_wrappers.cuh:498, kernel cuda_kernels.cuh:805-833).
extern "C" int h3_gpu_rms_norm_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in, const h3_gpu_tensor *w,
                                    uint32_t rows, uint32_t width, float eps) {
    size_t n = (size_t)rows * width;
    if (!h3_launch_ready(g)) return 0;
    if (!rows || !width || width % 8 || width > 64 * MAX_CHUNKS * 8)
        return h3_set_error(g, "RMSNorm: width must be a multiple of 8 up to 8192");
    if (!h3_require(g, in, H3_GPU_BF16, n, "RMSNorm input") || !h3_require(g, w, H3_GPU_BF16, width, "RMSNorm weight") ||
        !h3_require(g, out, H3_GPU_BF16, n, "RMSNorm output"))
        return 0;
    AdaLNArgs a{(uint16_t *)out->data, nullptr, (const uint16_t *)in->data, nullptr, (const uint16_t *)w->data,
                nullptr, nullptr, nullptr, rows, width, 0, 0, 0, 0, eps};
    launch_adaln<RMS_NORM>(g, a);
    return h3_launch_status(g, "RMSNorm");
}

extern "C" int h3_gpu_gate_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *res, const h3_gpu_tensor *branch,
                                const h3_gpu_tensor *mod, const h3_gpu_tensor *map, uint32_t rows, uint32_t width,
                                uint32_t slots, uint32_t gate_slot) {
    size_t n = (size_t)rows * width;
    if (!h3_launch_ready(g)) return 0;
    if (!rows || !width || width % 8 || gate_slot >= slots) return h3_set_error(g, "gate: width must be a multiple of 8");
    if (!h3_require(g, res, H3_GPU_BF16, n, "gate residual") || !h3_require(g, branch, H3_GPU_BF16, n, "gate branch") ||
        !h3_require(g, mod, H3_GPU_BF16, (size_t)slots * width, "gate modulation") || !check_map(g, map, rows, "gate") ||
        !h3_require(g, out, H3_GPU_BF16, n, "gate output"))
        return 0;
    hipLaunchKernelGGL(gate_kernel, dim3(blocks_for(n / 8, 256)), dim3(256), 0, g->compute, (uint16_t *)out->data,
                       (const uint16_t *)res->data, (const uint16_t *)branch->data, (const uint16_t *)mod->data,
                       (const uint32_t *)map->data, rows, width, slots, gate_slot);
    return h3_launch_status(g, "gate");
}

extern "C" int h3_gpu_gate_adaln_bf16(h3_gpu *g, h3_gpu_tensor *gated, h3_gpu_tensor *out, const h3_gpu_tensor *res,
                                      const h3_gpu_tensor *branch, const h3_gpu_tensor *w, const h3_gpu_tensor *gate_mod,
                                      const h3_gpu_tensor *norm_mod, const h3_gpu_tensor *map, uint32_t rows,
                                      uint32_t width, uint32_t slots, uint32_t gate_slot, uint32_t shift,
                                      uint32_t scale, float eps) {
    size_t n = (size_t)rows * width;
    if (!h3_launch_ready(g)) return 0;
    if (!rows || !width || width % 8 || width > 64 * MAX_CHUNKS * 8 || gate_slot >= slots || shift >= slots || scale >= slots)
        return h3_set_error(g, "gate AdaLN: width must be a multiple of 8 up to 8192 and slots valid");
    if (!h3_require(g, res, H3_GPU_BF16, n, "gate residual") || !h3_require(g, branch, H3_GPU_BF16, n, "gate branch") ||
        !h3_require(g, w, H3_GPU_BF16, width, "AdaLN norm") ||
        !h3_require(g, gate_mod, H3_GPU_BF16, (size_t)slots * width, "gate modulation") ||
        !h3_require(g, norm_mod, H3_GPU_BF16, (size_t)slots * width, "AdaLN modulation") ||
        !check_map(g, map, rows, "gate AdaLN") || !h3_require(g, gated, H3_GPU_BF16, n, "gated residual") ||
        !h3_require(g, out, H3_GPU_BF16, n, "AdaLN output"))
        return 0;
    if (gated == out || gated == branch || out == res || out == branch)
        return h3_set_error(g, "gate AdaLN: outputs must not alias the branch or each other");
    AdaLNArgs a{(uint16_t *)out->data, (uint16_t *)gated->data, (const uint16_t *)res->data, (const uint16_t *)branch->data,
                (const uint16_t *)w->data, (const uint16_t *)norm_mod->data, (const uint16_t *)gate_mod->data,
                (const uint32_t *)map->data, rows, width, slots, shift, scale, gate_slot, eps};
    launch_adaln<GATE_ADALN>(g, a);
    return h3_launch_status(g, "gate AdaLN");
}

static int qkv_rope(h3_gpu *g, h3_gpu_tensor *q, h3_gpu_tensor *k, h3_gpu_tensor *v, const h3_gpu_tensor *qkv,
                    const h3_gpu_tensor *qw, const h3_gpu_tensor *kw, const h3_gpu_tensor *c, const h3_gpu_tensor *s,
                    uint32_t seq, uint32_t heads, uint32_t dim, uint32_t half, float eps, int grouped) {
    size_t n = (size_t)seq * heads * dim;
    if (!h3_launch_ready(g)) return 0;
    if (!seq || !heads || !dim || dim > 256 || half * 2 > dim || (!qw) != (!kw))
        return h3_set_error(g, "QKV RoPE: need dim <= 256, 2*rope_half <= dim, both or neither norm weights");
    if (!h3_require(g, qkv, H3_GPU_BF16, n * 3, "QKV") || !h3_require(g, q, H3_GPU_BF16, n, "Q") ||
        !h3_require(g, k, H3_GPU_BF16, n, "K") || !h3_require(g, v, H3_GPU_BF16, n, "V") ||
        (qw && (!h3_require(g, qw, H3_GPU_BF16, dim, "Q norm") || !h3_require(g, kw, H3_GPU_BF16, dim, "K norm"))) ||
        (half && (!h3_require(g, c, H3_GPU_BF16, (size_t)seq * half, "RoPE cos") ||
                  !h3_require(g, s, H3_GPU_BF16, (size_t)seq * half, "RoPE sin"))))
        return 0;
    QkvArgs a{(uint16_t *)q->data, (uint16_t *)k->data, (uint16_t *)v->data, (const uint16_t *)qkv->data,
              qw ? (const uint16_t *)qw->data : nullptr, kw ? (const uint16_t *)kw->data : nullptr,
              half ? (const uint16_t *)c->data : nullptr, half ? (const uint16_t *)s->data : nullptr,
              seq, heads, dim, half, eps, grouped};
    if (dim == 128 && half % 8 == 0 && half <= 64)
        hipLaunchKernelGGL(qkv_rope_vec, dim3(blocks_for((size_t)seq * heads, 16)), dim3(256), 0, g->compute, a);
    else
        hipLaunchKernelGGL(qkv_rope_kernel, dim3(blocks_for((size_t)seq * heads, 4)), dim3(256), 0, g->compute, a);
    return h3_launch_status(g, "QKV norm/RoPE");
}

extern "C" int h3_gpu_qkv_rope_bf16(h3_gpu *g, h3_gpu_tensor *q, h3_gpu_tensor *k, h3_gpu_tensor *v, const h3_gpu_tensor *qkv,
                                    const h3_gpu_tensor *qw, const h3_gpu_tensor *kw, const h3_gpu_tensor *c,
                                    const h3_gpu_tensor *s, uint32_t seq, uint32_t heads, uint32_t dim, uint32_t half,
                                    float eps) {
    return g && qkv_rope(g, q, k, v, qkv, qw, kw, c, s, seq, heads, dim, half, eps, 0);
}

extern "C" int h3_gpu_grouped_qkv_rope_bf16(h3_gpu *g, h3_gpu_tensor *q, h3_gpu_tensor *k, h3_gpu_tensor *v,
                                            const h3_gpu_tensor *qkv, const h3_gpu_tensor *qw, const h3_gpu_tensor *kw,
                                            const h3_gpu_tensor *c, const h3_gpu_tensor *s, uint32_t seq,
                                            uint32_t heads, uint32_t dim, uint32_t half, float eps) {
    return g && qkv_rope(g, q, k, v, qkv, qw, kw, c, s, seq, heads, dim, half, eps, 1);
}

extern "C" int h3_gpu_gelu_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in, uint32_t n, int approximate) {
    if (!h3_launch_ready(g)) return 0;
    if (!h3_require(g, in, H3_GPU_BF16, n, "GELU input") || !h3_require(g, out, H3_GPU_BF16, n, "GELU output")) return 0;
    if (!n) return 1;
    hipLaunchKernelGGL(gelu_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, g->compute, (uint16_t *)out->data,
                       (const uint16_t *)in->data, (size_t)n, approximate ? 1 : 0);
    return h3_launch_status(g, "GELU");
}

extern "C" int h3_gpu_swiglu_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *fused, uint32_t rows, uint32_t width) {
    if (!h3_launch_ready(g)) return 0;
    size_t n = (size_t)rows * width;
    if (!h3_require(g, fused, H3_GPU_BF16, n * 2, "SwiGLU input") || !h3_require(g, out, H3_GPU_BF16, n, "SwiGLU output"))
        return 0;
    if (!n) return 1;
    hipLaunchKernelGGL(swiglu_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, g->compute, (uint16_t *)out->data,
                       (const uint16_t *)fused->data, rows, width);
    return h3_launch_status(g, "SwiGLU");
}

extern "C" int h3_gpu_euler_bf16(h3_gpu *g, h3_gpu_tensor *sample, size_t offset, const h3_gpu_tensor *last,
                                 const h3_gpu_tensor *previous, uint32_t n, float delta, float ratio) {
    if (!h3_launch_ready(g)) return 0;
    if (!sample || sample->dtype != H3_GPU_F32 || offset > sample->elements || n > sample->elements - offset)
        return h3_set_error(g, "Euler: sample range out of bounds");
    if (!h3_require(g, last, H3_GPU_BF16, n, "Euler last") || !h3_require(g, previous, H3_GPU_BF16, n, "Euler previous"))
        return 0;
    if (!n) return 1;
    hipLaunchKernelGGL(euler_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, g->compute, (float *)sample->data + offset,
                       (const uint16_t *)last->data, (const uint16_t *)previous->data, n, delta, ratio);
    return h3_launch_status(g, "Euler");
}

namespace {
__global__ __launch_bounds__(256) void add_kernel(uint16_t *out, const uint16_t *l, const uint16_t *r, size_t n) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = f32_to_bf16(bf16_to_f32(l[i]) + bf16_to_f32(r[i]));
}
__global__ __launch_bounds__(256) void silu_kernel(uint16_t *out, const uint16_t *in, size_t n) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float v = bf16_to_f32(in[i]);
    out[i] = f32_to_bf16(v / (1.0f + expf(-v)));
}
}  // namespace

// gpu.h:750 (src/cuda/cuda_kernels.cuh:1170-1177).
extern "C" int h3_gpu_add_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *l, const h3_gpu_tensor *r, uint32_t n) {
    if (!h3_launch_ready(g)) return 0;
    if (!h3_require(g, l, H3_GPU_BF16, n, "add left") || !h3_require(g, r, H3_GPU_BF16, n, "add right") ||
        !h3_require(g, out, H3_GPU_BF16, n, "add output"))
        return 0;
    if (!n) return 1;
    hipLaunchKernelGGL(add_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, g->compute, (uint16_t *)out->data,
                       (const uint16_t *)l->data, (const uint16_t *)r->data, (size_t)n);
    return h3_launch_status(g, "add");
}

// gpu.h:564 (src/cuda/cuda_kernels.cuh:796-803).
extern "C" int h3_gpu_silu_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in, uint32_t n) {
    if (!h3_launch_ready(g)) return 0;
    if (!h3_require(g, in, H3_GPU_BF16, n, "SiLU input") || !h3_require(g, out, H3_GPU_BF16, n, "SiLU output")) return 0;
    if (!n) return 1;
    hipLaunchKernelGGL(silu_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, g->compute, (uint16_t *)out->data,
                       (const uint16_t *)in->data, (size_t)n);
    return h3_launch_status(g, "SiLU");
}

namespace {
__global__ __launch_bounds__(256) void cast_f32_bf16_kernel(uint16_t *out, const float *in, size_t n) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = f32_to_bf16(in[i]);
}
__global__ __launch_bounds__(256) void cast_bf16_f32_kernel(float *out, const uint16_t *in, size_t n) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = bf16_to_f32(in[i]);
}
}  // namespace

// gpu.h:329 and gpu.h:331.
extern "C" int h3_gpu_cast_f32_to_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in, uint32_t n) {
    if (!h3_launch_ready(g)) return 0;
    if (!h3_require(g, in, H3_GPU_F32, n, "cast input") || !h3_require(g, out, H3_GPU_BF16, n, "cast output")) return 0;
    if (!n) return 1;
    hipLaunchKernelGGL(cast_f32_bf16_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, g->compute,
                       (uint16_t *)out->data, (const float *)in->data, (size_t)n);
    return h3_launch_status(g, "cast f32->bf16");
}
extern "C" int h3_gpu_cast_bf16_to_f32(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in, uint32_t n) {
    if (!h3_launch_ready(g)) return 0;
    if (!h3_require(g, in, H3_GPU_BF16, n, "cast input") || !h3_require(g, out, H3_GPU_F32, n, "cast output")) return 0;
    if (!n) return 1;
    hipLaunchKernelGGL(cast_bf16_f32_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, g->compute,
                       (float *)out->data, (const uint16_t *)in->data, (size_t)n);
    return h3_launch_status(g, "cast bf16->f32");
}

namespace {
__global__ __launch_bounds__(256) void sub_kernel(uint16_t *out, const uint16_t *l, const uint16_t *r, size_t n) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = f32_to_bf16(bf16_to_f32(l[i]) - bf16_to_f32(r[i]));
}
__global__ __launch_bounds__(256) void silu_mul_kernel(uint16_t *out, const uint16_t *gate, const uint16_t *up, size_t n) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float v = bf16_to_f32(gate[i]);
    out[i] = f32_to_bf16(v / (1.0f + expf(-v)) * bf16_to_f32(up[i]));
}

// In-place per-head RMSNorm, one wave per (row, head), head_dim <= 256.
__global__ __launch_bounds__(256) void head_rms_norm_kernel(uint16_t *t, const uint16_t *w, unsigned seq, unsigned heads,
                                                            unsigned dim, float eps) {
    const size_t items = (size_t)seq * heads, item = (size_t)blockIdx.x * 4 + threadIdx.x / 64;
    const unsigned lane = threadIdx.x % 64;
    if (item >= items) return;
    uint16_t *p = t + item * dim;
    float v[4], ss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        unsigned d = lane + 64 * i;
        v[i] = d < dim ? bf16_to_f32(p[d]) : 0.f;
        ss = fmaf(v[i], v[i], ss);
    }
    const float inv = rsqrtf(wave_sum(ss) / (float)dim + eps);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        unsigned d = lane + 64 * i;
        if (d < dim) p[d] = f32_to_bf16(v[i] * inv * bf16_to_f32(w[d]));
    }
}

// FP32 patch projection with BF16 output: y[map(r), n] = bf16(bias[n] + sum_k x[r,k] W[n,k]),
// k ascending from the bias (the accumulation order of src/cuda/cuda_kernels.cuh:237-265).
// 64x64 output tile per 256 threads, 4x4 outputs per thread, K staged through LDS.
__global__ __launch_bounds__(256) void patch_linear_kernel(uint16_t *out, const float *x, const float *w, const float *bias,
                                                           const uint32_t *map, unsigned out_rows, unsigned m,
                                                           unsigned k, unsigned n) {
    __shared__ float xs[16][65], ws[16][65];
    const unsigned tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    const unsigned row0 = blockIdx.y * 64, col0 = blockIdx.x * 64;
    float acc[4][4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        unsigned c = col0 + tx + 16 * j;
        float b = bias && c < n ? bias[c] : 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i][j] = b;
    }
    for (unsigned k0 = 0; k0 < k; k0 += 16) {
        // 64 rows x 16 k of X and 64 cols x 16 k of W; thread loads 4 of each.
#pragma unroll
        for (int i = 0; i < 4; i++) {
            unsigned r = ty + 16 * i, kk = k0 + tx;
            xs[tx][r] = row0 + r < m && kk < k ? x[(size_t)(row0 + r) * k + kk] : 0.f;
            ws[tx][r] = col0 + r < n && kk < k ? w[(size_t)(col0 + r) * k + kk] : 0.f;
        }
        __syncthreads();
        const unsigned kn = min(16u, k - k0);
        for (unsigned kk = 0; kk < kn; kk++) {
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = fmaf(xs[kk][ty + 16 * i], ws[kk][tx + 16 * j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        unsigned r = row0 + ty + 16 * i;
        if (r >= m) continue;
        unsigned orow = map ? map[r] : r;
        if (orow >= out_rows) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            unsigned c = col0 + tx + 16 * j;
            if (c < n) out[(size_t)orow * n + c] = f32_to_bf16(acc[i][j]);
        }
    }
}

int patch_linear(h3_gpu *g, h3_gpu_tensor *o, size_t oo, const h3_gpu_tensor *x, size_t xo, const h3_gpu_tensor *w,
                 const h3_gpu_tensor *b, const h3_gpu_tensor *map, uint32_t out_rows, uint32_t m, uint32_t k, uint32_t n) {
    if (!h3_launch_ready(g)) return 0;
    if (!o || !x || !w || o->dtype != H3_GPU_BF16 || x->dtype != H3_GPU_F32 || w->dtype != H3_GPU_F32 ||
        xo > x->elements || (size_t)m * k > x->elements - xo || oo > o->elements ||
        (size_t)out_rows * n > o->elements - oo || w->elements < (size_t)k * n ||
        (b && (b->dtype != H3_GPU_F32 || b->elements < n)))
        return h3_set_error(g, "patch linear: F32 input/weight/bias and BF16 output of the stated sizes required");
    if (map && (map->dtype != H3_GPU_U32 || map->elements < m)) return h3_set_error(g, "patch linear row map");
    if (!m || !n) return 1;
    dim3 grid((n + 63) / 64, (m + 63) / 64);
    hipLaunchKernelGGL(patch_linear_kernel, grid, dim3(256), 0, g->compute, (uint16_t *)o->data + oo,
                       (const float *)x->data + xo, (const float *)w->data, b ? (const float *)b->data : nullptr,
                       map ? (const uint32_t *)map->data : nullptr, out_rows, m, k, n);
    g->stats.linear_dispatches++;
    return h3_launch_status(g, "patch linear");
}
}  // namespace

// gpu.h:753 (src/cuda/cuda_kernels.cuh:1179-1185).
extern "C" int h3_gpu_sub_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *l, const h3_gpu_tensor *r, uint32_t n) {
    if (!h3_launch_ready(g)) return 0;
    if (!h3_require(g, l, H3_GPU_BF16, n, "sub left") || !h3_require(g, r, H3_GPU_BF16, n, "sub right") ||
        !h3_require(g, out, H3_GPU_BF16, n, "sub output"))
        return 0;
    if (!n) return 1;
    hipLaunchKernelGGL(sub_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, g->compute, (uint16_t *)out->data,
                       (const uint16_t *)l->data, (const uint16_t *)r->data, (size_t)n);
    return h3_launch_status(g, "sub");
}

// gpu.h:845 (src/cuda/cuda_kernels.cuh:1321-1329).
extern "C" int h3_gpu_silu_mul_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *gate, const h3_gpu_tensor *up,
                                    uint32_t n) {
    if (!h3_launch_ready(g)) return 0;
    if (!h3_require(g, gate, H3_GPU_BF16, n, "SiLU-mul gate") || !h3_require(g, up, H3_GPU_BF16, n, "SiLU-mul up") ||
        !h3_require(g, out, H3_GPU_BF16, n, "SiLU-mul output"))
        return 0;
    if (!n) return 1;
    hipLaunchKernelGGL(silu_mul_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, g->compute, (uint16_t *)out->data,
                       (const uint16_t *)gate->data, (const uint16_t *)up->data, (size_t)n);
    return h3_launch_status(g, "SiLU-mul");
}

// gpu.h:733 (src/cuda/cuda_reference_wrappers.cuh:732, kernel cuda_kernels.cuh:1117-1133).
extern "C" int h3_gpu_head_rms_norm_bf16(h3_gpu *g, h3_gpu_tensor *t, const h3_gpu_tensor *w, uint32_t seq,
                                         uint32_t heads, uint32_t dim, float eps) {
    if (!h3_launch_ready(g)) return 0;
    if (!dim || dim > 256) return h3_set_error(g, "head RMSNorm: head_dim must be 1..256");
    if (!h3_require(g, t, H3_GPU_BF16, (size_t)seq * heads * dim, "head RMSNorm tensor") ||
        !h3_require(g, w, H3_GPU_BF16, dim, "head RMSNorm weight"))
        return 0;
    if (!seq || !heads) return 1;
    hipLaunchKernelGGL(head_rms_norm_kernel, dim3(blocks_for((size_t)seq * heads, 4)), dim3(256), 0, g->compute,
                       (uint16_t *)t->data, (const uint16_t *)w->data, seq, heads, dim, eps);
    return h3_launch_status(g, "head RMSNorm");
}

// gpu.h:307-325 (src/cuda/gpu_cuda.cu:1090-1108): the DiT patch-embedding projection.
extern "C" int h3_gpu_patch_linear_bf16_offset(h3_gpu *g, h3_gpu_tensor *o, size_t oo, const h3_gpu_tensor *x, size_t xo,
                                               const h3_gpu_tensor *w, const h3_gpu_tensor *b, uint32_t m, uint32_t k,
                                               uint32_t n) {
    return patch_linear(g, o, oo, x, xo, w, b, nullptr, m, m, k, n);
}
extern "C" int h3_gpu_patch_linear_bf16(h3_gpu *g, h3_gpu_tensor *o, const h3_gpu_tensor *x, const h3_gpu_tensor *w,
                                        const h3_gpu_tensor *b, uint32_t m, uint32_t k, uint32_t n) {
    return patch_linear(g, o, 0, x, 0, w, b, nullptr, m, m, k, n);
}
extern "C" int h3_gpu_patch_linear_bf16_map(h3_gpu *g, h3_gpu_tensor *o, const h3_gpu_tensor *x, const h3_gpu_tensor *w,
                                            const h3_gpu_tensor *b, const h3_gpu_tensor *map, uint32_t out_rows, uint32_t m,
                                            uint32_t k, uint32_t n) {
    if (!map) return h3_set_error(g, "patch linear: row map required");
    return patch_linear(g, o, 0, x, 0, w, b, map, out_rows, m, k, n);
}
