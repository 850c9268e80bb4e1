// Sage-style quantized attention for gfx950 (D = 128, non-causal).
//
// Arithmetic contract (structure of reference
// src/cuda/cuda_sage2.cu:13-95 and src/cuda/cuda_sage_internal.cuh:68-117):
//  * K is smoothed by its per-(head, channel) mean over the sequence, rounded
//    to BF16 (k' = bf16(k - mean)); the mean cancels in softmax;
//  * Q and K' are quantized to int8 with one fp32 scale per 64-token block per
//    head, scale = fmaf(max|x|, 1/127, 1e-7), code = round-half-away(x / scale);
//  * Q.K^T runs as int8 dot products with int32 accumulation
//    (v_mfma_i32_32x32x32_i8) and is dequantized by q_scale * k_scale;
//  * P = 2^(s - m + log2 448) lies in (0, 448]: the running row max is the
//    per-row scale, and P is rounded to fp8 e4m3;
//  * V is fp8 e4m3 with one scale per (head, channel) = max|v| / 448, and P.V
//    runs on v_mfma_f32_32x32x64_f8f6f4 with fp32 accumulation;
//  * out = (P.V) * v_scale / sum(P), BF16.
// The quantizers are deterministic: every integer code and scale is bit-exact
// against the CPU restatement in oracle/ (which follows the same operation order).
#include "common.h"
#include "internal.h"
#include "attn_common.h"
#include "sage.h"

namespace {
constexpr int D = 128;
constexpr int BN = 64;
constexpr unsigned PARTIAL_ROWS = 256;     // rows per partial K sum
constexpr int K8_STRIDE = D + 16;          // LDS bytes per K row
constexpr int V8_STRIDE = BN + 16;         // LDS bytes per transposed V row
constexpr int K8_BYTES = BN * K8_STRIDE;
constexpr int V8_BYTES = D * V8_STRIDE;
constexpr int SAGE_STAGE = K8_BYTES + V8_BYTES;
constexpr float LOG2_448 = 8.807354922057604f;

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }
}  // namespace

h3_sage_layout h3_sage_plan(unsigned seq, unsigned heads) {
    h3_sage_layout L{};
    L.seq = seq; L.heads = heads;
    L.padded = (seq + 63) / 64 * 64;
    L.blocks = L.padded / 64;
    L.partials = (seq + PARTIAL_ROWS - 1) / PARTIAL_ROWS;
    size_t c = 0;
    auto take = [&](size_t bytes) { size_t at = align256(c); c = at + bytes; return at; };
    L.q8 = take((size_t)heads * L.padded * D);
    L.k8 = take((size_t)heads * L.padded * D);
    L.v8 = take((size_t)heads * L.padded * D);
    L.q_scale = take((size_t)heads * L.blocks * 4);
    L.k_scale = take((size_t)heads * L.blocks * 4);
    L.v_scale = take((size_t)heads * D * 4);
    L.v_recip = take((size_t)heads * D * 4);
    L.k_mean = take((size_t)heads * D * 2);
    L.sums = take((size_t)heads * L.partials * D * 4);
    L.maxima = take((size_t)heads * L.partials * D * 4);
    L.total = align256(c) + 256;
    return L;
}

void h3_sage_workspace_free(h3_sage_workspace *w) {
    if (w->base) hipFree(w->base);
    w->base = nullptr; w->bytes = 0;
}

// ---------------------------------------------------------------- quantizers
// Partial K sums and V maxima: thread = (partial, head, 8-channel chunk), rows
// of the partial summed in row order in fp32.
__global__ __launch_bounds__(256) void sage_reduce_partials(const uint16_t *k, const uint16_t *v, float *sums,
                                                           float *maxima, unsigned seq, unsigned heads,
                                                           unsigned partials, unsigned *fault) {
    unsigned idx = blockIdx.x * 256 + threadIdx.x;
    unsigned chunk = idx % 16, rest = idx / 16, head = rest % heads, p = rest / heads;
    if (p >= partials) return;
    float sum[8], vmax[8];
#pragma unroll
    for (int e = 0; e < 8; e++) { sum[e] = 0.f; vmax[e] = 0.f; }
    bool bad = false;
    unsigned end = min(seq, (p + 1) * PARTIAL_ROWS);
    const size_t stride = (size_t)heads * D;
    const size_t col = (size_t)head * D + chunk * 8;
#pragma unroll 4
    for (unsigned row = p * PARTIAL_ROWS; row < end; row++) {
        u16x8 kx = *reinterpret_cast<const u16x8 *>(k + row * stride + col);
        u16x8 vx = *reinterpret_cast<const u16x8 *>(v + row * stride + col);
        bad |= bf16_vec_nonfinite(kx) | bf16_vec_nonfinite(vx);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float x = bf16_to_f32(kx[e]), y = bf16_to_f32(vx[e]);
            sum[e] = __fadd_rn(sum[e], x);
            vmax[e] = fmaxf(vmax[e], fabsf(y));
        }
    }
    size_t at = ((size_t)head * partials + p) * D + chunk * 8;
#pragma unroll
    for (int e = 0; e < 8; e++) { sums[at + e] = sum[e]; maxima[at + e] = vmax[e]; }
    if (bad) fault[1] = 1u;
}

// Per (head, channel): mean = bf16(sum_p partial_p / seq) (partials in order),
// v_scale = max|v| / 448 and its encode factor 448 / max|v|.
__global__ __launch_bounds__(128) void sage_reduce_finish(const float *sums, const float *maxima, uint16_t *mean,
                                                         float *v_scale, float *v_recip, unsigned seq,
                                                         unsigned partials) {
    unsigned head = blockIdx.x, d = threadIdx.x;
    float sum = 0.f, vmax = 0.f;
    for (unsigned p = 0; p < partials; p++) {
        size_t at = ((size_t)head * partials + p) * D + d;
        sum = __fadd_rn(sum, sums[at]);
        vmax = fmaxf(vmax, maxima[at]);
    }
    mean[head * D + d] = f32_to_bf16(__fdiv_rn(sum, (float)seq));
    v_scale[head * D + d] = __fdiv_rn(vmax, 448.0f);
    v_recip[head * D + d] = vmax > 0.f ? __fdiv_rn(448.0f, vmax) : 0.f;
}

// int8 codes for one 64-row block of one head. Thread t: channel chunk t % 16,
// rows t / 16 + 16 i. KEY subtracts the BF16 mean first (rounded to BF16).
template <bool KEY>
__global__ __launch_bounds__(256) void sage_quant_int8(const uint16_t *x, const uint16_t *mean, int8_t *codes,
                                                      float *scales, unsigned seq, unsigned heads,
                                                      unsigned padded, unsigned *fault) {
    const unsigned blk = blockIdx.x, head = blockIdx.y, t = threadIdx.x;
    const unsigned chunk = t % 16, r0 = t / 16;
    const size_t stride = (size_t)heads * D;
    float val[4][8];
    float amax = 0.f;
    bool bad = false;
    float mu[8];
    if (KEY) {
#pragma unroll
        for (int e = 0; e < 8; e++) mu[e] = bf16_to_f32(mean[head * D + chunk * 8 + e]);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        unsigned row = blk * 64 + r0 + 16 * i;
        u16x8 raw = row < seq ? *reinterpret_cast<const u16x8 *>(x + row * stride + (size_t)head * D + chunk * 8) : u16x8{};
        if (!KEY) bad |= bf16_vec_nonfinite(raw);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float f = bf16_to_f32(raw[e]);
            if (KEY && row < seq) f = bf16_to_f32(f32_to_bf16(__fsub_rn(f, mu[e])));
            val[i][e] = f;
            amax = fmaxf(amax, fabsf(f));
        }
    }
    // Block max: wave reduction, then across the 4 waves through LDS.
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    __shared__ float wave_max[4];
    if (t % 64 == 0) wave_max[t / 64] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(wave_max[0], wave_max[1]), fmaxf(wave_max[2], wave_max[3]));
    const float scale = __fmaf_rn(amax, 1.0f / 127.0f, 1e-7f);
    if (t == 0) scales[head * (padded / 64) + blk] = scale;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        unsigned row = blk * 64 + r0 + 16 * i;
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float qv = __fdiv_rn(val[i][e], scale);
            int c = (int)__fadd_rn(qv, qv >= 0.f ? 0.5f : -0.5f);
            c = c > 127 ? 127 : c < -127 ? -127 : c;
            uint32_t b = (uint32_t)(c & 0xff);
            if (e < 4) lo |= b << (8 * e); else hi |= b << (8 * (e - 4));
        }
        *reinterpret_cast<i32x2 *>(codes + ((size_t)head * padded + row) * D + chunk * 8) = i32x2{(int)lo, (int)hi};
    }
    if (bad) fault[1] = 1u;
}

// fp8 V, transposed to [head, channel, padded] with sage_v_position order per tile.
__global__ __launch_bounds__(256) void sage_pack_v(const uint16_t *v, const float *v_recip, uint8_t *codes,
                                                  unsigned seq, unsigned heads, unsigned padded) {
    __shared__ uint16_t tile[BN][D + 8];
    const unsigned blk = blockIdx.x, head = blockIdx.y, t = threadIdx.x;
    const size_t stride = (size_t)heads * D;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        unsigned c = t + 256 * i, key = c / 16, ch = c % 16, row = blk * BN + key;
        u16x8 raw = row < seq ? *reinterpret_cast<const u16x8 *>(v + row * stride + (size_t)head * D + ch * 8) : u16x8{};
        *reinterpret_cast<u16x8 *>(&tile[key][ch * 8]) = raw;
    }
    __syncthreads();
    const unsigned d = t / 2, half = t % 2;
    const float rcp = v_recip[head * D + d];
    uint32_t w[8];
#pragma unroll
    for (int j = 0; j < 8; j++) w[j] = 0;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        // Position p = half*32 + i holds key mb*32 + (r/4)*8 + half*4 + r%4 with mb = i/16, r = i%16.
        unsigned mb = i / 16, r = i % 16;
        unsigned key = mb * 32 + (r / 4) * 8 + half * 4 + (r % 4);
        uint8_t code = f32_to_e4m3(__fmul_rn(bf16_to_f32(tile[key][d]), rcp));
        w[i / 4] |= (uint32_t)code << (8 * (i % 4));
    }
    uint8_t *dst = codes + ((size_t)head * D + d) * padded + blk * BN + half * 32;
    *reinterpret_cast<i32x4 *>(dst) = i32x4{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
    *reinterpret_cast<i32x4 *>(dst + 16) = i32x4{(int)w[4], (int)w[5], (int)w[6], (int)w[7]};
}

int h3_sage_quantize(h3_gpu *g, const h3_sage_layout &L, char *ws, const uint16_t *q, const uint16_t *k,
                     const uint16_t *v) {
    unsigned threads = L.partials * L.heads * 16;
    hipLaunchKernelGGL(sage_reduce_partials, dim3((threads + 255) / 256), dim3(256), 0, g->compute, k, v,
                       (float *)(ws + L.sums), (float *)(ws + L.maxima), L.seq, L.heads, L.partials, g->fault);
    hipLaunchKernelGGL(sage_reduce_finish, dim3(L.heads), dim3(128), 0, g->compute, (const float *)(ws + L.sums),
                       (const float *)(ws + L.maxima), (uint16_t *)(ws + L.k_mean), (float *)(ws + L.v_scale),
                       (float *)(ws + L.v_recip), L.seq, L.partials);
    hipLaunchKernelGGL(sage_quant_int8<false>, dim3(L.blocks, L.heads), dim3(256), 0, g->compute, q,
                       (const uint16_t *)nullptr, (int8_t *)(ws + L.q8), (float *)(ws + L.q_scale), L.seq, L.heads,
                       L.padded, g->fault);
    hipLaunchKernelGGL(sage_quant_int8<true>, dim3(L.blocks, L.heads), dim3(256), 0, g->compute, k,
                       (const uint16_t *)(ws + L.k_mean), (int8_t *)(ws + L.k8), (float *)(ws + L.k_scale), L.seq,
                       L.heads, L.padded, g->fault);
    hipLaunchKernelGGL(sage_pack_v, dim3(L.blocks, L.heads), dim3(256), 0, g->compute, v,
                       (const float *)(ws + L.v_recip), (uint8_t *)(ws + L.v8), L.seq, L.heads, L.padded);
    return h3_launch_status(g, "Sage quantization");
}

// ---------------------------------------------------------------- attention kernel
namespace {
struct SArgs {
    uint16_t *out;
    const int8_t *q8, *k8;
    const uint8_t *v8;
    const float *q_scale, *k_scale, *v_scale;
    unsigned seq, heads, padded, blocks;
    float scale_log2;
    int head_major;
    const uint32_t *kv_list, *kv_count;
    unsigned list_stride;
    unsigned *fault;
};

template <int WAVES, bool SPARSE>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * WAVES, 64 * WAVES), amdgpu_waves_per_eu(1, 1)))
void sage_attn_kernel(SArgs a) {
    constexpr int T = 64 * WAVES, BM = 64 * WAVES;
    constexpr int KC = (BN * D / 16) / T;        // 16-byte K8 chunks per thread
    constexpr int VC = (D * BN / 16) / T;        // 16-byte V8 chunks per thread
    static_assert(KC * T == BN * D / 16 && VC * T == D * BN / 16, "tile split");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

    const unsigned tid = threadIdx.x, wave = tid / 64, lane = tid % 64, n = lane % 32, hf = lane / 32;
    const unsigned nqb = (a.seq + BM - 1) / BM;
    const unsigned id = xcd_remap(blockIdx.x, gridDim.x);
    const unsigned head = id / nqb, qb = id % nqb, q0 = qb * BM;
    const unsigned ntiles = a.padded / BN;
    const int8_t *qh = a.q8 + (size_t)head * a.padded * D;
    const int8_t *kh = a.k8 + (size_t)head * a.padded * D;
    const uint8_t *vh = a.v8 + (size_t)head * D * a.padded;

    unsigned count;
    const uint32_t *list = nullptr;
    if constexpr (SPARSE) { count = a.kv_count[qb]; list = a.kv_list + (size_t)qb * a.list_stride; }
    else count = ntiles;

    i32x4 qf[2][4];
#pragma unroll
    for (int nb = 0; nb < 2; nb++) {
        unsigned row = min(q0 + wave * 64 + nb * 32 + n, a.padded - 1);
#pragma unroll
        for (int ks = 0; ks < 4; ks++) qf[nb][ks] = *reinterpret_cast<const i32x4 *>(qh + (size_t)row * D + ks * 32 + hf * 16);
    }
    const unsigned qblk = min((q0 + wave * 64) / 64, a.blocks - 1);
    const float qs = a.q_scale[head * a.blocks + qblk] * a.scale_log2;

    f32x16 o[4][2];
#pragma unroll
    for (int md = 0; md < 4; md++)
#pragma unroll
        for (int nb = 0; nb < 2; nb++) o[md][nb] = f32x16{};
    float m[2] = {-1e30f, -1e30f}, l[2] = {0.f, 0.f};

    i32x4 rk[KC], rv[VC];
    auto load_tile = [&](unsigned tile) {
        const bool ok = tile < ntiles;
#pragma unroll
        for (int j = 0; j < KC; j++) {
            unsigned c = tid + T * j, row = c / 8, ch = c % 8;
            rk[j] = ok ? *reinterpret_cast<const i32x4 *>(kh + ((size_t)tile * BN + row) * D + ch * 16) : i32x4{};
        }
#pragma unroll
        for (int j = 0; j < VC; j++) {
            unsigned c = tid + T * j, d = c / 4, ch = c % 4;
            rv[j] = ok ? *reinterpret_cast<const i32x4 *>(vh + (size_t)d * a.padded + (size_t)tile * BN + ch * 16) : i32x4{};
        }
    };
    auto store_tile = [&](int stage) {
        uint8_t *ks = lds + stage * SAGE_STAGE;
        uint8_t *vs = ks + K8_BYTES;
#pragma unroll
        for (int j = 0; j < KC; j++) {
            unsigned c = tid + T * j, row = c / 8, ch = c % 8;
            *reinterpret_cast<i32x4 *>(ks + row * K8_STRIDE + ch * 16) = rk[j];
        }
#pragma unroll
        for (int j = 0; j < VC; j++) {
            unsigned c = tid + T * j, d = c / 4, ch = c % 4;
            *reinterpret_cast<i32x4 *>(vs + d * V8_STRIDE + ch * 16) = rv[j];
        }
    };

    if (count) { load_tile(SPARSE ? list[0] : 0); store_tile(0); }
    __syncthreads();

    for (unsigned it = 0; it < count; it++) {
        const int cur = it & 1;
        const unsigned tile = SPARSE ? list[it] : it;
        const bool more = it + 1 < count;
        if (more) load_tile(SPARSE ? list[it + 1] : it + 1);
        const uint8_t *ks = lds + cur * SAGE_STAGE;
        const uint8_t *vs = ks + K8_BYTES;

        i32x16 si[2][2];
#pragma unroll
        for (int mb = 0; mb < 2; mb++)
#pragma unroll
            for (int nb = 0; nb < 2; nb++) si[mb][nb] = i32x16{};
#pragma unroll
        for (int kstep = 0; kstep < 4; kstep++) {
#pragma unroll
            for (int mb = 0; mb < 2; mb++) {
                i32x4 kf = *reinterpret_cast<const i32x4 *>(ks + (mb * 32 + n) * K8_STRIDE + kstep * 32 + hf * 16);
#pragma unroll
                for (int nb = 0; nb < 2; nb++)
                    si[mb][nb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf, qf[nb][kstep], si[mb][nb], 0, 0, 0);
            }
        }
        const float c = qs * a.k_scale[head * a.blocks + min(tile, a.blocks - 1)];
        f32x16 s[2][2];
#pragma unroll
        for (int mb = 0; mb < 2; mb++)
#pragma unroll
            for (int nb = 0; nb < 2; nb++)
#pragma unroll
                for (int r = 0; r < 16; r++) s[mb][nb][r] = (float)si[mb][nb][r] * c;
        if (tile * BN + BN > a.seq) {
#pragma unroll
            for (int mb = 0; mb < 2; mb++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    unsigned key = tile * BN + mb * 32 + (r / 4) * 8 + hf * 4 + (r % 4);
                    if (key >= a.seq) { s[mb][0][r] = -INFINITY; s[mb][1][r] = -INFINITY; }
                }
        }

        i32x8 pf[2];
#pragma unroll
        for (int nb = 0; nb < 2; nb++) {
            float mx = -INFINITY;
#pragma unroll
            for (int mb = 0; mb < 2; mb++)
#pragma unroll
                for (int r = 0; r < 16; r++) mx = fmaxf(mx, s[mb][nb][r]);
            mx = half_max(mx);
            const float mnew = fmaxf(m[nb], mx);
            const float alpha = exp2f_fast(m[nb] - mnew);
            m[nb] = mnew;
            const float bias = LOG2_448 - mnew;
            float psum = 0.f;
            float p[32];
#pragma unroll
            for (int i = 0; i < 32; i++) {
                p[i] = exp2f_fast(s[i / 16][nb][i % 16] + bias);
                psum += p[i];
            }
#pragma unroll
            for (int w = 0; w < 8; w++) {
                int packed = __builtin_amdgcn_cvt_pk_fp8_f32(p[4 * w], p[4 * w + 1], 0, false);
                packed = __builtin_amdgcn_cvt_pk_fp8_f32(p[4 * w + 2], p[4 * w + 3], packed, true);
                pf[nb][w] = packed;
            }
            l[nb] = fmaf(l[nb], alpha, psum);
#pragma unroll
            for (int md = 0; md < 4; md++) o[md][nb] *= alpha;
        }

#pragma unroll
        for (int md = 0; md < 4; md++) {
            i32x8 vf = *reinterpret_cast<const i32x8 *>(vs + (md * 32 + n) * V8_STRIDE + hf * 32);
#pragma unroll
            for (int nb = 0; nb < 2; nb++)
                o[md][nb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vf, pf[nb], o[md][nb], 0, 0, 0, 0, 0, 0);
        }

        if (more) store_tile(cur ^ 1);
        __syncthreads();
    }

    bool bad = false;
    const float *vsc = a.v_scale + head * D;
#pragma unroll
    for (int nb = 0; nb < 2; nb++) {
        const float total = half_sum(l[nb]);
        const float inv = total > 0.f ? 1.f / total : 0.f;
        const unsigned q = q0 + wave * 64 + nb * 32 + n;
        if (q >= a.seq) continue;
        uint16_t *dst = a.out + (a.head_major ? ((size_t)head * a.seq + q) * D : ((size_t)q * a.heads + head) * D);
#pragma unroll
        for (int md = 0; md < 4; md++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                u16x4 w;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    unsigned d = md * 32 + g4 * 8 + hf * 4 + i;
                    float x = o[md][nb][g4 * 4 + i] * (vsc[d] * inv);
                    bad |= !finite_f32(x);
                    w[i] = f32_to_bf16(x);
                }
                *reinterpret_cast<u16x4 *>(dst + md * 32 + g4 * 8 + hf * 4) = w;
            }
    }
    if (bad) a.fault[0] = 1u;
}

template <int WAVES, bool SPARSE>
int launch_sage(h3_gpu *g, const SArgs &a, unsigned groups) {
    constexpr size_t shared = 2 * SAGE_STAGE;
    hipLaunchKernelGGL((sage_attn_kernel<WAVES, SPARSE>), dim3(groups), dim3(64 * WAVES), shared, g->compute, a);
    return h3_launch_status(g, "Sage attention");
}
}  // namespace

int h3_sage_attention(h3_gpu *g, h3_sage_workspace *w, uint16_t *out, const uint16_t *q, const uint16_t *k,
                      const uint16_t *v, unsigned seq, unsigned heads, float scale, bool head_major,
                      const uint32_t *kv_list, const uint32_t *kv_count, unsigned list_stride) {
    h3_sage_layout L = h3_sage_plan(seq, heads);
    if (w->bytes < L.total) {
        // A previous call may still read the old workspace.
        if (w->base && !h3_hip_check(g, hipStreamSynchronize(g->compute), "Sage workspace fence")) return 0;
        h3_sage_workspace_free(w);
        if (!h3_hip_check(g, hipMalloc(&w->base, L.total), "Sage workspace")) { w->base = nullptr; return 0; }
        w->bytes = L.total;
    }
    char *ws = (char *)w->base;
    if (!h3_sage_quantize(g, L, ws, q, k, v)) return 0;
    SArgs a;
    a.out = out; a.q8 = (const int8_t *)(ws + L.q8); a.k8 = (const int8_t *)(ws + L.k8); a.v8 = (const uint8_t *)(ws + L.v8);
    a.q_scale = (const float *)(ws + L.q_scale); a.k_scale = (const float *)(ws + L.k_scale);
    a.v_scale = (const float *)(ws + L.v_scale);
    a.seq = seq; a.heads = heads; a.padded = L.padded; a.blocks = L.blocks;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.head_major = head_major ? 1 : 0;
    a.kv_list = kv_list; a.kv_count = kv_count; a.list_stride = list_stride; a.fault = g->fault;
    if (kv_list) return launch_sage<2, true>(g, a, (seq + 127) / 128 * heads);
    return launch_sage<4, false>(g, a, (seq + 255) / 256 * heads);
}

extern "C" unsigned h3_hip_sage_v_position(unsigned j) { return sage_v_position(j & 63); }

extern "C" int h3_hip_sage_pack(h3_gpu *g, const h3_gpu_tensor *q, const h3_gpu_tensor *k, const h3_gpu_tensor *v,
                                uint32_t seq, uint32_t heads, h3_gpu_tensor *q8, h3_gpu_tensor *k8, h3_gpu_tensor *v8,
                                h3_gpu_tensor *q_scale, h3_gpu_tensor *k_scale, h3_gpu_tensor *v_scale,
                                h3_gpu_tensor *k_mean) {
    if (!h3_launch_ready(g)) return 0;
    if (!seq || !heads) return h3_set_error(g, "Sage pack: empty shape");
    h3_sage_layout L = h3_sage_plan(seq, heads);
    size_t n = (size_t)seq * heads * D, codes = (size_t)heads * L.padded * D;
    if (!h3_require(g, q, H3_GPU_BF16, n, "Sage Q") || !h3_require(g, k, H3_GPU_BF16, n, "Sage K") ||
        !h3_require(g, v, H3_GPU_BF16, n, "Sage V") || !h3_require(g, q8, H3_GPU_I8, codes, "Sage q8") ||
        !h3_require(g, k8, H3_GPU_I8, codes, "Sage k8") || !h3_require(g, v8, H3_GPU_I8, codes, "Sage v8") ||
        !h3_require(g, q_scale, H3_GPU_F32, (size_t)heads * L.blocks, "Sage q scale") ||
        !h3_require(g, k_scale, H3_GPU_F32, (size_t)heads * L.blocks, "Sage k scale") ||
        !h3_require(g, v_scale, H3_GPU_F32, (size_t)heads * D, "Sage v scale") ||
        !h3_require(g, k_mean, H3_GPU_BF16, (size_t)heads * D, "Sage k mean"))
        return 0;
    char *ws = nullptr;
    if (!h3_hip_check(g, hipMallocAsync((void **)&ws, L.total, g->compute), "Sage pack workspace")) return 0;
    int ok = h3_sage_quantize(g, L, ws, (const uint16_t *)q->data, (const uint16_t *)k->data, (const uint16_t *)v->data);
    auto copy = [&](h3_gpu_tensor *t, size_t off, size_t bytes) {
        return h3_hip_check(g, hipMemcpyAsync(t->data, ws + off, bytes, hipMemcpyDeviceToDevice, g->compute), "Sage pack copy");
    };
    ok = ok && copy(q8, L.q8, codes) && copy(k8, L.k8, codes) && copy(v8, L.v8, codes) &&
         copy(q_scale, L.q_scale, (size_t)heads * L.blocks * 4) && copy(k_scale, L.k_scale, (size_t)heads * L.blocks * 4) &&
         copy(v_scale, L.v_scale, (size_t)heads * D * 4) && copy(k_mean, L.k_mean, (size_t)heads * D * 2);
    hipFreeAsync(ws, g->compute);
    return ok;
}
