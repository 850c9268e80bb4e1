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
//  * out = (P.V) * v_scale / sum(P), BF16, with sum(P) over the fp8 P that
//    enter P.V (a 16x16x128 fp8 MFMA against a lane-selecting ones matrix).
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
    // One byte per (head, 32-query wave) of the attention launch, whatever its
    // workgroup shape: W waves per workgroup pad a head to
    // ceil(seq / 32W) W <= ceil(seq / 32) + W - 1 waves, W <= 12.
    L.retry = take((size_t)heads * ((seq + 31) / 32 + 11));
    L.total = align256(c) + 256;
    return L;
}

void h3_sage_workspace_free(h3_sage_workspace *w) {
    if (w->base) hipFree(w->base);
    w->base = nullptr; w->bytes = 0;
}

// ---------------------------------------------------------------- quantizers
// Partial K sums and V maxima: thread = (partial, head, channel pair), rows of
// the partial summed in row order in fp32. A wave covers one head's 128
// channels, so every row read is one contiguous 256-byte segment.
__global__ __launch_bounds__(256) void sage_reduce_partials(const uint16_t *k, const uint16_t *v, float *sums,
                                                           float *maxima, unsigned seq, unsigned heads,
                                                           unsigned partials, unsigned *fault) {
    const unsigned idx = blockIdx.x * 256 + threadIdx.x;
    const unsigned pair = idx % 64, rest = idx / 64, head = rest % heads, p = rest / heads;
    if (p >= partials) return;
    float s0 = 0.f, s1 = 0.f, m0 = 0.f, m1 = 0.f;
    uint32_t bad = 0;
    const unsigned end = min(seq, (p + 1) * PARTIAL_ROWS);
    const size_t stride = (size_t)heads * D;
    const size_t col = (size_t)head * D + pair * 2;
#pragma unroll 8
    for (unsigned row = p * PARTIAL_ROWS; row < end; row++) {
        const uint32_t kx = *reinterpret_cast<const uint32_t *>(k + row * stride + col);
        const uint32_t vx = *reinterpret_cast<const uint32_t *>(v + row * stride + col);
        bad |= bf16x2_nonfinite(kx) | bf16x2_nonfinite(vx);
        s0 = __fadd_rn(s0, bf16_to_f32((uint16_t)kx));
        s1 = __fadd_rn(s1, bf16_to_f32((uint16_t)(kx >> 16)));
        m0 = fmaxf(m0, fabsf(bf16_to_f32((uint16_t)vx)));
        m1 = fmaxf(m1, fabsf(bf16_to_f32((uint16_t)(vx >> 16))));
    }
    const size_t at = ((size_t)head * partials + p) * D + pair * 2;
    *reinterpret_cast<f32x2 *>(sums + at) = f32x2{s0, s1};
    *reinterpret_cast<f32x2 *>(maxima + at) = f32x2{m0, m1};
    if (bad) fault[1] = 1u;
}

// Per (head, channel): mean = bf16(sum_p partial_p / seq) (partials in order),
// v_scale = max|v| / 448 and its encode factor 448 / max|v|.
__global__ __launch_bounds__(128) void sage_reduce_finish(const float *sums, const float *maxima, uint16_t *mean,
                                                         float *v_scale, float *v_recip, unsigned seq,
                                                         unsigned partials) {
    unsigned head = blockIdx.x, d = threadIdx.x;
    float sum = 0.f, vmax = 0.f;
#pragma unroll 8
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
    // Hardware RNE encode (v_cvt_pk_fp8_f32, OCP e4m3): |v| * 448 / max|v| stays
    // below 464, the first value that would overflow, so it matches the
    // saturating software encoder f32_to_e4m3 bit for bit.
    int w[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        float f[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            // Position p = half*32 + i holds key mb*32 + (r/4)*8 + half*4 + r%4 with mb = i/16, r = i%16.
            const unsigned i = 4 * j + u, mb = i / 16, r = i % 16;
            const unsigned key = mb * 32 + (r / 4) * 8 + half * 4 + (r % 4);
            f[u] = __fmul_rn(bf16_to_f32(tile[key][d]), rcp);
        }
        w[j] = __builtin_amdgcn_cvt_pk_fp8_f32(f[0], f[1], 0, false);
        w[j] = __builtin_amdgcn_cvt_pk_fp8_f32(f[2], f[3], w[j], true);
    }
    uint8_t *dst = codes + ((size_t)head * D + d) * padded + blk * BN + half * 32;
    *reinterpret_cast<i32x4 *>(dst) = i32x4{w[0], w[1], w[2], w[3]};
    *reinterpret_cast<i32x4 *>(dst + 16) = i32x4{w[4], w[5], w[6], w[7]};
}

int h3_sage_quantize(h3_gpu *g, const h3_sage_layout &L, char *ws, const uint16_t *q, const uint16_t *k,
                     const uint16_t *v) {
    unsigned threads = L.partials * L.heads * 64;
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
    int buffered;                           // k8 and v8 below 4 GiB: buffer loads with 32-bit offsets
    uint8_t *retry;                         // per (head, wave): rows the exact launch recomputes
};

constexpr int Q8_TILE = BN * D;             // K8 tile bytes: 64 rows x 128 B
constexpr int V8_TILE = D * BN;             // V8 tile bytes: 128 rows x 64 B
constexpr int SAGE_TILE = Q8_TILE + V8_TILE;
constexpr float P_SLACK = 2.0f;             // log2 units the running max may lag (P <= 448)
// QK^T accumulators start at the bits of the float 1.5 * 2^23: an integer
// dot product s (|s| <= 128 * 127 * 127 < 2^22) added to them leaves the
// exponent alone, so the accumulator read as a float is exactly 1.5 * 2^23 + s
// and needs no int-to-float conversion.
constexpr int MAGIC_BITS = 0x4B400000;
constexpr float MAGIC_F = 12582912.0f;
constexpr int MASKED_BITS = (int)0xFF000000u;   // float -1.7e38: a key past seq
// Largest logit scale c of the fast exponent (1.5 * 2^23 c <= 2^23): its
// rounding bound then stays below 0.7 log2 units.
constexpr float MAGIC_C_MAX = 2.0f / 3.0f;

// 16-byte chunk swizzles of the LDS tiles: each 16-lane group of a
// ds_read_b128 hits 16 distinct 4-bank groups.
__device__ inline unsigned k8_chunk(unsigned key, unsigned ch) { return ch ^ ((key >> 1) & 7); }
__device__ inline unsigned v8_chunk(unsigned d, unsigned ch) { return ch ^ ((d >> 2) & 3); }

// WAVES wavefronts of 32 queries; OCC waves per SIMD overlap softmax with MFMA.
// EXACT: the recomputation launch. It runs only workgroups with a flagged
// wave, computes P's exponent without the biased-accumulator shortcut and
// writes the flagged waves' rows.
template <int WAVES, int OCC, bool SPARSE, bool EXACT = false>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * WAVES, 64 * WAVES), amdgpu_waves_per_eu(OCC, OCC)))
void sage_attn_kernel(SArgs a) {
    constexpr int BM = 32 * WAVES;
    constexpr int BLOCKS = Q8_TILE / 1024;  // 1 KB load blocks per operand tile
    static_assert(Q8_TILE == V8_TILE, "tile split");
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];

    // wave and head are read as uniform values so that LDS destinations and
    // buffer offsets stay scalar.
    const unsigned tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / 64), lane = tid % 64;
    const unsigned n = lane % 32, hf = lane / 32;
    const unsigned nqb = (a.seq + BM - 1) / BM;
    const unsigned id = xcd_remap(blockIdx.x, gridDim.x);
    const unsigned head = __builtin_amdgcn_readfirstlane(id / nqb), qb = __builtin_amdgcn_readfirstlane(id % nqb);
    const unsigned q0 = qb * BM;
    const unsigned ntiles = a.padded / BN;
    uint8_t *const retry = a.retry + ((size_t)head * nqb + qb) * WAVES;
    bool redo = true;                      // EXACT: this wave's rows are recomputed
    if constexpr (EXACT) {
        bool any = false;
#pragma unroll
        for (int w = 0; w < WAVES; w++) any |= __builtin_amdgcn_readfirstlane(retry[w]) != 0;
        if (!any) return;                  // uniform, before any barrier
        redo = __builtin_amdgcn_readfirstlane(retry[wave]) != 0;
    }
    bool failed = false;                   // fast launch: c can exceed MAGIC_C_MAX
    const int8_t *qh = a.q8 + (size_t)head * a.padded * D;
    const int8_t *kh = a.k8 + (size_t)head * a.padded * D;
    const uint8_t *vh = a.v8 + (size_t)head * D * a.padded;

    unsigned count;
    const uint32_t *list = nullptr;
    if constexpr (SPARSE) {
        count = __builtin_amdgcn_readfirstlane(load_uniform(a.kv_count + qb));
        list = a.kv_list + (size_t)qb * a.list_stride;
    } else count = ntiles;

    // Query fragments (B operand of S^T = K Q^T): 4 k-steps of 32 channels.
    i32x4 qf[4];
    const unsigned qrow = min(q0 + wave * 32 + n, a.padded - 1);
#pragma unroll
    for (int ks = 0; ks < 4; ks++) qf[ks] = *reinterpret_cast<const i32x4 *>(qh + (size_t)qrow * D + ks * 32 + hf * 16);
    const unsigned qblk = min((q0 + wave * 32) / 64, a.blocks - 1);
    const float qs = a.q_scale[head * a.blocks + qblk] * a.scale_log2;
    if constexpr (!EXACT) {
        // The largest c this wave's tiles can have: qs times the head's
        // largest key-block scale.
        float kmax = 0.f;
        for (unsigned b = lane; b < a.blocks; b += 64) kmax = fmaxf(kmax, a.k_scale[head * a.blocks + b]);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) kmax = fmaxf(kmax, __shfl_xor(kmax, off, 64));
        failed = __builtin_amdgcn_readfirstlane(qs * kmax > MAGIC_C_MAX ? 1 : 0) != 0;
    }

    f32x16 o[4];
#pragma unroll
    for (int md = 0; md < 4; md++) o[md] = f32x16{};
    // Row sums on a 16x16x128 MFMA: lane l's B operand (its P^T fragment)
    // counts as keys 32 (l / 16) .. + 31 of column l % 16, which is query
    // l % 32 = 16 ((l / 16) % 2) + l % 16. The ones matrix keeps, for output
    // rows 4b .. 4b + 3, the key groups g with b + g even, so every lane's
    // four results hold the full sum of its own query.
    f32x4 lsum = f32x4{};
    float m = -1e30f;
    i32x8 ones;                              // fp8 e4m3 1.0 = 0x38, or 0 where not kept
#pragma unroll
    for (int i = 0; i < 8; i++) ones[i] = (((lane % 16) / 4 + lane / 16) & 1) ? 0 : 0x38383838;

    // Direct global->LDS tile loads, one contiguous KB per wave instruction.
    // Buffered: a uniform byte offset per load plus one lane offset each for
    // K and V (block wave + WAVES i sits 8 WAVES i keys / 16 WAVES i channels
    // further on, with the same swizzle).
    const __amdgpu_buffer_rsrc_t krsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)a.k8, (short)0, (int)(uint32_t)((size_t)a.heads * a.padded * D), 0x00020000);
    const __amdgpu_buffer_rsrc_t vrsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)a.v8, (short)0, (int)(uint32_t)((size_t)a.heads * D * a.padded), 0x00020000);
    const uint32_t koff = (8 * wave + lane / 8) * D + k8_chunk(8 * wave + lane / 8, lane % 8) * 16;
    const uint32_t voff = (16 * wave + lane / 4) * a.padded + v8_chunk(16 * wave + lane / 4, lane % 4) * 16;
    auto load_tile = [&](unsigned tile, int stage, auto buf_only_tag) {
        constexpr bool BUF_ONLY = decltype(buf_only_tag)::value;   // caller checked a.buffered
        const unsigned t = min(tile, ntiles - 1);
        uint8_t *ks = lds + stage * SAGE_TILE;
        uint8_t *vs = ks + Q8_TILE;
        if (BUF_ONLY || a.buffered) {
#pragma unroll
            for (unsigned i = 0; i < (BLOCKS + WAVES - 1) / WAVES; i++) {
                const unsigned b = wave + WAVES * i;
                if (b >= BLOCKS) break;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    krsrc, (__attribute__((address_space(3))) void *)(ks + b * 1024), 16, koff,
                    (unsigned)(((size_t)head * a.padded + (size_t)t * BN + 8 * WAVES * i) * D), 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    vrsrc, (__attribute__((address_space(3))) void *)(vs + b * 1024), 16, voff,
                    (unsigned)(((size_t)head * D + 16 * WAVES * i) * a.padded + (size_t)t * BN), 0, 0);
            }
            return;
        }
#pragma unroll
        for (unsigned b = wave; b < BLOCKS; b += WAVES) {
            unsigned key = 8 * b + lane / 8, ph = lane % 8;
            const int8_t *src = kh + ((size_t)t * BN + key) * D + k8_chunk(key, ph) * 16;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                             (__attribute__((address_space(3))) void *)(ks + b * 1024), 16, 0, 0);
            unsigned d = 16 * b + lane / 4, vp = lane % 4;
            const uint8_t *vsrc = vh + (size_t)d * a.padded + (size_t)t * BN + v8_chunk(d, vp) * 16;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)vsrc,
                                             (__attribute__((address_space(3))) void *)(vs + b * 1024), 16, 0, 0);
        }
    };

    auto process = [&](const uint8_t *ks, const uint8_t *vs, unsigned tile, auto full_tag) {
        constexpr bool FULL = decltype(full_tag)::value;   // every key of the tile < seq
        // Dense kernel: keep the fp8 ones in registers (hipcc otherwise
        // rebuilds them with 7 moves per tile); the sparse kernel has no room.
        if constexpr (!SPARSE) asm volatile("" : "+v"(ones));
        i32x16 si[2];
        {
            i32x16 mg;
#pragma unroll
            for (int r = 0; r < 16; r++) mg[r] = MAGIC_BITS;
            si[0] = mg; si[1] = mg;
        }
        // The QK^T MFMAs issue at raised wave priority: with three waves per
        // SIMD in independent workgroups, the one starting its scores gets
        // them into the matrix pipe ahead of the others' softmax VALU work
        // (1.3% faster; the same around P.V, or in the BF16 kernel, is not).
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int kstep = 0; kstep < 4; kstep++) {
#pragma unroll
            for (int mb = 0; mb < 2; mb++) {
                const unsigned key = mb * 32 + n;
                i32x4 kf = *reinterpret_cast<const i32x4 *>(ks + key * D + k8_chunk(key, kstep * 2 + hf) * 16);
                si[mb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf, qf[kstep], si[mb], 0, 0, 0);
            }
        }
        __builtin_amdgcn_s_setprio(0);
        const float c = qs * load_uniform(a.k_scale + head * a.blocks + min(tile, a.blocks - 1));
        const bool masked = !FULL && tile * BN + BN > a.seq;
        if (masked) {
#pragma unroll
            for (int mb = 0; mb < 2; mb++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    unsigned key = tile * BN + mb * 32 + (r / 4) * 8 + hf * 4 + (r % 4);
                    if (key >= a.seq) si[mb][r] = MASKED_BITS;
                }
        }
        // Integer row max (3-input; the biased accumulators order as the
        // scores do), then one scale.
        int mi0 = max(si[0][0], si[0][1]), mi1 = max(si[1][0], si[1][1]);
#pragma unroll
        for (int r = 2; r < 16; r += 2) {
            mi0 = max(max(mi0, si[0][r]), si[0][r + 1]);
            mi1 = max(max(mi1, si[1][r]), si[1][r + 1]);
        }
        const float mx = (half_max_swap(__builtin_bit_cast(float, max(mi0, mi1))) - MAGIC_F) * c;
        // Fast launch: the exponent below carries the magnitude 1.5 * 2^23 c +
        // |m| and rounds by up to 2^-24 of it; P stays <= 448 (fp8 e4m3 encodes
        // 464 and above as NaN) if the max lags by less than the slack minus
        // twice that. A wave whose c can exceed MAGIC_C_MAX on some tile
        // (scores spread over 10^5 log2 units and more) was flagged for the
        // exact launch at the start.
        float lag_max = P_SLACK;
        if constexpr (!EXACT) lag_max = P_SLACK - fmaf(MAGIC_F, c, fmaf(2.f, fabsf(m), 16.f)) * 0x1p-23f;
        if (__builtin_amdgcn_ballot_w64(mx > m + lag_max)) {
            const float mnew = fmaxf(m, mx);
            const float alpha = exp2f_fast(m - mnew);
            m = mnew;
            lsum *= alpha;
#pragma unroll
            for (int md = 0; md < 4; md++) o[md] *= alpha;
        }
        // P = 2^(s - m + log2 448 - slack) <= 448, rounded to fp8 e4m3. Masked
        // keys (huge negative score) give exactly 0.
        // (1.5 * 2^23 + s) c + bias = s c + log2 448 - slack - m, rounded by at
        // most 2^-24 |bias| (far below the int8 quantization error of s c);
        // exact launch: (F - 1.5 * 2^23) c + log2 448 - slack - m.
        const float bias = EXACT ? LOG2_448 - P_SLACK - m : fmaf(-MAGIC_F, c, LOG2_448 - P_SLACK - m);
        i32x8 pf;
#pragma unroll
        for (int w = 0; w < 8; w++) {
            float p[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int idx = 4 * w + i;
                // Copied to a scalar first: hipcc's bit cast of a vector
                // element lvalue reads element 0.
                const int bits = si[idx / 16][idx % 16];
                const float f = __builtin_bit_cast(float, bits);
                p[i] = exp2f_fast(fmaf(EXACT ? f - MAGIC_F : f, c, bias));
            }
            // The first pack's other word is overwritten by the second, so
            // its old value may be any dead register (p[0]'s own: no copy).
            int packed = __builtin_amdgcn_cvt_pk_fp8_f32(p[0], p[1], __builtin_bit_cast(int, p[0]), false);
            pf[w] = __builtin_amdgcn_cvt_pk_fp8_f32(p[2], p[3], packed, true);
        }
        // O^T[md] += V^T[md] P^T (fp8, K = 64 keys); row sums from ones . P^T.
#pragma unroll
        for (int md = 0; md < 4; md++) {
            const unsigned d = md * 32 + n;
            i32x4 lo = *reinterpret_cast<const i32x4 *>(vs + d * BN + v8_chunk(d, hf * 2) * 16);
            i32x4 hi = *reinterpret_cast<const i32x4 *>(vs + d * BN + v8_chunk(d, hf * 2 + 1) * 16);
            i32x8 vf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            o[md] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vf, pf, o[md], 0, 0, 0, 0, 0, 0);
        }
        lsum = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ones, pf, lsum, 0, 0, 0, 0, 0, 0);
    };

    // Sparse tile ids are wave-uniform and read one iteration ahead (see the
    // BF16 kernel): the id load completes under the tile-load wait.
    unsigned tile = 0, next = 1;
    if constexpr (SPARSE) {
        if (count) tile = __builtin_amdgcn_readfirstlane(load_uniform(list));
        if (count > 1) next = __builtin_amdgcn_readfirstlane(load_uniform(list + 1));
    }
    if (count) load_tile(tile, 0, std::false_type{});
    wait_vm_loads();
    __syncthreads();
    // One tile step. FULL (dense, buffer loads): every key of the tile is
    // below seq, and no masking or global-load code is compiled in; those
    // tiles run in a loop of their own so that its code stays compact.
    auto step = [&](unsigned it, auto full_tag) {
        const int cur = it & 1;
        if (it + 1 < count) load_tile(next, cur ^ 1, full_tag);
        uint32_t later = it + 2;
        if constexpr (SPARSE) later = it + 2 < count ? load_uniform(list + it + 2) : 0u;
        const uint8_t *ks = lds + cur * SAGE_TILE;
        process(ks, ks + Q8_TILE, tile, full_tag);
        wait_vm_loads();
        __syncthreads();
        tile = next;
        next = SPARSE ? __builtin_amdgcn_readfirstlane(later) : later;
    };
    unsigned it0 = 0;
    if constexpr (!SPARSE) {
        if (a.buffered)
            for (const unsigned full = a.seq / BN; it0 < full; it0++) step(it0, std::true_type{});
    }
    for (unsigned it = it0; it < count; it++) step(it, std::false_type{});

    if constexpr (!EXACT) {
        if (lane == 0) retry[wave] = failed ? 1 : 0;
        if (failed) return;                // after the last barrier
    } else if (!redo) {
        return;
    }
    bool bad = false;
    const float *vsc = a.v_scale + head * D;
    const float total = lsum[0];
    const float inv = total > 0.f ? 1.f / total : 0.f;
    const unsigned q = q0 + wave * 32 + n;
    if (q < a.seq) {
        uint16_t *dst = a.out + (a.head_major ? ((size_t)head * a.seq + q) * D : ((size_t)q * a.heads + head) * D);
#pragma unroll
        for (int md = 0; md < 4; md++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                u16x4 w;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    unsigned d = md * 32 + g4 * 8 + hf * 4 + i;
                    float x = o[md][g4 * 4 + i] * (vsc[d] * inv);
                    bad |= !finite_f32(x);
                    w[i] = f32_to_bf16(x);
                }
                *reinterpret_cast<u16x4 *>(dst + md * 32 + g4 * 8 + hf * 4) = w;
            }
    }
    if (bad) a.fault[0] = 1u;
}

// ------------------------------------------------------------ hand-scheduled dense kernel
// sage_pipe: sage_attn_kernel<4, 3, false>'s arithmetic (the same operations
// in the same order, so the two agree bit for bit) at one wave per SIMD:
// four waves of 64 queries (two 32-query blocks b = 0, 1), so every K or V
// fragment read from LDS feeds two MFMAs. The softmax VALU work of one block
// (integer row max, the raise test, 32 exponentials and 16 fp8 packs per
// lane) is longer than the MFMA work of both, so the key sweep is one
// inline-asm block ordered for the VALU: independent chains for the row max,
// and the exponentials software-pipelined over groups of four scores (fmas
// of group k, exponentials of group k - 1, packs of group k - 2), so that no
// instruction waits on the one before it. Per 64-key tile j the MFMA stream is
//   S0(j) | PV1(j-1) | S1(j) | PV0(j)
// (S: 8 int8 MFMAs; PV: 4 fp8 MFMAs and the row-sum MFMA), and block b's
// softmax of tile j runs under the two phases after its scores. Fragment
// registers are double-buffered by tile parity, so the V fragments of tile j
// are read under S0(j) and the K fragments of tile j + 1 a phase or two
// before their MFMAs. Groups of four tiles share a barrier (after phase 2 of
// their last tile); the tiles two groups ahead are loaded in that tile's
// phase 4 into the stage just released. Fragment bases carry the stage (bit
// 15), flipped after every group, so the loop body is one group.
//
// Fixed registers inside the sweep:
//   v[0:31]    scores / P of block 0 (P packed in v[0:7]), v[32:63] block 1;
//   v[64:127]  O^T of block 0 (4 channel blocks of 16), v[128:191] block 1;
//   v[192:207] the biased accumulator start (1.5 * 2^23 as float bits);
//   v[216:219], v[220:223] the row sums of blocks 0 and 1;
//   a[0:63]    K fragments of a tile (set s = tile parity at 32 s; k-step ks,
//              key half mb at 8 ks + 4 mb);
//   a[64:127]  V fragments (set s at 64 + 32 s; channel block md at 8 md);
//   a[128:159] Q fragments (block b, k-step ks); a[160:167] the row-sum ones.
// LDS (128 KB): K tile j of stage s at 32 KB s + 8 KB j, V tile j of stage s
// at 64 KB + 32 KB s + 8 KB j, in sage_attn_kernel's swizzled layouts.
constexpr int SP_GROUP_TILES = 4;
constexpr int SP_STAGE = SP_GROUP_TILES * Q8_TILE;   // 32 KB: the K (or V) tiles of one group
constexpr int SP_LDS = 4 * SP_STAGE;

#define SP_S(b, mb) "v[32*" #b "+16*" #mb ":32*" #b "+16*" #mb "+15]"
#define SP_R(b, i) "v[32*" #b "+" #i "]"
#define SP_P(b) "v[32*" #b ":32*" #b "+7]"
#define SP_O(b, md) "v[64+64*" #b "+16*" #md ":64+64*" #b "+16*" #md "+15]"
#define SP_OR(b, md, e) "v[64+64*" #b "+16*" #md "+" #e "]"
#define SP_L(b) "v[216+4*" #b ":219+4*" #b "]"
#define SP_LR(b, e) "v[216+4*" #b "+" #e "]"
#define SP_K(ks, mb, s) "a[32*" #s "+8*" #ks "+4*" #mb ":32*" #s "+8*" #ks "+4*" #mb "+3]"
#define SP_V(md, s) "a[64+32*" #s "+8*" #md ":71+32*" #s "+8*" #md "]"
#define SP_VH(md, h, s) "a[64+32*" #s "+8*" #md "+4*" #h ":67+32*" #s "+8*" #md "+4*" #h "]"
#define SP_Q(b, ks) "a[128+16*" #b "+4*" #ks ":131+16*" #b "+4*" #ks "]"

// MFMAs (s: the fragment set). Scores start from the biased block.
#define SP_SM(b, ks, mb, s) "v_mfma_i32_32x32x32_i8 " SP_S(b, mb) ", " SP_K(ks, mb, s) ", " SP_Q(b, ks) ", " SP_S(b, mb) "\n"
#define SP_SM0(b, mb, s) "v_mfma_i32_32x32x32_i8 " SP_S(b, mb) ", " SP_K(0, mb, s) ", " SP_Q(b, 0) ", v[192:207]\n"
#define SP_PVM(b, md, s) "v_mfma_f32_32x32x64_f8f6f4 " SP_O(b, md) ", " SP_V(md, s) ", " SP_P(b) ", " SP_O(b, md) "\n"
#define SP_RSM(b) "v_mfma_f32_16x16x128_f8f6f4 " SP_L(b) ", a[160:167], " SP_P(b) ", " SP_L(b) "\n"
#define SP_SMFMA(b, s) SP_SM0(b, 0, s), SP_SM0(b, 1, s), SP_SM(b, 1, 0, s), SP_SM(b, 1, 1, s), SP_SM(b, 2, 0, s),   \
    SP_SM(b, 2, 1, s), SP_SM(b, 3, 0, s), SP_SM(b, 3, 1, s)
#define SP_PVMFMA(b, s) SP_PVM(b, 0, s), SP_PVM(b, 1, s), SP_PVM(b, 2, s), SP_PVM(b, 3, s), SP_RSM(b)
#define SP_NOMFMA8 "", "", "", "", "", "", "", ""
#define SP_NOMFMA5 "", "", "", "", ""
#define SP_NONE8 "", "", "", "", "", "", "", ""
#define SP_NONE5 "", "", "", "", ""
// Phases: MFMA M_k, then the memory slot F_k (LDS reads, tile loads, scale
// loads), then the VALU slot E_k. Issuing the memory instructions ahead of
// the exponentials measured 2% faster than after them.
#define SP_PH8(M0, M1, M2, M3, M4, M5, M6, M7, E0, E1, E2, E3, E4, E5, E6, E7, F0, F1, F2, F3, F4, F5, F6, F7)  \
    M0 F0 E0 M1 F1 E1 M2 F2 E2 M3 F3 E3 M4 F4 E4 M5 F5 E5 M6 F6 E6 M7 F7 E7
#define SP_PH5(M0, M1, M2, M3, M4, E0, E1, E2, E3, E4, F0, F1, F2, F3, F4) M0 F0 E0 M1 F1 E1 M2 F2 E2 M3 F3 E3 M4 F4 E4
#define SP_PH8_EXP(...) SP_PH8(__VA_ARGS__)
#define SP_PH5_EXP(...) SP_PH5(__VA_ARGS__)

// Keys at or past S (last group): score i of block b is key tile*64 + 32 (i / 16)
// + 8 ((i % 16) / 4) + 4 hf + i % 4; lim<J> = S - tile*64 - 4 hf (tile J of
// the group).
#define SP_KEEP(b, i, J)                                                                                          \
    "v_cmp_lt_i32 vcc, 32*((" #i ")/16)+8*(((" #i ")%%16)/4)+((" #i ")%%4), %[lim" #J "]\n"                          \
    "v_cndmask_b32 " SP_R(b, i) ", %[masked], " SP_R(b, i) ", vcc\n"
#define SP_KEEP8(b, i, J) SP_KEEP(b, i, J) SP_KEEP(b, i+1, J) SP_KEEP(b, i+2, J) SP_KEEP(b, i+3, J)               \
    SP_KEEP(b, i+4, J) SP_KEEP(b, i+5, J) SP_KEEP(b, i+6, J) SP_KEEP(b, i+7, J)
#define SP_MASK(b, J) "s_nop 7\n s_nop 7\n s_nop 7\n" SP_KEEP8(b, 0, J) SP_KEEP8(b, 8, J) SP_KEEP8(b, 16, J)         \
    SP_KEEP8(b, 24, J)
#define SP_NOMASK(b, J) ""

// Softmax of block b, first part: c = k_scale(tile) qs (the tile's scale in
// sks<J>); the raise threshold m + (2 - (1.5 * 2^23 c + 2 |m| + 16) 2^-23);
// the integer row max of key half 0 as two chains (u: scores 0-7, x: 8-15).
// The scale register of tile J of a group (tiles alternate sks0, sks1).
#define SP_SKS_0 "sks0"
#define SP_SKS_1 "sks1"
#define SP_SKS_2 "sks0"
#define SP_SKS_3 "sks1"
#define SP_SKS(J) SP_SKS_##J
#define SP_MA(b, J)                                                                                               \
    "v_mul_f32 %[c" #b "], %[" SP_SKS(J) "], %[qs]\n"                                                                 \
    "v_fma_f32 %[t" #b "], |%[rm" #b "]|, 2.0, %[k16]\n"                                                          \
    "v_max_i32 %[u" #b "], " SP_R(b, 0) ", " SP_R(b, 1) "\n"                                                      \
    "v_max_i32 %[x" #b "], " SP_R(b, 8) ", " SP_R(b, 9) "\n"                                                      \
    "v_fmac_f32 %[t" #b "], 0x4b400000, %[c" #b "]\n"                                                             \
    "v_max3_i32 %[u" #b "], %[u" #b "], " SP_R(b, 2) ", " SP_R(b, 3) "\n"                                         \
    "v_max3_i32 %[x" #b "], %[x" #b "], " SP_R(b, 10) ", " SP_R(b, 11) "\n"                                       \
    "v_fma_f32 %[t" #b "], %[t" #b "], %[nk23], 2.0\n"                                                            \
    "v_max3_i32 %[u" #b "], %[u" #b "], " SP_R(b, 4) ", " SP_R(b, 5) "\n"                                         \
    "v_max3_i32 %[x" #b "], %[x" #b "], " SP_R(b, 12) ", " SP_R(b, 13) "\n"                                       \
    "v_add_f32 %[t" #b "], %[rm" #b "], %[t" #b "]\n"                                                             \
    "v_max3_i32 %[u" #b "], %[u" #b "], " SP_R(b, 6) ", " SP_R(b, 7) "\n"                                         \
    "v_max3_i32 %[x" #b "], %[x" #b "], " SP_R(b, 14) ", " SP_R(b, 15) "\n"
// Key half 1 (written by the phase's last MFMA, read a slot later) as two
// chains (w: 16-23, y: 24-31), then the four combined.
#define SP_MB(b)                                                                                                  \
    "v_max_i32 %[w" #b "], " SP_R(b, 16) ", " SP_R(b, 17) "\n"                                                    \
    "v_max_i32 %[y" #b "], " SP_R(b, 24) ", " SP_R(b, 25) "\n"                                                    \
    "v_max3_i32 %[w" #b "], %[w" #b "], " SP_R(b, 18) ", " SP_R(b, 19) "\n"                                       \
    "v_max3_i32 %[y" #b "], %[y" #b "], " SP_R(b, 26) ", " SP_R(b, 27) "\n"                                       \
    "v_max3_i32 %[w" #b "], %[w" #b "], " SP_R(b, 20) ", " SP_R(b, 21) "\n"                                       \
    "v_max3_i32 %[y" #b "], %[y" #b "], " SP_R(b, 28) ", " SP_R(b, 29) "\n"                                       \
    "v_max3_i32 %[w" #b "], %[w" #b "], " SP_R(b, 22) ", " SP_R(b, 23) "\n"                                       \
    "v_max3_i32 %[y" #b "], %[y" #b "], " SP_R(b, 30) ", " SP_R(b, 31) "\n"                                       \
    "v_max3_i32 %[u" #b "], %[u" #b "], %[x" #b "], %[w" #b "]\n"                                                 \
    "v_max_i32 %[u" #b "], %[u" #b "], %[y" #b "]\n"
// Second part: the max over both 32-lane halves, mx = (max - 1.5 * 2^23) c;
// when some lane's mx passes the threshold (rare), m = max(m, mx) and l and
// O^T scale by 2^(m_old - m) (after the block's P.V MFMAs in flight); then
// the bias log2 448 - 2 - m - 1.5 * 2^23 c of the exponents.
#define SP_MC(b, L)                                                                                               \
    "v_mov_b32 %[w" #b "], %[u" #b "]\n"                                                                          \
    "s_nop 1\n"                                                                                                   \
    "v_permlane32_swap_b32 %[u" #b "], %[w" #b "]\n"                                                              \
    "v_max_f32 %[u" #b "], %[u" #b "], %[w" #b "]\n"                                                              \
    "v_add_f32 %[u" #b "], 0xcb400000, %[u" #b "]\n"                                                              \
    "v_mul_f32 %[u" #b "], %[c" #b "], %[u" #b "]\n"                                                              \
    "v_cmp_gt_f32 vcc, %[u" #b "], %[t" #b "]\n"                                                                  \
    "s_cbranch_vccz sp_" #L "_%=\n"                                                                               \
    "s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n"                             \
    "v_max_f32 %[u" #b "], %[rm" #b "], %[u" #b "]\n"                                                             \
    "v_sub_f32 %[w" #b "], %[rm" #b "], %[u" #b "]\n"                                                             \
    "v_exp_f32 %[w" #b "], %[w" #b "]\n"                                                                          \
    "v_mov_b32 %[rm" #b "], %[u" #b "]\n"                                                                         \
    "s_nop 1\n"                                                                                                   \
    "v_mul_f32 " SP_LR(b, 0) ", " SP_LR(b, 0) ", %[w" #b "]\n"                                                    \
    "v_mul_f32 " SP_LR(b, 1) ", " SP_LR(b, 1) ", %[w" #b "]\n"                                                    \
    "v_mul_f32 " SP_LR(b, 2) ", " SP_LR(b, 2) ", %[w" #b "]\n"                                                    \
    "v_mul_f32 " SP_LR(b, 3) ", " SP_LR(b, 3) ", %[w" #b "]\n"                                                    \
    SP_OMUL16(b, 0) SP_OMUL16(b, 1) SP_OMUL16(b, 2) SP_OMUL16(b, 3)                                               \
    "sp_" #L "_%=:\n"                                                                                             \
    "v_sub_f32 %[t" #b "], 0x40d9d5da, %[rm" #b "]\n"                                                             \
    "v_fmac_f32 %[t" #b "], 0xcb400000, %[c" #b "]\n"
#define SP_OMUL(b, md, e) "v_mul_f32 " SP_OR(b, md, e) ", %[w" #b "], " SP_OR(b, md, e) "\n"
#define SP_OMUL16(b, md) SP_OMUL(b, md, 0) SP_OMUL(b, md, 1) SP_OMUL(b, md, 2) SP_OMUL(b, md, 3) SP_OMUL(b, md, 4)   \
    SP_OMUL(b, md, 5) SP_OMUL(b, md, 6) SP_OMUL(b, md, 7) SP_OMUL(b, md, 8) SP_OMUL(b, md, 9) SP_OMUL(b, md, 10)      \
    SP_OMUL(b, md, 11) SP_OMUL(b, md, 12) SP_OMUL(b, md, 13) SP_OMUL(b, md, 14) SP_OMUL(b, md, 15)

// P of score group g (scores 4g .. 4g + 3) of block b: x = fma(s, c, bias)
// in place (F), 2^x in place (E), two fp8 packs into register g (C; the
// scores of g were consumed by an earlier group, or by this one). Steps
// interleave F of group k, E of group k - 1 and C of group k - 2.
#define SP_F(b, g, i) "v_fma_f32 " SP_R(b, 4*g+i) ", " SP_R(b, 4*g+i) ", %[c" #b "], %[t" #b "]\n"
#define SP_E(b, g, i) "v_exp_f32 " SP_R(b, 4*g+i) ", " SP_R(b, 4*g+i) "\n"
#define SP_CL(b, g) "v_cvt_pk_fp8_f32 " SP_R(b, g) ", " SP_R(b, 4*g) ", " SP_R(b, 4*g+1) "\n"
#define SP_CH(b, g) "v_cvt_pk_fp8_f32 " SP_R(b, g) ", " SP_R(b, 4*g+2) ", " SP_R(b, 4*g+3) " op_sel:[0,0,1]\n"
#define SP_F4(b, g) SP_F(b, g, 0) SP_F(b, g, 1) SP_F(b, g, 2) SP_F(b, g, 3)
#define SP_FE(b, f, e) SP_F(b, f, 0) SP_E(b, e, 0) SP_F(b, f, 1) SP_E(b, e, 1) SP_F(b, f, 2) SP_E(b, e, 2)           \
    SP_F(b, f, 3) SP_E(b, e, 3)
#define SP_FECA(b, f, e, c) SP_F(b, f, 0) SP_E(b, e, 0) SP_F(b, f, 1) SP_E(b, e, 1) SP_CL(b, c)
#define SP_FECB(b, f, e, c) SP_F(b, f, 2) SP_E(b, e, 2) SP_F(b, f, 3) SP_E(b, e, 3) SP_CH(b, c)
#define SP_FEC(b, f, e, c) SP_FECA(b, f, e, c) SP_FECB(b, f, e, c)
#define SP_EC(b, e, c) SP_E(b, e, 0) SP_E(b, e, 1) SP_CL(b, c) SP_E(b, e, 2) SP_E(b, e, 3) SP_CH(b, c)
#define SP_C(b, c) SP_CL(b, c) SP_CH(b, c)

// Block b's softmax as 13 slot strings (tile J, its scale in sks<J>): 5 under
// a PV phase, then 8 under an S phase; the P.V MFMAs that read P follow after
// two wait states. MSK: SP_MASK / SP_NOMASK; L: a label unique in the block.
#define SP_SOFT_A(b, MSK, J, L) MSK(b, J) SP_MA(b, J), SP_MB(b) SP_MC(b, L), SP_F4(b, 0) SP_FE(b, 1, 0),              \
    SP_FEC(b, 2, 1, 0), SP_FEC(b, 3, 2, 1)
#define SP_SOFT_B(b) SP_FECA(b, 4, 3, 2), SP_FECB(b, 4, 3, 2), SP_FECA(b, 5, 4, 3), SP_FECB(b, 5, 4, 3),              \
    SP_FEC(b, 6, 5, 4), SP_FEC(b, 7, 6, 5), SP_EC(b, 7, 6), SP_C(b, 7) "s_nop 1\n"

// Fragment reads into set s: K (ks, mb) of tile J; V channel block md (both
// 16-byte halves) of tile J; K of the next group's tile 0 (bases kn<ks>). The
// bases point into the current stage (the V bases include the 64 KB).
#define SP_RK(ks, mb, J, s) "ds_read_b128 " SP_K(ks, mb, s) ", %[kb" #ks "] offset:" #mb "*4096+" #J "*8192\n"
#define SP_RKN(ks, mb, s) "ds_read_b128 " SP_K(ks, mb, s) ", %[kn" #ks "] offset:" #mb "*4096\n"
#define SP_RV(md, J, s)                                                                                           \
    "ds_read_b128 " SP_VH(md, 0, s) ", %[vb0] offset:" #md "*2048+" #J "*8192\n"                                    \
    "ds_read_b128 " SP_VH(md, 1, s) ", %[vb1] offset:" #md "*2048+" #J "*8192\n"
// Slot lists: K reads, two per slot in the first four slots.
#define SP_RK_SLOTS(J, s) SP_RK(0, 0, J, s) SP_RK(0, 1, J, s), SP_RK(1, 0, J, s) SP_RK(1, 1, J, s),                   \
    SP_RK(2, 0, J, s) SP_RK(2, 1, J, s), SP_RK(3, 0, J, s) SP_RK(3, 1, J, s)
#define SP_RKN_SLOTS(s) SP_RKN(0, 0, s) SP_RKN(0, 1, s), SP_RKN(1, 0, s) SP_RKN(1, 1, s),                             \
    SP_RKN(2, 0, s) SP_RKN(2, 1, s), SP_RKN(3, 0, s) SP_RKN(3, 1, s)

// Loads of tile lt (clamped to the last tile) into slot J of the current
// stage (m0 base mc): this wave's two 1 KB blocks of K (keys 8 wave + 32 i +
// lane / 8) and of V (channels 16 wave + 64 i + lane / 4).
#define SP_LTILE                                                                                                  \
    "s_min_u32 %[tt], %[lt], %[tmax]\n"                                                                           \
    "s_lshl_b32 %[sk], %[tt], 13\n"                                                                               \
    "s_add_u32 %[sk], %[sk], %[hk]\n"                                                                             \
    "s_lshl_b32 %[sv], %[tt], 6\n"                                                                                \
    "s_add_u32 %[sv], %[sv], %[hv]\n"                                                                             \
    "s_add_u32 %[lt], %[lt], 1\n"
#define SP_LD(J)                                                                                                  \
    "s_add_u32 m0, %[mc], " #J "*8192\n"                                                                             \
    "buffer_load_dwordx4 %[ko], %[kr], %[sk] offen lds\n"                                                         \
    "s_add_u32 m0, %[mc], " #J "*8192+4096\n"                                                                        \
    "s_add_u32 %[sk], %[sk], 4096\n"                                                                              \
    "buffer_load_dwordx4 %[ko], %[kr], %[sk] offen lds\n"                                                         \
    "s_add_u32 m0, %[mc], 65536+" #J "*8192\n"                                                                       \
    "buffer_load_dwordx4 %[vo], %[vr], %[sv] offen lds\n"                                                         \
    "s_add_u32 m0, %[mc], 65536+" #J "*8192+4096\n"                                                                  \
    "s_add_u32 %[sv], %[sv], %[v64]\n"                                                                            \
    "buffer_load_dwordx4 %[vo], %[vr], %[sv] offen lds\n"
#define SP_LOADS() "", SP_LTILE SP_LD(0), SP_LTILE SP_LD(1), SP_LTILE SP_LD(2), SP_LTILE SP_LD(3)
#define SP_NOLOADS() SP_NONE5
// The next tile's key scale k_scale[head, min(tile, blocks - 1)] into sks<N>.
#define SP_KSCALE(N) "s_min_u32 %[tk], %[st], %[bmax]\n s_lshl_b32 %[tk], %[tk], 2\n"                             \
    "s_load_dword %[sks" #N "], %[ksp], %[tk]\n s_add_u32 %[st], %[st], 1\n"

#define SP_WAIT_LDS "s_waitcnt lgkmcnt(0)\n"
#define SP_BARRIER "s_waitcnt vmcnt(0) lgkmcnt(0)\n s_barrier\n"

// Tiles of a group. Even tile J (fragment set 0; PREV: block 1's softmax of
// the previous tile, SP_SOFT_B(1) or SP_NONE8): V of tile J read in phase 1,
// K of tile JN = J + 1 (set 1) in phase 2. Tile 1: K of tile 2 (set 0) in
// phase 2. Tile 3: the barrier after phase 2, K of the next group's tile 0
// (set 0, the other stage) in phase 3, the loads (LD) in phase 4, then the
// stage flip.
#define SP_TILE_E(PREV, MSK, J, JN, L)                                                                            \
    SP_PH8_EXP(SP_SMFMA(0, 0), PREV, SP_KSCALE(1) SP_RV(0, J, 0), SP_RV(1, J, 0), SP_RV(2, J, 0), SP_RV(3, J, 0),   \
               "", "", "", "")                                                                                     \
    SP_PH5_EXP(SP_PVMFMA(1, 1), SP_SOFT_A(0, MSK, J, L##a), SP_RK_SLOTS(JN, 1), "")                               \
    SP_PH8_EXP(SP_SMFMA(1, 0), SP_SOFT_B(0), SP_NONE8)                                                            \
    SP_WAIT_LDS                                                                                                   \
    SP_PH5_EXP(SP_PVMFMA(0, 0), SP_SOFT_A(1, MSK, J, L##b), SP_NONE5)                                             \
    SP_WAIT_LDS
#define SP_TILE_1(MSK, L)                                                                                         \
    SP_PH8_EXP(SP_SMFMA(0, 1), SP_SOFT_B(1), SP_KSCALE(0) SP_RV(0, 1, 1), SP_RV(1, 1, 1), SP_RV(2, 1, 1),           \
               SP_RV(3, 1, 1), "", "", "", "")                                                                     \
    SP_PH5_EXP(SP_PVMFMA(1, 0), SP_SOFT_A(0, MSK, 1, L##a), SP_RK_SLOTS(2, 0), "")                                \
    SP_PH8_EXP(SP_SMFMA(1, 1), SP_SOFT_B(0), SP_NONE8)                                                            \
    SP_WAIT_LDS                                                                                                   \
    SP_PH5_EXP(SP_PVMFMA(0, 1), SP_SOFT_A(1, MSK, 1, L##b), SP_NONE5)                                             \
    SP_WAIT_LDS
#define SP_TILE_3(MSK, L, LD)                                                                                     \
    SP_PH8_EXP(SP_SMFMA(0, 1), SP_SOFT_B(1), SP_KSCALE(0) SP_RV(0, 3, 1), SP_RV(1, 3, 1), SP_RV(2, 3, 1),           \
               SP_RV(3, 3, 1), "", "", "", "")                                                                     \
    SP_PH5_EXP(SP_PVMFMA(1, 0), SP_SOFT_A(0, MSK, 3, L##a), SP_NONE5)                                             \
    SP_BARRIER                                                                                                    \
    SP_PH8_EXP(SP_SMFMA(1, 1), SP_SOFT_B(0), SP_RKN_SLOTS(0), "", "", "", "")                                     \
    SP_WAIT_LDS                                                                                                   \
    SP_PH5_EXP(SP_PVMFMA(0, 1), SP_SOFT_A(1, MSK, 3, L##b), LD())                                                   \
    SP_WAIT_LDS                                                                                                   \
    SP_FLIP
// The next group's stage: fragment bases and the load base flip bit 15.
#define SP_FLIP "v_xor_b32 %[kb0], 0x8000, %[kb0]\n v_xor_b32 %[kb1], 0x8000, %[kb1]\n"                             \
    "v_xor_b32 %[kb2], 0x8000, %[kb2]\n v_xor_b32 %[kb3], 0x8000, %[kb3]\n"                                      \
    "v_xor_b32 %[kn0], 0x8000, %[kn0]\n v_xor_b32 %[kn1], 0x8000, %[kn1]\n"                                      \
    "v_xor_b32 %[kn2], 0x8000, %[kn2]\n v_xor_b32 %[kn3], 0x8000, %[kn3]\n"                                      \
    "v_xor_b32 %[vb0], 0x8000, %[vb0]\n v_xor_b32 %[vb1], 0x8000, %[vb1]\n"                                      \
    "s_xor_b32 %[mc], %[mc], 0x8000\n"
// A group (tiles 0 to 3).
#define SP_GROUP(MSK, L, LD) SP_TILE_E(SP_SOFT_B(1), MSK, 0, 1, L##0) SP_TILE_1(MSK, L##1)                          \
    SP_TILE_E(SP_SOFT_B(1), MSK, 2, 3, L##2) SP_TILE_3(MSK, L##3, LD)
// Group 0: no block-1 softmax before its first scores and no P.V of block 1
// in its first phase 2 (the MFMA results of S0 are waited for instead).
#define SP_GROUP_FIRST                                                                                            \
    SP_PH8_EXP(SP_SMFMA(0, 0), SP_NONE8, SP_KSCALE(1) SP_RV(0, 0, 0), SP_RV(1, 0, 0), SP_RV(2, 0, 0),              \
               SP_RV(3, 0, 0), "", "", "", "")                                                                     \
    "s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n"                                                           \
    SP_PH5_EXP(SP_NOMFMA5, SP_SOFT_A(0, SP_NOMASK, 0, f0a), SP_RK_SLOTS(1, 1), "")                                \
    SP_PH8_EXP(SP_SMFMA(1, 0), SP_SOFT_B(0), SP_NONE8)                                                            \
    SP_WAIT_LDS                                                                                                   \
    SP_PH5_EXP(SP_PVMFMA(0, 0), SP_SOFT_A(1, SP_NOMASK, 0, f0b), SP_NONE5)                                        \
    SP_WAIT_LDS                                                                                                   \
    SP_TILE_1(SP_NOMASK, f1) SP_TILE_E(SP_SOFT_B(1), SP_NOMASK, 2, 3, f2) SP_TILE_3(SP_NOMASK, f3, SP_LOADS)
// After the last tile (J = 3): block 1's softmax and P.V, and a wait for
// every MFMA result before the accumulators leave the asm block.
#define SP_TAIL                                                                                                   \
    SP_PH8_EXP(SP_NOMFMA8, SP_SOFT_B(1), SP_NONE8)                                                                \
    "s_nop 7\n"                                                                                                   \
    SP_PH5_EXP(SP_PVMFMA(1, 1), SP_NONE5, SP_NONE5)                                                               \
    "s_waitcnt vmcnt(0) lgkmcnt(0)\n"                                                                             \
    "s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n"

#define SP_CL10(p, x) #p #x "0", #p #x "1", #p #x "2", #p #x "3", #p #x "4", #p #x "5", #p #x "6", #p #x "7",          \
    #p #x "8", #p #x "9"
#define SP_CLOBBERS                                                                                               \
    "v0", "v1", "v2", "v3", "v4", "v5", "v6", "v7", "v8", "v9", SP_CL10(v, 1), SP_CL10(v, 2), SP_CL10(v, 3),           \
    SP_CL10(v, 4), SP_CL10(v, 5), "v60", "v61", "v62", "v63",                                                      \
    "a0", "a1", "a2", "a3", "a4", "a5", "a6", "a7", "a8", "a9", SP_CL10(a, 1), SP_CL10(a, 2), SP_CL10(a, 3),           \
    SP_CL10(a, 4), SP_CL10(a, 5), SP_CL10(a, 6), SP_CL10(a, 7), SP_CL10(a, 8), SP_CL10(a, 9), SP_CL10(a, 10),          \
    SP_CL10(a, 11), "a120", "a121", "a122", "a123", "a124", "a125", "a126", "a127", "m0", "vcc", "scc", "memory"

__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void sage_pipe(SArgs a) {
    constexpr int BM = 256;
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    const unsigned tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / 64), lane = tid % 64;
    const unsigned n = lane % 32, hf = lane / 32;
    const unsigned nqb = (a.seq + BM - 1) / BM;
    const unsigned id = xcd_remap(blockIdx.x, gridDim.x);
    const unsigned head = __builtin_amdgcn_readfirstlane(id / nqb), qb = __builtin_amdgcn_readfirstlane(id % nqb);
    const unsigned q0 = qb * BM;
    const unsigned ntiles = a.padded / BN;               // the launcher ensures ntiles >= 9
    const unsigned groups = (ntiles + SP_GROUP_TILES - 1) / SP_GROUP_TILES;
    const int8_t *qh = a.q8 + (size_t)head * a.padded * D;

    // Q fragments of both blocks (rows past the padding repeat the last row).
    i32x4 qf[2][4];
#pragma unroll
    for (int b = 0; b < 2; b++) {
        const unsigned qrow = min(q0 + wave * 64 + b * 32 + n, a.padded - 1);
#pragma unroll
        for (int ks = 0; ks < 4; ks++)
            qf[b][ks] = *reinterpret_cast<const i32x4 *>(qh + (size_t)qrow * D + ks * 32 + hf * 16);
    }
    // One 64-row quantization block per wave: both blocks share q_scale.
    const unsigned qblk = min((q0 + wave * 64) / 64, a.blocks - 1);
    const float qs = a.q_scale[head * a.blocks + qblk] * a.scale_log2;
    float kmax = 0.f;
    for (unsigned b = lane; b < a.blocks; b += 64) kmax = fmaxf(kmax, a.k_scale[head * a.blocks + b]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) kmax = fmaxf(kmax, __shfl_xor(kmax, off, 64));
    const bool failed = __builtin_amdgcn_readfirstlane(qs * kmax > MAGIC_C_MAX ? 1 : 0) != 0;

    // Tile loads: block wave + 4 i of a tile (i = 0, 1) holds keys
    // 8 wave + 32 i + lane / 8 of K and channels 16 wave + 64 i + lane / 4 of V.
    const i32x4 kr = {(int)__builtin_amdgcn_readfirstlane((unsigned)(uint64_t)a.k8),
                      (int)__builtin_amdgcn_readfirstlane((unsigned)((uint64_t)a.k8 >> 32)),
                      (int)__builtin_amdgcn_readfirstlane((unsigned)((size_t)a.heads * a.padded * D)), 0x00020000};
    const i32x4 vr = {(int)__builtin_amdgcn_readfirstlane((unsigned)(uint64_t)a.v8),
                      (int)__builtin_amdgcn_readfirstlane((unsigned)((uint64_t)a.v8 >> 32)),
                      (int)__builtin_amdgcn_readfirstlane((unsigned)((size_t)a.heads * D * a.padded)), 0x00020000};
    const unsigned koff = (8 * wave + lane / 8) * D + k8_chunk(8 * wave + lane / 8, lane % 8) * 16;
    const unsigned voff = (16 * wave + lane / 4) * a.padded + v8_chunk(16 * wave + lane / 4, lane % 4) * 16;
    const unsigned hk = __builtin_amdgcn_readfirstlane(head * a.padded * D);
    const unsigned hv = __builtin_amdgcn_readfirstlane(head * D * a.padded);
    const unsigned v64 = __builtin_amdgcn_readfirstlane(64 * a.padded);
    const unsigned tmax = ntiles - 1;
    // Tiles 0..7 (groups 0 and 1) into stages 0 and 1.
#pragma unroll
    for (int t8 = 0; t8 < 2 * SP_GROUP_TILES; t8++) {
        const unsigned tile = min((unsigned)t8, tmax);
        uint8_t *ks = lds + (t8 / SP_GROUP_TILES) * SP_STAGE + (t8 % SP_GROUP_TILES) * Q8_TILE;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                *reinterpret_cast<const __amdgpu_buffer_rsrc_t *>(&kr),
                (__attribute__((address_space(3))) void *)(ks + (wave + 4 * i) * 1024), 16, koff,
                hk + tile * Q8_TILE + 4096 * i, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                *reinterpret_cast<const __amdgpu_buffer_rsrc_t *>(&vr),
                (__attribute__((address_space(3))) void *)(ks + 2 * SP_STAGE + (wave + 4 * i) * 1024), 16, voff,
                hv + tile * BN + v64 * i, 0, 0);
        }
    }
    wait_vm_loads();
    __syncthreads();

    // Fragment bases (stage 0, tile 0): K (ks, mb) at kb<ks> + 4 KB mb; V
    // channel block md at vb<h> + 2 KB md (h: the 16-byte half).
    unsigned kb[4], kn[4], vb[2];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        kb[ks] = n * D + k8_chunk(n, 2 * ks + hf) * 16;
        kn[ks] = kb[ks] + SP_STAGE;
    }
#pragma unroll
    for (int h = 0; h < 2; h++) vb[h] = 2 * SP_STAGE + n * BN + v8_chunk(n, 2 * hf + h) * 16;

    f32x16 o0[4], o1[4];
#pragma unroll
    for (int md = 0; md < 4; md++) { o0[md] = f32x16{}; o1[md] = f32x16{}; }
    f32x4 l0 = f32x4{}, l1 = f32x4{};
    i32x16 magic;
#pragma unroll
    for (int r = 0; r < 16; r++) magic[r] = MAGIC_BITS;
    i32x8 ones;                              // fp8 e4m3 1.0 = 0x38, or 0 where not kept
#pragma unroll
    for (int i = 0; i < 8; i++) ones[i] = (((lane % 16) / 4 + lane / 16) & 1) ? 0 : 0x38383838;
    float m0v = -1e30f, m1v = -1e30f;
    unsigned mc = __builtin_amdgcn_readfirstlane(wave * 1024);
    unsigned lt = 2 * SP_GROUP_TILES, gl = groups - 2, st = 1;
    const unsigned last0 = SP_GROUP_TILES * (groups - 1) * BN;
    const int lim0 = (int)a.seq - (int)last0 - 4 * (int)hf, lim1 = lim0 - BN, lim2 = lim1 - BN, lim3 = lim2 - BN;
    const uint64_t kspv = (uint64_t)(a.k_scale + head * a.blocks);
    // (readfirstlane returns int: widen through unsigned, not by sign extension)
    const uint64_t ksp = ((uint64_t)(unsigned)__builtin_amdgcn_readfirstlane((unsigned)(kspv >> 32)) << 32) |
                         (uint64_t)(unsigned)__builtin_amdgcn_readfirstlane((unsigned)kspv);
    float sks0 = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(           // tile 0's key scale
        __builtin_bit_cast(unsigned, a.k_scale[head * a.blocks]))), sks1 = 0.f;
    const float k16 = 16.f, nk23 = -0x1p-23f;
    const int masked = MASKED_BITS;
    float c0, c1, t0, t1, u0, u1, w0, w1, x0, x1, y0, y1;
    unsigned tt, tk, sk, sv;
    asm volatile(
        SP_RK(0, 0, 0, 0) SP_RK(0, 1, 0, 0) SP_RK(1, 0, 0, 0) SP_RK(1, 1, 0, 0)
        SP_RK(2, 0, 0, 0) SP_RK(2, 1, 0, 0) SP_RK(3, 0, 0, 0) SP_RK(3, 1, 0, 0)
        SP_WAIT_LDS
        SP_GROUP_FIRST
        "sp_loop_%=:\n"
        SP_GROUP(SP_NOMASK, gp, SP_LOADS)
        "s_sub_u32 %[gl], %[gl], 1\n"
        "s_cmp_lg_u32 %[gl], 0\n"
        "s_cbranch_scc1 sp_loop_%=\n"
        SP_GROUP(SP_MASK, gl, SP_NOLOADS)
        SP_TAIL
        : [o00] "+{v[64:79]}"(o0[0]), [o01] "+{v[80:95]}"(o0[1]), [o02] "+{v[96:111]}"(o0[2]),
          [o03] "+{v[112:127]}"(o0[3]), [o10] "+{v[128:143]}"(o1[0]), [o11] "+{v[144:159]}"(o1[1]),
          [o12] "+{v[160:175]}"(o1[2]), [o13] "+{v[176:191]}"(o1[3]), [l0] "+{v[216:219]}"(l0),
          [l1] "+{v[220:223]}"(l1),
          [rm0] "+v"(m0v), [rm1] "+v"(m1v), [kb0] "+v"(kb[0]), [kb1] "+v"(kb[1]), [kb2] "+v"(kb[2]),
          [kb3] "+v"(kb[3]), [kn0] "+v"(kn[0]), [kn1] "+v"(kn[1]), [kn2] "+v"(kn[2]), [kn3] "+v"(kn[3]),
          [vb0] "+v"(vb[0]), [vb1] "+v"(vb[1]), [mc] "+s"(mc),
          [lt] "+s"(lt), [gl] "+s"(gl), [st] "+s"(st), [sks0] "+s"(sks0), [sks1] "+s"(sks1),
          [c0] "=&v"(c0), [c1] "=&v"(c1), [t0] "=&v"(t0), [t1] "=&v"(t1), [u0] "=&v"(u0), [u1] "=&v"(u1),
          [w0] "=&v"(w0), [w1] "=&v"(w1), [x0] "=&v"(x0), [x1] "=&v"(x1), [y0] "=&v"(y0), [y1] "=&v"(y1), [tt] "=&s"(tt), [tk] "=&s"(tk), [sk] "=&s"(sk), [sv] "=&s"(sv)
        : [q00] "{a[128:131]}"(qf[0][0]), [q01] "{a[132:135]}"(qf[0][1]), [q02] "{a[136:139]}"(qf[0][2]),
          [q03] "{a[140:143]}"(qf[0][3]), [q10] "{a[144:147]}"(qf[1][0]), [q11] "{a[148:151]}"(qf[1][1]),
          [q12] "{a[152:155]}"(qf[1][2]), [q13] "{a[156:159]}"(qf[1][3]),
          [mg] "{v[192:207]}"(magic), [ones] "{a[160:167]}"(ones),
          [qs] "v"(qs), [k16] "s"(k16), [nk23] "s"(nk23), [masked] "v"(masked), [ksp] "s"(ksp),
          [bmax] "s"(a.blocks - 1), [kr] "s"(kr), [vr] "s"(vr), [tmax] "s"(tmax), [hk] "s"(hk), [hv] "s"(hv),
          [v64] "s"(v64), [ko] "v"(koff), [vo] "v"(voff),
          [lim0] "v"(lim0), [lim1] "v"(lim1), [lim2] "v"(lim2), [lim3] "v"(lim3)
        : SP_CLOBBERS);

    // Output as sage_attn_kernel writes it; a wave whose logit scale can
    // exceed the fast exponent's range leaves its rows to the exact launch,
    // whose retry bytes are laid out per 32-query wave of 128-query workgroups.
    const unsigned nqb4 = (a.seq + 127) / 128;
    const float *vsc = a.v_scale + head * D;
#pragma unroll
    for (int b = 0; b < 2; b++) {
        const unsigned qstart = q0 + wave * 64 + b * 32;
        if (lane == 0 && qstart / 32 < nqb4 * 4) a.retry[(size_t)head * nqb4 * 4 + qstart / 32] = failed ? 1 : 0;
        if (failed) continue;
        const f32x16 *o = b ? o1 : o0;
        const float total = b ? l1[0] : l0[0];
        const float inv = total > 0.f ? 1.f / total : 0.f;
        const unsigned q = qstart + n;
        bool bad = false;
        if (q < a.seq) {
            uint16_t *dst = a.out + (a.head_major ? ((size_t)head * a.seq + q) * D : ((size_t)q * a.heads + head) * D);
#pragma unroll
            for (int md = 0; md < 4; md++)
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++) {
                    u16x4 w;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        unsigned d = md * 32 + g4 * 8 + hf * 4 + i;
                        float x = o[md][g4 * 4 + i] * (vsc[d] * inv);
                        bad |= !finite_f32(x);
                        w[i] = f32_to_bf16(x);
                    }
                    *reinterpret_cast<u16x4 *>(dst + md * 32 + g4 * 8 + hf * 4) = w;
                }
        }
        if (bad) a.fault[0] = 1u;
    }
}

int launch_sage_pipe(h3_gpu *g, const SArgs &a) {
    static bool configured = false;
    if (!configured) {
        if (!h3_hip_check(g, hipFuncSetAttribute((const void *)sage_pipe, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 SP_LDS), "Sage shared memory"))
            return 0;
        configured = true;
    }
    hipEvent_t timing = h3_kernel_timing_begin(g);
    hipLaunchKernelGGL(sage_pipe, dim3((a.seq + 255) / 256 * a.heads), dim3(256), SP_LDS, g->compute, a);
    if (!h3_launch_status(g, "Sage attention")) {
        h3_kernel_timing_end(g, timing);
        return 0;
    }
    hipLaunchKernelGGL((sage_attn_kernel<4, 3, false, true>), dim3((a.seq + 127) / 128 * a.heads), dim3(256),
                       2 * SAGE_TILE, g->compute, a);
    h3_kernel_timing_end(g, timing);
    return h3_launch_status(g, "Sage exact recomputation");
}

// The fast launch, then the recomputation launch, whose workgroups return at
// once unless one of their waves was flagged.
template <int WAVES, int OCC, bool SPARSE>
int launch_sage(h3_gpu *g, const SArgs &a, unsigned groups) {
    constexpr size_t shared = 2 * SAGE_TILE;
    hipEvent_t timing = h3_kernel_timing_begin(g);
    hipLaunchKernelGGL((sage_attn_kernel<WAVES, OCC, SPARSE>), dim3(groups), dim3(64 * WAVES), shared, g->compute, a);
    if (!h3_launch_status(g, "Sage attention")) {
        h3_kernel_timing_end(g, timing);
        return 0;
    }
    hipLaunchKernelGGL((sage_attn_kernel<WAVES, OCC, SPARSE, true>), dim3(groups), dim3(64 * WAVES), shared,
                       g->compute, a);
    // Both launches inside one timing window, as the BF16 path times them.
    h3_kernel_timing_end(g, timing);
    return h3_launch_status(g, "Sage exact recomputation");
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
    a.retry = (uint8_t *)(ws + L.retry);
    // Variant 13: the global-load path that operands of 4 GiB and more take.
    a.buffered = (size_t)heads * L.padded * D < (1ull << 32) && g->attention_variant != 13;
    // 4 waves x 32 queries per workgroup, three workgroups per CU (three
    // waves per SIMD, 166 VGPRs each); block-sparse lists are per 128-query
    // block, the same shape. The workgroups' barriers are independent, so the
    // waves that share a SIMD drift into different phases of their tiles (one
    // 12-wave workgroup per CU keeps all twelve in step: 6% slower, variant 2;
    // 8 waves at two per SIMD: variant 1).
    if (kv_list) return launch_sage<4, 3, true>(g, a, (seq + 127) / 128 * heads);
    if (g->attention_variant == 1) return launch_sage<8, 2, false>(g, a, (seq + 255) / 256 * heads);
    if (g->attention_variant == 2) return launch_sage<12, 3, false>(g, a, (seq + 383) / 384 * heads);
    // Dense, buffered, more than 512 keys: the hand-scheduled kernel (four
    // waves of 64 queries, one per SIMD), bit-identical to the 4-wave kernel
    // that variant 14 forces.
    if (a.buffered && seq > 512 && g->attention_variant != 14) return launch_sage_pipe(g, a);
    return launch_sage<4, 3, false>(g, a, (seq + 127) / 128 * heads);
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
