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
        count = __builtin_amdgcn_readfirstlane(a.kv_count[qb]);
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
        const float c = qs * a.k_scale[head * a.blocks + min(tile, a.blocks - 1)];
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
        if (count) tile = __builtin_amdgcn_readfirstlane(list[0]);
        if (count > 1) next = __builtin_amdgcn_readfirstlane(list[1]);
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
        if constexpr (SPARSE) later = it + 2 < count ? list[it + 2] : 0u;
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
