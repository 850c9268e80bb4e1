// FlashAttention-style BF16 self-attention for gfx950 (D = 128, non-causal).
//
// Semantics follow the reference's online-softmax operator
// (src/cuda/cuda_attention.cuh:7-51): softmax(scale * Q K^T) V with FP32 scores,
// FP32 running max / denominator and FP32 P.V accumulation, BF16 output. The
// difference is where P meets V: P is rounded to BF16 so that P.V runs on the
// BF16 matrix cores, as the reference's tensor-core path and FlashAttention do.
//
// Work decomposition (MI355X-first, not a translation of the CUDA kernels):
//  * one workgroup = WAVES wavefronts x 32 queries of one head; the query
//    fragments of a wave stay in VGPRs for the whole key sweep, and two waves
//    share each SIMD so one wave's softmax overlaps the other's MFMAs;
//  * scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_bf16:
//    each lane then owns one query column, so the row max is a register max
//    plus one v_permlane32_swap between the two 32-lane halves, and the FP32
//    score accumulator, rounded to BF16, is already laid out as the B operand
//    of O^T += V^T P^T;
//  * V is transposed once per call by a bandwidth-bound pre-pass into
//    [head, channel, key] with the key order the score accumulator produces;
//  * K and V^T tiles go from global memory straight into LDS
//    (global_load_lds, 16 bytes per lane) in XOR-swizzled 16-byte chunks, so
//    both operand reads are free of bank conflicts; the next interval's tiles
//    load while the current one is processed (two LDS stages);
//  * the dense kernel covers 128 keys per barrier interval (two 64-key
//    sub-tiles) and requests all fragments of a sub-tile before its first
//    MFMA, so LDS latency is paid once per sub-tile;
//  * the running max is only raised when a tile's max exceeds it by more than
//    8 (log2 units; P then stays below 256), so the accumulator rescale runs a
//    handful of times per row instead of per tile;
//  * workgroup ids are remapped so that the workgroups of one head share an XCD
//    (and its L2), which is where their K/V tiles are re-read.
#include "common.h"
#include "internal.h"
#include "attn_common.h"

namespace {

constexpr int D = 128;
constexpr int BN = 64;                     // keys per tile
constexpr int K_BYTES = BN * D * 2;        // K tile: 64 rows x 256 B, 16-byte chunks XOR-swizzled
constexpr int V_BYTES = D * BN * 2;        // V^T tile: 128 rows x 128 B, 16-byte chunks XOR-swizzled
constexpr int STAGE_BYTES = K_BYTES + V_BYTES;
constexpr float RESCALE_SLACK = 8.0f;      // log2 units the running max may lag
constexpr float PSUM_LIMIT = 1048576.0f;   // 2^20: bound on a lane's 32-key partial row sum
constexpr int RETRY_EXP = 32;              // partial sums from 2^32 up send the rows to the recomputation

// LDS chunk swizzles (16-byte chunks): every 16-lane group of a ds_read_b128
// touches 16 distinct 4-bank groups for both operand reads.
__device__ inline unsigned k_chunk(unsigned key, unsigned ch) { return ch ^ (key & 15); }
__device__ inline unsigned v_chunk(unsigned d, unsigned ch) { return ch ^ ((d >> 1) & 7); }

struct Args {
    uint16_t *out;
    const uint16_t *q, *k;
    const uint16_t *vt;                    // [heads, 128, padded] permuted keys
    unsigned seq, heads, padded;
    float scale_log2;                      // softmax scale * log2(e)
    int head_major;
    // Sparse: kept 64-key tile ids in ascending order, per 128-query block
    // (host masks, all heads) or per (head, 64-query block) (routed kernel).
    const uint32_t *kv_list;
    const uint32_t *kv_count;              // sparse: number of entries per list
    unsigned list_stride;
    unsigned *fault;
    // Dense kernel: one byte per (head, 256-query block, wave), set when the
    // wave's rows need the recomputation launch.
    uint8_t *retry;
    // SOL centroid phase (listed kernel with CENT): per (head, query block) the
    // centroid tile list, its length and the approximate-block mask of each
    // tile; centroid K rows [key_blocks][heads][128] and transposed V
    // [heads][128][kc_padded] in the V^T key order.
    const uint32_t *cent_list, *cent_count;
    const uint64_t *cent_mask;
    unsigned cent_stride, key_blocks, kc_padded;
    const uint16_t *kc, *vct;
    // Dense kernel only: query rows when they are fewer than the keys (a query
    // range; q and out point at its first row, the head-major output keeps the
    // full sequence stride), 0 for all seq rows; and an optional FP32 log-sum-
    // exp per (head, query row) of scale * q.k in natural-log units.
    unsigned qrows;
    float *lse;
    // Listed kernel only: a slab of query blocks [qb0, qb0 + qslab) (lists
    // indexed slab-relative, [head][qslab]); qslab 0 covers the sequence.
    unsigned qb0, qslab;
    // K and V^T fit 32-bit buffer offsets (below 4 GiB each): the dense
    // kernels then load tiles with buffer loads.
    int buffered;
};

// Whether K [seq, heads, 128] and V^T [heads, 128, padded] both fit 32-bit
// buffer offsets.
static int fits_buffer(const Args &a) {
    return (size_t)a.seq * a.heads * D * 2 < (1ull << 32) && (size_t)a.heads * D * a.padded * 2 < (1ull << 32);
}

// Position of key j (0..63) inside a transposed V row: keys are grouped by 16
// and, inside a group, ordered the way a lane half holds them in the S^T
// accumulator (rows (r/4)*8 + half*4 + r%4 of a 32x32 MFMA output).
__host__ __device__ inline unsigned v_position(unsigned j) {
    unsigned k16 = j & 15;
    return (j & ~15u) + ((k16 >> 2) & 1) * 8 + (k16 >> 3) * 4 + (k16 & 3);
}

// V [seq, heads, 128] -> Vt [heads, 128, padded]; one workgroup per (64-key tile,
// head). The pass also screens this tile's K and V rows for Inf/NaN.
__global__ __launch_bounds__(256) void transpose_v(const uint16_t *v, const uint16_t *k, uint16_t *vt, unsigned seq,
                                                  unsigned heads, unsigned padded, unsigned *fault) {
    __shared__ uint16_t tile[BN][D + 8];
    const unsigned blk = blockIdx.x, head = blockIdx.y, t = threadIdx.x;
    const size_t stride = (size_t)heads * D;
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        unsigned c = t + 256 * i, key = c / 16, ch = c % 16, row = blk * BN + key;
        u16x8 raw = row < seq ? *reinterpret_cast<const u16x8 *>(v + row * stride + (size_t)head * D + ch * 8) : u16x8{};
        u16x8 kraw = row < seq ? *reinterpret_cast<const u16x8 *>(k + row * stride + (size_t)head * D + ch * 8) : u16x8{};
        bad |= bf16_vec_nonfinite(raw) | bf16_vec_nonfinite(kraw);
        *reinterpret_cast<u16x8 *>(&tile[key][ch * 8]) = raw;
    }
    if (bad) fault[0] = 1u;
    __syncthreads();
    // Thread t writes channel d = t / 2, positions half*32 .. half*32+31.
    const unsigned d = t / 2, half = t % 2;
    u16x8 w[4];
#pragma unroll
    for (int p = 0; p < 32; p++) {
        unsigned pos = half * 32 + p;
        // Inverse of v_position inside the 16-key group.
        unsigned p16 = pos & 15, hf = p16 >> 3, i = p16 & 7;
        unsigned key = (pos & ~15u) + (i >> 2) * 8 + hf * 4 + (i & 3);
        w[p / 8][p % 8] = tile[key][d];
    }
    uint16_t *dst = vt + ((size_t)head * D + d) * padded + blk * BN + half * 32;
#pragma unroll
    for (int j = 0; j < 4; j++) *reinterpret_cast<u16x8 *>(dst + j * 8) = w[j];
}

// WAVES wavefronts per workgroup, each owning NB x 32 queries; OCC waves share a
// SIMD (register budget 512 / OCC), so the hardware overlaps one wave's softmax
// with another's MFMAs.
// MSUM: row sums of P on the matrix core (ones . P^T) instead of VALU adds.
template <int WAVES, int NB, int OCC, bool SPARSE, bool MSUM>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * WAVES, 64 * WAVES), amdgpu_waves_per_eu(OCC, OCC)))
void attn_bf16_kernel(Args a) {
    constexpr int T = 64 * WAVES;
    constexpr int BM = 32 * NB * WAVES;
    constexpr int WQ = 32 * NB;             // queries per wave
    constexpr int BLOCKS = K_BYTES / 1024;  // 1 KB direct-to-LDS load blocks per operand tile
    static_assert(K_BYTES == V_BYTES, "tile split");
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];

    const unsigned tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const unsigned n = lane % 32, hf = lane / 32;
    const unsigned nqb = (a.seq + BM - 1) / BM;
    const unsigned id = xcd_remap(blockIdx.x, gridDim.x);
    const unsigned head = id / nqb, qb = id % nqb;
    const unsigned q0 = qb * BM;
    const size_t stride = (size_t)a.heads * D;
    const uint16_t *qh = a.q + (size_t)head * D;
    const uint16_t *kh = a.k + (size_t)head * D;
    const uint16_t *vth = a.vt + (size_t)head * D * a.padded;
    const float c = a.scale_log2;

    unsigned count;
    const uint32_t *list = nullptr;
    if constexpr (SPARSE) {
        count = __builtin_amdgcn_readfirstlane(load_uniform(a.kv_count + qb));
        list = a.kv_list + (size_t)qb * a.list_stride;
    } else {
        count = (a.seq + BN - 1) / BN;
    }

    // Query fragments: B operand of S^T = K Q^T, 8 k-steps of 16 channels.
    bf16x8 qf[NB][8];
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        unsigned row = q0 + wave * WQ + nb * 32 + n;
        row = row < a.seq ? row : a.seq - 1;
        const uint16_t *p = qh + (size_t)row * stride + hf * 8;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) qf[nb][ks] = *reinterpret_cast<const bf16x8 *>(p + ks * 16);
    }
    {
        bool bad = false;
#pragma unroll
        for (int nb = 0; nb < NB; nb++)
#pragma unroll
            for (int ks = 0; ks < 8; ks++) bad |= bf16_vec_nonfinite(qf[nb][ks]);
        if (bad) a.fault[0] = 1u;
    }

    f32x16 o[4][NB];
#pragma unroll
    for (int md = 0; md < 4; md++)
#pragma unroll
        for (int nb = 0; nb < NB; nb++) o[md][nb] = f32x16{};
    float m[NB], l[NB];
    f32x16 lsum[MSUM ? NB : 1];              // MSUM: every element holds the query's running sum
#pragma unroll
    for (int nb = 0; nb < NB; nb++) { m[nb] = -1e30f; l[nb] = 0.f; }
#pragma unroll
    for (int nb = 0; nb < (MSUM ? NB : 1); nb++) lsum[nb] = f32x16{};
    bf16x8 ones;
#pragma unroll
    for (int i = 0; i < 8; i++) ones[i] = (__bf16)1.0f;

    // Tile loads go straight from global memory to LDS (global_load_lds_dwordx4):
    // each wave instruction fills one contiguous KB, lane i writing bytes
    // [16i, 16i+16), so each lane fetches the logical chunk that the swizzle
    // places there. Keys past the end are clamped (their scores are masked) and
    // the transposed V is zero-padded to a whole tile.
    auto load_tile = [&](unsigned tile, int stage) {
        const unsigned key0 = tile * BN;
        uint8_t *ks = smem + stage * STAGE_BYTES;
        uint8_t *vs = ks + K_BYTES;
#pragma unroll
        for (unsigned b = wave; b < BLOCKS; b += WAVES) {
            // K block b: keys 4b .. 4b+3, lane -> (key, physical chunk).
            unsigned key = 4 * b + lane / 16, phys = lane % 16;
            unsigned row = min(key0 + key, a.seq - 1);
            const uint16_t *src = kh + (size_t)row * stride + k_chunk(key, phys) * 8;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                             (__attribute__((address_space(3))) void *)(ks + b * 1024), 16, 0, 0);
            // V^T block b: channels 8b .. 8b+7.
            unsigned d = 8 * b + lane / 8, vph = lane % 8;
            unsigned col = min(key0, a.padded - BN);
            const uint16_t *vsrc = vth + (size_t)d * a.padded + col + v_chunk(d, vph) * 8;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)vsrc,
                                             (__attribute__((address_space(3))) void *)(vs + b * 1024), 16, 0, 0);
        }
    };

    // One key tile: scores, online softmax, P.V. MASKED handles keys >= seq.
    auto process = [&](const uint8_t *ks, const uint8_t *vs, unsigned tile) {
        const bool MASKED = tile * BN + BN > a.seq;
        f32x16 s[2][NB];
#pragma unroll
        for (int mb = 0; mb < 2; mb++)
#pragma unroll
            for (int nb = 0; nb < NB; nb++) s[mb][nb] = f32x16{};
#pragma unroll
        for (int kstep = 0; kstep < 8; kstep++) {
#pragma unroll
            for (int mb = 0; mb < 2; mb++) {
                const unsigned key = mb * 32 + n;
                bf16x8 kf = *reinterpret_cast<const bf16x8 *>(ks + key * 256 + k_chunk(key, kstep * 2 + hf) * 16);
#pragma unroll
                for (int nb = 0; nb < NB; nb++)
                    s[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[nb][kstep], s[mb][nb], 0, 0, 0);
            }
        }
        if (MASKED) {
#pragma unroll
            for (int mb = 0; mb < 2; mb++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    unsigned key = tile * BN + mb * 32 + (r / 4) * 8 + hf * 4 + (r % 4);
                    if (key >= a.seq) {
#pragma unroll
                        for (int nb = 0; nb < NB; nb++) s[mb][nb][r] = -INFINITY;
                    }
                }
        }
        bf16x8 pb[NB][4];
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            // Two chains of 3-input maxima over the lane's 32 scores.
            float mx0 = fmaxf(s[0][nb][0], s[0][nb][1]), mx1 = fmaxf(s[1][nb][0], s[1][nb][1]);
#pragma unroll
            for (int r = 2; r < 16; r += 2) {
                mx0 = fmaxf(fmaxf(mx0, s[0][nb][r]), s[0][nb][r + 1]);
                mx1 = fmaxf(fmaxf(mx1, s[1][nb][r]), s[1][nb][r + 1]);
            }
            const float mx = half_max_swap(fmaxf(mx0, mx1)) * c;
            // Raise the running max only when this tile exceeds it by the slack.
            if (__builtin_amdgcn_ballot_w64(mx > m[nb] + RESCALE_SLACK)) {
                const float mnew = fmaxf(m[nb], mx);
                const float alpha = exp2f_fast(m[nb] - mnew);
                m[nb] = mnew;
                if constexpr (MSUM) lsum[nb] *= alpha;
                else l[nb] *= alpha;
#pragma unroll
                for (int md = 0; md < 4; md++) o[md][nb] *= alpha;
            }
            const float neg = -m[nb];
            float psum = 0.f;
#pragma unroll
            for (int mb = 0; mb < 2; mb++)
#pragma unroll
                for (int r = 0; r < 16; r += 2) {
                    float p0 = exp2f_fast(fmaf(s[mb][nb][r], c, neg));
                    float p1 = exp2f_fast(fmaf(s[mb][nb][r + 1], c, neg));
                    if constexpr (!MSUM) psum += p0 + p1;
                    pb[nb][mb * 2 + r / 8][r % 8] = (__bf16)p0;
                    pb[nb][mb * 2 + r / 8][r % 8 + 1] = (__bf16)p1;
                }
            if constexpr (!MSUM) l[nb] += psum;
        }
        // O^T[md][nb] += V^T[md] P^T[nb]: 32 channels x 32 queries, 4 k-steps of 16 keys.
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
#pragma unroll
            for (int md = 0; md < 4; md++) {
                const unsigned d = md * 32 + n;
                bf16x8 vf = *reinterpret_cast<const bf16x8 *>(vs + d * 128 + v_chunk(d, kk * 2 + hf) * 16);
#pragma unroll
                for (int nb = 0; nb < NB; nb++)
                    o[md][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pb[nb][kk], o[md][nb], 0, 0, 0);
            }
            // Row sums of the BF16 P actually multiplied into V, on the matrix
            // core: ones(32 x 16) . P^T gives every row the 16-key sum per query.
            if constexpr (MSUM) {
#pragma unroll
                for (int nb = 0; nb < NB; nb++)
                    lsum[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ones, pb[nb][kk], lsum[nb], 0, 0, 0);
            }
        }
    };

    // Sparse tile ids are wave-uniform and read one iteration ahead, so the
    // id load completes under the tile-load wait instead of stalling the
    // next iteration's loads.
    unsigned tile = 0, next = 1;
    if constexpr (SPARSE) {
        if (count) tile = __builtin_amdgcn_readfirstlane(load_uniform(list));
        if (count > 1) next = __builtin_amdgcn_readfirstlane(load_uniform(list + 1));
    }
    if (count) load_tile(tile, 0);
    wait_vm_loads();
    __syncthreads();

    for (unsigned it = 0; it < count; it++) {
        const int cur = it & 1;
        if (it + 1 < count) load_tile(next, cur ^ 1);
        uint32_t later = it + 2;
        if constexpr (SPARSE) later = it + 2 < count ? load_uniform(list + it + 2) : 0u;
        const uint8_t *ks = smem + cur * STAGE_BYTES;
        process(ks, ks + K_BYTES, tile);
        wait_vm_loads();
        __syncthreads();
        tile = next;
        next = SPARSE ? __builtin_amdgcn_readfirstlane(later) : later;
    }

    // Normalize and store. Lane holds query column n, channels (r/4)*8 + hf*4 + r%4.
    bool bad = false;
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        const float total = MSUM ? lsum[nb][0] : half_sum_swap(l[nb]);
        const float inv = total > 0.f ? 1.f / total : 0.f;
        const unsigned q = q0 + wave * WQ + nb * 32 + n;
        if (q >= a.seq) continue;
        uint16_t *dst = a.out + (a.head_major ? ((size_t)head * a.seq + q) * D : ((size_t)q * a.heads + head) * D);
#pragma unroll
        for (int md = 0; md < 4; md++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                u16x4 w;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    float x = o[md][nb][g4 * 4 + i] * inv;
                    bad |= !finite_f32(x);
                    w[i] = f32_to_bf16(x);
                }
                *reinterpret_cast<u16x4 *>(dst + md * 32 + g4 * 8 + hf * 4) = w;
            }
    }
    if (bad) a.fault[0] = 1u;
}

template <int WAVES, int NB, int OCC, bool SPARSE, bool MSUM>
int launch(h3_gpu *g, const Args &a, unsigned groups) {
    constexpr size_t shared = 2 * STAGE_BYTES;
    static bool configured = false;
    auto kernel = attn_bf16_kernel<WAVES, NB, OCC, SPARSE, MSUM>;
    if (!configured) {
        if (!h3_hip_check(g, hipFuncSetAttribute((const void *)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shared),
                          "attention shared memory"))
            return 0;
        configured = true;
    }
    hipEvent_t timing = h3_kernel_timing_begin(g);
    hipLaunchKernelGGL(kernel, dim3(groups), dim3(64 * WAVES), shared, g->compute, a);
    h3_kernel_timing_end(g, timing);
    return h3_launch_status(g, "BF16 attention");
}

// Wide tiles: each barrier interval covers KT consecutive 64-key sub-tiles, so
// the per-interval fixed costs (the barrier, the load wait and the serial
// max / ballot chain) are paid once per KT * 64 keys.
template <int KT, bool SPARSE, bool MSUM, bool NOMAX, int WAVES = 8>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * WAVES, 64 * WAVES), amdgpu_waves_per_eu(2, 2)))
void attn_bf16_wide(Args a) {
    static_assert(!(NOMAX && MSUM), "the overflow test reads the VALU row sums");
    static_assert(WAVES == 8 || WAVES == 4, "retry bytes: 8 or 4 per workgroup");
    constexpr int BM = 32 * WAVES;
    constexpr int BLOCKS = K_BYTES / 1024;
    constexpr int STAGE = KT * (K_BYTES + V_BYTES);
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];

    // wave and head are read as uniform values so that LDS destinations and
    // buffer offsets stay scalar.
    const unsigned tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / 64), lane = tid % 64;
    const unsigned n = lane % 32, hf = lane / 32;
    const unsigned qrows = a.qrows ? a.qrows : a.seq;
    const unsigned nqb = (qrows + BM - 1) / BM;
    const unsigned id = xcd_remap(blockIdx.x, gridDim.x);
    const unsigned head = __builtin_amdgcn_readfirstlane(id / nqb), qb = __builtin_amdgcn_readfirstlane(id % nqb);
    const unsigned q0 = qb * BM;
    uint8_t *const retry = a.retry ? a.retry + ((size_t)head * nqb + qb) * WAVES : nullptr;
    // The recomputation launch runs only the workgroups the fast kernel flagged.
    if constexpr (!NOMAX) {
        if constexpr (WAVES == 8) {
            if (retry && *reinterpret_cast<const uint64_t *>(retry) == 0) return;
        } else {
            if (retry && *reinterpret_cast<const uint32_t *>(retry) == 0) return;
        }
    }
    const size_t stride = (size_t)a.heads * D;
    const uint16_t *qh = a.q + (size_t)head * D;
    const uint16_t *kh = a.k + (size_t)head * D;
    const uint16_t *vth = a.vt + (size_t)head * D * a.padded;
    const float c = a.scale_log2;

    unsigned count;  // 64-key sub-tiles
    const uint32_t *list = nullptr;
    if constexpr (SPARSE) {
        count = a.kv_count[qb];
        list = a.kv_list + (size_t)qb * a.list_stride;
    } else {
        count = (a.seq + BN - 1) / BN;
    }
    const unsigned groups = (count + KT - 1) / KT;
    auto sub_at = [&](unsigned i) { i = min(i, count - 1); return SPARSE ? list[i] : i; };

    bf16x8 qf[8];
    {
        unsigned row = q0 + wave * 32 + n;
        row = row < qrows ? row : qrows - 1;
        const uint16_t *p = qh + (size_t)row * stride + hf * 8;
        bool bad = false;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            qf[ks] = *reinterpret_cast<const bf16x8 *>(p + ks * 16);
            bad |= bf16_vec_nonfinite(qf[ks]);
        }
        if (bad) a.fault[0] = 1u;
    }

    // Byte offsets, inside a full tile, of this lane's first 16-byte load (LDS
    // block wave). Load t (block wave + WAVES t) sits 4 WAVES t keys / 8 WAVES t
    // channels further on, with the same swizzle (it depends on key % 16 and
    // channel / 2 % 8 only): a full tile is a uniform base plus one offset per
    // lane, with no per-load address arithmetic.
    constexpr int LOADS = BLOCKS / WAVES;
    static_assert((4 * WAVES) % 16 == 0 && (8 * WAVES) % 16 == 0, "load steps keep the swizzle");
    uint32_t koff, voff;
    {
        const unsigned key = 4 * wave + lane / 16, d = 8 * wave + lane / 8;
        koff = (key * (uint32_t)stride + k_chunk(key, lane % 16) * 8) * 2;
        voff = (d * a.padded + v_chunk(d, lane % 8) * 8) * 2;
    }

    // Dense: buffer loads straight to LDS, a uniform byte offset per load plus
    // the lane's koff / voff (no per-load address arithmetic). In the last
    // tile, lanes whose key is at or past seq take BUFFER_OOB and load zeros
    // (their scores are masked); group ids past the end are clamped.
    const __amdgpu_buffer_rsrc_t krsrc =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.k, (short)0, (int)(uint32_t)((size_t)a.seq * stride * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t vrsrc =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.vt, (short)0, (int)(uint32_t)((size_t)a.heads * D * a.padded * 2),
                                          0x00020000);
    // FULL: the caller has checked a.buffered and that group g's keys are all
    // below seq (neither the global-load path nor the tail select is then
    // compiled into that caller).
    auto load_group = [&](unsigned g, int stage, auto full_tag) {
        constexpr bool FULL = decltype(full_tag)::value;
        uint8_t *base = smem + stage * STAGE;
        if (!SPARSE && (FULL || a.buffered)) {
#pragma unroll
            for (int j = 0; j < KT; j++) {
                const unsigned key0 = min(g * KT + j, count - 1) * BN;
                const bool tail = !FULL && key0 + BN > a.seq;
#pragma unroll
                for (int t = 0; t < LOADS; t++) {
                    const unsigned so = (unsigned)(((size_t)head * D + ((size_t)key0 + 4 * WAVES * t) * stride) * 2);
                    auto *dst = (__attribute__((address_space(3))) void *)(base + j * K_BYTES + (wave + WAVES * t) * 1024);
                    if (tail) {
                        const unsigned key = key0 + 4 * WAVES * t + 4 * wave + lane / 16;
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(krsrc, dst, 16, key < a.seq ? koff : BUFFER_OOB, so, 0, 0);
                    } else {
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(krsrc, dst, 16, koff, so, 0, 0);
                    }
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(
                        vrsrc,
                        (__attribute__((address_space(3))) void *)(base + KT * K_BYTES + j * V_BYTES + (wave + WAVES * t) * 1024),
                        16, voff, (unsigned)(((size_t)head * D * a.padded + (size_t)8 * WAVES * t * a.padded + key0) * 2), 0, 0);
                }
            }
            return;
        }
#pragma unroll
        for (int j = 0; j < KT; j++) {
            const unsigned tile = sub_at(g * KT + j);
            const unsigned key0 = tile * BN;
            uint8_t *ks = base + j * K_BYTES;
            uint8_t *vs = base + KT * K_BYTES + j * V_BYTES;
            if (key0 + BN <= a.seq) {
#pragma unroll
                for (int t = 0; t < LOADS; t++) {
                    const __attribute__((address_space(1))) char *kt =
                        (const __attribute__((address_space(1))) char *)(kh + ((size_t)key0 + 4 * WAVES * t) * stride);
                    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(kt + koff),
                                                     (__attribute__((address_space(3))) void *)(ks + (wave + WAVES * t) * 1024),
                                                     16, 0, 0);
                }
            } else {
#pragma unroll
                for (unsigned b = wave; b < BLOCKS; b += WAVES) {
                    unsigned key = 4 * b + lane / 16, phys = lane % 16;
                    unsigned row = min(key0 + key, a.seq - 1);
                    const uint16_t *src = kh + (size_t)row * stride + k_chunk(key, phys) * 8;
                    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                                     (__attribute__((address_space(3))) void *)(ks + b * 1024), 16, 0, 0);
                }
            }
            // V^T is padded to whole tiles: always a uniform base plus offsets.
#pragma unroll
            for (int t = 0; t < LOADS; t++) {
                const __attribute__((address_space(1))) char *vt = (const __attribute__((address_space(1))) char *)(
                    vth + (size_t)8 * WAVES * t * a.padded + min(key0, a.padded - BN));
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(vt + voff),
                                                 (__attribute__((address_space(3))) void *)(vs + (wave + WAVES * t) * 1024),
                                                 16, 0, 0);
            }
        }
    };

    f32x16 o[4];
#pragma unroll
    for (int md = 0; md < 4; md++) o[md] = f32x16{};
    float m = -1e30f, l = 0.f;
    bool failed = false;   // a P overflowed: these rows are recomputed
    f32x16 lsum = f32x16{};
    bf16x8 ones;
#pragma unroll
    for (int i = 0; i < 8; i++) ones[i] = (__bf16)1.0f;

    if (groups) load_group(0, 0, std::false_type{});
    wait_vm_loads();
    __syncthreads();
    // One group of KT sub-tiles. FULL: a group past the first whose keys are
    // all below seq (dense, NOMAX, buffer loads): no masking, no group max
    // and no global-load path are compiled in. Those groups run in a loop of
    // their own, with the first group and the tail peeled off it, so the loop
    // holds one compact path with no cold branches between its hot code
    // (3.5-4% faster than one loop over all groups). Same arithmetic either
    // way.
    auto group = [&](unsigned g, auto full_tag) {
        constexpr bool FULL = decltype(full_tag)::value;
        const int cur = g & 1;
        if (g + 1 < groups) load_group(g + 1, cur ^ 1, full_tag);
        const uint8_t *base = smem + cur * STAGE;
        f32x16 s[KT][2];
#pragma unroll
        for (int j = 0; j < KT; j++) {
            const uint8_t *ks = base + j * K_BYTES;
            bf16x8 kfr[16];
#pragma unroll
            for (int x = 0; x < 16; x++) {
                const unsigned key = (x % 2) * 32 + n;
                kfr[x] = *reinterpret_cast<const bf16x8 *>(ks + key * 256 + k_chunk(key, (x / 2) * 2 + hf) * 16);
            }
            s[j][0] = f32x16{};
            s[j][1] = f32x16{};
#pragma unroll
            for (int kstep = 0; kstep < 8; kstep++)
#pragma unroll
                for (int mb = 0; mb < 2; mb++)
                    s[j][mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kfr[kstep * 2 + mb], qf[kstep], s[j][mb], 0, 0, 0);
        }
        // Mask keys past the sequence end and sub-tiles past the list end.
        if constexpr (!FULL)
#pragma unroll
        for (int j = 0; j < KT; j++) {
            const unsigned idx = g * KT + j;
            const unsigned tile = sub_at(idx);
            if (idx >= count || tile * BN + BN > a.seq) {
#pragma unroll
                for (int mb = 0; mb < 2; mb++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        unsigned key = tile * BN + mb * 32 + (r / 4) * 8 + hf * 4 + (r % 4);
                        if (idx >= count || key >= a.seq) s[j][mb][r] = -INFINITY;
                    }
            }
        }
        if (!FULL && (!NOMAX || g == 0)) {
        float mx0 = -INFINITY, mx1 = -INFINITY;
#pragma unroll
        for (int j = 0; j < KT; j++)
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                mx0 = fmaxf(fmaxf(mx0, s[j][0][r]), s[j][0][r + 1]);
                mx1 = fmaxf(fmaxf(mx1, s[j][1][r]), s[j][1][r + 1]);
            }
        const float mx = half_max_swap(fmaxf(mx0, mx1)) * c;
        if (__builtin_amdgcn_ballot_w64(mx > m + RESCALE_SLACK)) {
            const float mnew = fmaxf(m, mx);
            const float alpha = exp2f_fast(m - mnew);
            m = mnew;
            if constexpr (MSUM) lsum *= alpha;
            else l *= alpha;
#pragma unroll
            for (int md = 0; md < 4; md++) o[md] *= alpha;
        }
        }
        const float neg = -m;
        int raise = 0;   // exponent m rises by after this group (0 or more)
#pragma unroll
        for (int j = 0; j < KT; j++) {
            const uint8_t *vs = base + KT * K_BYTES + j * V_BYTES;
            bf16x8 vfr[16];
            auto load_v = [&]() {
#pragma unroll
                for (int x = 0; x < 16; x++) {
                    const unsigned d = (x % 4) * 32 + n;
                    vfr[x] = *reinterpret_cast<const bf16x8 *>(vs + d * 128 + v_chunk(d, (x / 4) * 2 + hf) * 16);
                }
            };
            load_v();
            bf16x8 pb[4];
            float psum = 0.f;
#pragma unroll
            for (int mb = 0; mb < 2; mb++)
#pragma unroll
                for (int r = 0; r < 16; r += 2) {
                    float p0 = exp2f_fast(fmaf(s[j][mb][r], c, neg));
                    float p1 = exp2f_fast(fmaf(s[j][mb][r + 1], c, neg));
                    if constexpr (!MSUM) psum += p0 + p1;
                    pb[mb * 2 + r / 8][r % 8] = (__bf16)p0;
                    pb[mb * 2 + r / 8][r % 8 + 1] = (__bf16)p1;
                }
            if constexpr (NOMAX) {
                // Past the first group the running max is raised only when the
                // row's 32-key partial sums leave [0, PSUM_LIMIT], so no
                // per-tile max is computed. Then m rises by e, the largest
                // exponent of the row's partial sums (a bound on every P of the
                // row), after the group's P.V, scaling l and O by 2^-e exactly.
                // A partial sum at or above 2^RETRY_EXP (or not finite: its
                // exponent reads 128) has already put P that large into O,
                // which for large |V| could overflow: the wave flags its rows
                // and the launch that follows recomputes them.
                // Branch-free: a branch here would keep the exponentials from
                // overlapping the P.V products.
                if (!(psum <= PSUM_LIMIT)) raise = max(raise, (int)((__builtin_bit_cast(uint32_t, psum) >> 23) & 0xFF) - 127);
            }
            if constexpr (!MSUM) l += psum;
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
#pragma unroll
                for (int md = 0; md < 4; md++)
                    o[md] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vfr[kk * 4 + md], pb[kk], o[md], 0, 0, 0);
                if constexpr (MSUM) lsum = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ones, pb[kk], lsum, 0, 0, 0);
            }
        }
        if constexpr (NOMAX) {
            if (__builtin_amdgcn_ballot_w64(raise != 0)) {
                // Both lanes of a query (one per 32-key half) take the larger.
                raise = (int)half_max_swap((float)raise);
                failed |= raise >= RETRY_EXP;
                if (raise >= RETRY_EXP) raise = 0;
                const float alpha = ldexpf(1.f, -raise);
                m += (float)raise;
                l *= alpha;
#pragma unroll
                for (int md = 0; md < 4; md++) o[md] *= alpha;
            }
        }
        wait_vm_loads();
        __syncthreads();
    };
    unsigned g0 = 0;
    if constexpr (NOMAX && !SPARSE) {
        if (a.buffered) {
            const unsigned full = a.seq / (KT * BN);
            if (groups) group(0u, std::false_type{});
            // Group g + 1, loaded by group g, must be full as well.
            for (g0 = 1; g0 + 1 < full; g0++) group(g0, std::true_type{});
            g0 = max(g0, 1u);
        }
    }
    for (unsigned g = g0; g < groups; g++) group(g, std::false_type{});

    const float total = MSUM ? lsum[0] : half_sum_swap(l);
    const float inv = total > 0.f ? 1.f / total : 0.f;
    const unsigned q = q0 + wave * 32 + n;
    bool bad = false;
    if (q < qrows) {
        uint16_t *dst = a.out + (a.head_major ? ((size_t)head * a.seq + q) * D : ((size_t)q * a.heads + head) * D);
#pragma unroll
        for (int md = 0; md < 4; md++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                u16x4 w;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    float x = o[md][g4 * 4 + i] * inv;
                    bad |= !finite_f32(x);
                    w[i] = f32_to_bf16(x);
                }
                *reinterpret_cast<u16x4 *>(dst + md * 32 + g4 * 8 + hf * 4) = w;
            }
    }
    if constexpr (NOMAX) {
        // A non-finite output with no flagged partial sum comes from P below
        // 2^RETRY_EXP times a large |V| (or from a non-finite input): the
        // per-tile-max launch recomputes those rows too, and raises the
        // fault only if its own output is not finite.
        failed |= bad;
        const bool any = __builtin_amdgcn_ballot_w64(failed) != 0;
        if (lane == 0) retry[wave] = any ? 1 : 0;
        if (any) return;
    }
    if (bad) a.fault[0] = 1u;
    // m + log2(total) is log2 of sum_j 2^(c s_j) = log2 sum_j e^(scale s_j).
    if (a.lse && hf == 0 && q < qrows) a.lse[(size_t)head * qrows + q] = (m + log2f(total)) * 0.6931471805599453f;
}

template <int KT, bool SPARSE, bool MSUM, bool NOMAX, int WAVES = 8>
int configure_wide(h3_gpu *g) {
    static bool configured = false;
    if (!configured) {
        if (!h3_hip_check(g, hipFuncSetAttribute((const void *)attn_bf16_wide<KT, SPARSE, MSUM, NOMAX, WAVES>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)(2 * KT * STAGE_BYTES)),
                          "attention shared memory"))
            return 0;
        configured = true;
    }
    return 1;
}

// NOMAX: the fast kernel, then the per-tile-max kernel over the workgroups
// the fast one flagged (most of its workgroups exit at once); both inside one
// timing window.
template <int KT, bool SPARSE, bool MSUM, bool NOMAX = false, int WAVES = 8>
int launch_wide(h3_gpu *g, const Args &a, unsigned groups) {
    constexpr size_t shared = 2 * KT * STAGE_BYTES;
    if (!configure_wide<KT, SPARSE, MSUM, false, WAVES>(g)) return 0;
    if (NOMAX && !configure_wide<KT, SPARSE, MSUM, true, WAVES>(g)) return 0;
    hipEvent_t timing = h3_kernel_timing_begin(g);
    hipLaunchKernelGGL((attn_bf16_wide<KT, SPARSE, MSUM, NOMAX, WAVES>), dim3(groups), dim3(64 * WAVES), shared,
                       g->compute, a);
    if (NOMAX) {
        if (!h3_launch_status(g, "BF16 attention")) return 0;
        hipLaunchKernelGGL((attn_bf16_wide<KT, SPARSE, MSUM, false, WAVES>), dim3(groups), dim3(64 * WAVES), shared,
                           g->compute, a);
    }
    h3_kernel_timing_end(g, timing);
    return h3_launch_status(g, "BF16 attention");
}

// ------------------------------------------------------------ hand-scheduled dense kernel
// attn_bf16_pipe: the dense NOMAX kernel's arithmetic (same operations in the
// same order, so its outputs equal attn_bf16_wide<2, false, false, true>'s
// bit for bit) with half the LDS fragment traffic. Four waves of 64 queries
// (two 32-query blocks b = 0, 1), one wave per SIMD: every K or V^T fragment
// read from LDS feeds two MFMAs, one per block. With no second wave on the
// SIMD, the key sweep is one inline-asm block whose instruction order does
// the overlapping (hipcc's schedule for this shape left the exponentials
// between their own MFMAs). Per 64-key sub-tile j the MFMA stream is
//   S0(j) | PV1(j-1) | S1(j) | PV0(j)          (16 MFMAs each)
// and block b's softmax of sub-tile j (32 exponentials per lane, the FP32 row
// sum, P rounded to BF16 in place over its scores) runs under the two phases
// that follow its scores, so its P.V is issued a phase after the last
// exponential. V^T fragments of sub-tile j are read under S1(j), K fragments
// of sub-tile j + 1 under PV0(j). Groups of 128 keys (two sub-tiles) share a
// barrier, placed after the last V^T read of the group; the tiles two groups
// ahead are loaded (buffer_load ... lds) into the stage just released, the
// first right after the barrier, the second in the next group's first phase. The loop body holds two groups, one per stage, so every LDS
// address is a base register plus a constant; K rows past S are caught by
// the buffer's bounds check on the per-lane offset (tile base + row), which
// makes the loads the same for every group. Running max, the row-sum test that raises it, the recomputation
// bytes and the output follow the NOMAX wide kernel; the first group's max is
// computed in C++ before the sweep, and the last group masks keys past S.
//
// Fixed registers inside the sweep:
//   v[0:31]    scores / P of block 0 (v[0:15] keys 0-31, v[16:31] keys 32-63),
//              v[32:63] block 1: clobbered;
//   v[64:127]  O^T of block 0 (channel blocks of 16 registers), v[128:191]
//              block 1: operands bound to these registers;
//   a[0:63]    the 16 K fragments of a sub-tile, a[64:127] the 16 V^T
//              fragments: clobbered;
//   a[128:191] Q fragments (block 0, then block 1): operands.
// LDS (128 KB): K tile j of stage s at 32 KB s + 16 KB j, V^T tile j of
// stage s at 64 KB + 32 KB s + 16 KB j, in the wide kernel's swizzled
// layouts (every read offset then fits the 16-bit ds_read offset).
constexpr int PIPE_STAGE = 2 * (K_BYTES + V_BYTES);   // 64 KB: two 64-key tiles

#define AP_S(b, mb) "v[32*" #b "+16*" #mb ":32*" #b "+16*" #mb "+15]"
#define AP_SR(b, mb, r) "v[32*" #b "+16*" #mb "+" #r "]"
#define AP_P(b, kk) "v[32*" #b "+16*(" #kk "/2)+4*(" #kk "%%2):32*" #b "+16*(" #kk "/2)+4*(" #kk "%%2)+3]"
#define AP_O(b, md) "v[64+64*" #b "+16*" #md ":64+64*" #b "+16*" #md "+15]"
#define AP_K(x) "a[4*(" #x "):4*(" #x ")+3]"
#define AP_V(x) "a[64+4*(" #x "):64+4*(" #x ")+3]"
#define AP_Q(b, ks) "a[128+32*" #b "+4*" #ks ":128+32*" #b "+4*" #ks "+3]"

// Scores of block b (keys x queries): kstep ks of key half mb.
#define AP_SM(b, ks, mb) "v_mfma_f32_32x32x16_bf16 " AP_S(b, mb) ", " AP_K(2*ks+mb) ", " AP_Q(b, ks) ", " AP_S(b, mb) "\n"
#define AP_SM0(b, mb) "v_mfma_f32_32x32x16_bf16 " AP_S(b, mb) ", " AP_K(mb) ", " AP_Q(b, 0) ", 0\n"
// O^T of block b += V^T P^T: channel block md, 16-key chunk kk.
#define AP_PV(b, kk, md) "v_mfma_f32_32x32x16_bf16 " AP_O(b, md) ", " AP_V(4*kk+md) ", " AP_P(b, kk) ", " AP_O(b, md) "\n"

// 16 MFMAs M0..M15 with E_k after M_k.
#define AP_PH(M0, M1, M2, M3, M4, M5, M6, M7, M8, M9, M10, M11, M12, M13, M14, M15, E0, E1, E2, E3, E4, E5, E6, E7, \
              E8, E9, E10, E11, E12, E13, E14, E15)                                                              \
    M0 E0 M1 E1 M2 E2 M3 E3 M4 E4 M5 E5 M6 E6 M7 E7 M8 E8 M9 E9 M10 E10 M11 E11 M12 E12 M13 E13 M14 E14 M15 E15
#define AP_PH_EXP(...) AP_PH(__VA_ARGS__)
#define AP_SMFMA(b) AP_SM0(b, 0), AP_SM0(b, 1), AP_SM(b, 1, 0), AP_SM(b, 1, 1), AP_SM(b, 2, 0), AP_SM(b, 2, 1),       \
    AP_SM(b, 3, 0), AP_SM(b, 3, 1), AP_SM(b, 4, 0), AP_SM(b, 4, 1), AP_SM(b, 5, 0), AP_SM(b, 5, 1), AP_SM(b, 6, 0),    \
    AP_SM(b, 6, 1), AP_SM(b, 7, 0), AP_SM(b, 7, 1)
#define AP_PVMFMA(b) AP_PV(b, 0, 0), AP_PV(b, 0, 1), AP_PV(b, 0, 2), AP_PV(b, 0, 3), AP_PV(b, 1, 0), AP_PV(b, 1, 1),   \
    AP_PV(b, 1, 2), AP_PV(b, 1, 3), AP_PV(b, 2, 0), AP_PV(b, 2, 1), AP_PV(b, 2, 2), AP_PV(b, 2, 3), AP_PV(b, 3, 0),    \
    AP_PV(b, 3, 1), AP_PV(b, 3, 2), AP_PV(b, 3, 3)

// Softmax of scores 8h + 2i, 8h + 2i + 1 of key half mb of block b, in two
// parts: A computes p = exp2(fma(s, c, -m)) in place, B adds p0 + p1 to psum
// and writes the BF16 pair over score 4h + i. At least one instruction must
// separate a v_exp_f32 from the first VALU that reads its result (gfx950's
// transcendental forwarding hazard: read right after, the result is stale in
// part of the wave), so B always follows A after an MFMA or another A.
#define AP_A(b, mb, h, i)                                                                                         \
    "v_fma_f32 " AP_SR(b, mb, 8*h+2*i) ", " AP_SR(b, mb, 8*h+2*i) ", %[c], %[nm" #b "]\n"                          \
    "v_fma_f32 " AP_SR(b, mb, 8*h+2*i+1) ", " AP_SR(b, mb, 8*h+2*i+1) ", %[c], %[nm" #b "]\n"                      \
    "v_exp_f32 " AP_SR(b, mb, 8*h+2*i) ", " AP_SR(b, mb, 8*h+2*i) "\n"                                             \
    "v_exp_f32 " AP_SR(b, mb, 8*h+2*i+1) ", " AP_SR(b, mb, 8*h+2*i+1) "\n"
#define AP_B(b, mb, h, i)                                                                                         \
    "v_add_f32 %[t" #b "], " AP_SR(b, mb, 8*h+2*i) ", " AP_SR(b, mb, 8*h+2*i+1) "\n"                                \
    "v_add_f32 %[ps" #b "], %[ps" #b "], %[t" #b "]\n"                                                             \
    "v_cvt_pk_bf16_f32 " AP_SR(b, mb, 4*h+i) ", " AP_SR(b, mb, 8*h+2*i) ", " AP_SR(b, mb, 8*h+2*i+1) "\n"
// Last group: score r of half mb is key tile*64 + 32 mb + 8 (r / 4) + 4 hf + r % 4;
// lim<J> = S - tile*64 - 4 hf, and keys at or past S score -inf.
#define AP_KEEP(b, mb, r, J)                                                                                      \
    "v_cmp_lt_i32 vcc, 32*" #mb "+8*((" #r ")/4)+((" #r ")%%4), %[lim" #J "]\n"                                       \
    "v_cndmask_b32 " AP_SR(b, mb, r) ", %[ninf], " AP_SR(b, mb, r) ", vcc\n"
// Part A unmasked (AP_UA) or masked with lim<J> (AP_MA).
#define AP_UA(b, mb, h, i, J) AP_A(b, mb, h, i)
#define AP_MA(b, mb, h, i, J) AP_KEEP(b, mb, 8*h+2*i, J) AP_KEEP(b, mb, 8*h+2*i+1, J) AP_A(b, mb, h, i)
// A whole 16-key chunk (mb, h) with nothing to interleave: A0 A1 B0 A2 B1 A3 B2 (nop) B3.
#define AP_CHUNK(b, mb, h, U, J)                                                                                  \
    U(b, mb, h, 0, J) U(b, mb, h, 1, J) AP_B(b, mb, h, 0) U(b, mb, h, 2, J) AP_B(b, mb, h, 1) U(b, mb, h, 3, J)     \
    AP_B(b, mb, h, 2) "s_nop 0\n" AP_B(b, mb, h, 3)

// After a sub-tile of block b: l += psum; the row-sum test (psum not below
// 2^20: raise = max(raise, exponent of psum)); psum = 0.
#define AP_FIN(b)                                                                                                 \
    "v_add_f32 %[l" #b "], %[l" #b "], %[ps" #b "]\n"                                                              \
    "v_cmp_nge_f32 vcc, 0x49800000, %[ps" #b "]\n"                                                                \
    "v_bfe_u32 %[t" #b "], %[ps" #b "], 23, 8\n"                                                                  \
    "v_subrev_u32 %[t" #b "], 127, %[t" #b "]\n"                                                                  \
    "v_max_i32 %[t" #b "], %[r" #b "], %[t" #b "]\n"                                                              \
    "v_cndmask_b32 %[r" #b "], %[r" #b "], %[t" #b "], vcc\n"                                                    \
    "v_mov_b32 %[ps" #b "], 0\n"

#define AP_OMUL(b, md, e) "v_mul_f32 v[64+64*" #b "+16*" #md "+" #e "], v[64+64*" #b "+16*" #md "+" #e "], %[t" #b "]\n"
#define AP_OMUL16(b, md) AP_OMUL(b, md, 0) AP_OMUL(b, md, 1) AP_OMUL(b, md, 2) AP_OMUL(b, md, 3) AP_OMUL(b, md, 4)     \
    AP_OMUL(b, md, 5) AP_OMUL(b, md, 6) AP_OMUL(b, md, 7) AP_OMUL(b, md, 8) AP_OMUL(b, md, 9) AP_OMUL(b, md, 10)      \
    AP_OMUL(b, md, 11) AP_OMUL(b, md, 12) AP_OMUL(b, md, 13) AP_OMUL(b, md, 14) AP_OMUL(b, md, 15)
// End of a group for block b: when any lane's raise is set, both lanes of a
// query take the larger; a raise of 32 or more marks the rows for the
// recomputation launch (and is dropped); m rises by raise, l and O^T scale by
// 2^-raise. The wait covers P.V MFMAs of the block still in flight. L: a
// label unique within the asm block.
#define AP_GEND(b, L)                                                                                             \
    "v_cmp_ne_u32 vcc, 0, %[r" #b "]\n"                                                                           \
    "s_cbranch_vccz ap_" #L "_%=\n"                                                                               \
    "s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n"                             \
    "v_cvt_f32_i32 %[t" #b "], %[r" #b "]\n"                                                                       \
    "v_mov_b32 %[u" #b "], %[t" #b "]\n"                                                                           \
    "s_nop 1\n"                                                                                                    \
    "v_permlane32_swap_b32 %[t" #b "], %[u" #b "]\n"                                                               \
    "v_max_f32 %[t" #b "], %[t" #b "], %[u" #b "]\n"                                                               \
    "v_cvt_i32_f32 %[r" #b "], %[t" #b "]\n"                                                                       \
    "v_cmp_le_i32 vcc, 32, %[r" #b "]\n"                                                                          \
    "v_cndmask_b32_e64 %[f" #b "], %[f" #b "], 1, vcc\n"                                                          \
    "v_cndmask_b32_e64 %[r" #b "], %[r" #b "], 0, vcc\n"                                                          \
    "v_sub_u32 %[t" #b "], 0, %[r" #b "]\n"                                                                        \
    "v_ldexp_f32 %[t" #b "], 1.0, %[t" #b "]\n"                                                                    \
    "v_cvt_f32_i32 %[u" #b "], %[r" #b "]\n"                                                                       \
    "v_sub_f32 %[nm" #b "], %[nm" #b "], %[u" #b "]\n"                                                             \
    "v_mul_f32 %[l" #b "], %[l" #b "], %[t" #b "]\n"                                                               \
    AP_OMUL16(b, 0) AP_OMUL16(b, 1) AP_OMUL16(b, 2) AP_OMUL16(b, 3)                                               \
    "ap_" #L "_%=:\n"                                                                                             \
    "v_mov_b32 %[r" #b "], 0\n"

// Fragment reads: K fragment (ks, mb) of tile J of stage ST; V^T fragment
// (kk, md) of tile J of stage ST (the V^T bases include the 64 KB).
#define AP_RK(ks, mb, J, ST) "ds_read_b128 " AP_K(2*ks+mb) ", %[kb" #ks "] offset:" #mb "*8192+" #J "*16384+" #ST "*32768\n"
#define AP_RV(kk, md, J, ST) "ds_read_b128 " AP_V(4*kk+md) ", %[vb" #kk "] offset:" #md "*4096+" #J "*16384+" #ST "*32768\n"

// Loads of the tile lt (clamped to the last tile) into slot J of stage ST:
// K rows 16 T + 4 wave + lane / 16 at per-lane offset ko<T> + tile base (rows
// at or past S are out of the buffer's range and load zeros), V^T channel
// rows 32 T + 8 wave + lane / 8.
#define AP_LTILE                                                                                                  \
    "s_min_u32 %[tt], %[lt], %[tmax]\n"                                                                           \
    "s_mul_i32 %[sk], %[tt], %[k64]\n"                                                                            \
    "s_lshl_b32 %[sv], %[tt], 7\n"                                                                                \
    "s_add_u32 %[sv], %[sv], %[hv]\n"                                                                             \
    "s_add_u32 %[lt], %[lt], 1\n"
#define AP_LK(ST, J, T, TV)                                                                                       \
    "s_add_u32 m0, %[mc], " #ST "*32768+" #J "*16384+" #T "*4096\n"                                                \
    "v_add_u32 %[" #TV "], %[sk], %[ko" #T "]\n"                                                                   \
    "buffer_load_dwordx4 %[" #TV "], %[kr], %[hk] offen lds\n"
#define AP_LV(ST, J, T)                                                                                           \
    "s_add_u32 m0, %[mc], 65536+" #ST "*32768+" #J "*16384+" #T "*4096\n"                                          \
    "buffer_load_dwordx4 %[vo], %[vr], %[sv] offen lds\n"                                                         \
    "s_add_u32 %[sv], %[sv], %[v32]\n"

// Phase slot lists (16 extras each). Softmax pair i of a phase: part A in
// slot 2i, part B in slot 2i + 1.
// Phase 1: block 1's softmax of the previous sub-tile, key half 1 (U: AP_UA or AP_MA, J).
#define AP_X1(U, J) U(1, 1, 0, 0, J), AP_B(1, 1, 0, 0), U(1, 1, 0, 1, J), AP_B(1, 1, 0, 1), U(1, 1, 0, 2, J),        \
    AP_B(1, 1, 0, 2), U(1, 1, 0, 3, J), AP_B(1, 1, 0, 3), U(1, 1, 1, 0, J), AP_B(1, 1, 1, 0), U(1, 1, 1, 1, J),        \
    AP_B(1, 1, 1, 1), U(1, 1, 1, 2, J), AP_B(1, 1, 1, 2), U(1, 1, 1, 3, J), AP_B(1, 1, 1, 3) AP_FIN(1)
#define AP_X1_NONE "", "", "", "", "", "", "", "", "", "", "", "", "", "", "", ""
// Phase 1 with the second tile's loads of the previous group (B0..B7, one
// ahead of each part A: memory instructions go before the exponentials).
#define AP_X1L(U, J, B0, B1, B2, B3, B4, B5, B6, B7)                                                              \
    B0 U(1, 1, 0, 0, J), AP_B(1, 1, 0, 0), B1 U(1, 1, 0, 1, J), AP_B(1, 1, 0, 1), B2 U(1, 1, 0, 2, J),                  \
    AP_B(1, 1, 0, 2), B3 U(1, 1, 0, 3, J), AP_B(1, 1, 0, 3), B4 U(1, 1, 1, 0, J), AP_B(1, 1, 1, 0),                     \
    B5 U(1, 1, 1, 1, J), AP_B(1, 1, 1, 1), B6 U(1, 1, 1, 2, J), AP_B(1, 1, 1, 2), B7 U(1, 1, 1, 3, J),                  \
    AP_B(1, 1, 1, 3) AP_FIN(1)
#define AP_X1L_EXP(...) AP_X1L(__VA_ARGS__)
// Phase 2: G (group end of block 0 or nothing), block 0's softmax, half 0.
#define AP_X2(G, U, J) G U(0, 0, 0, 0, J), AP_B(0, 0, 0, 0), U(0, 0, 0, 1, J), AP_B(0, 0, 0, 1), U(0, 0, 0, 2, J),    \
    AP_B(0, 0, 0, 2), U(0, 0, 0, 3, J), AP_B(0, 0, 0, 3), U(0, 0, 1, 0, J), AP_B(0, 0, 1, 0), U(0, 0, 1, 1, J),        \
    AP_B(0, 0, 1, 1), U(0, 0, 1, 2, J), AP_B(0, 0, 1, 2), U(0, 0, 1, 3, J), AP_B(0, 0, 1, 3)
// Phase 3: G (group end of block 1 or nothing), V^T reads of tile J of stage
// ST, block 0's softmax of half 1, its sub-tile end.
#define AP_X3(G, U, J, ST) G AP_RV(0, 0, J, ST) AP_RV(0, 1, J, ST) U(0, 1, 0, 0, J),                                 \
    AP_RV(0, 2, J, ST) AP_RV(0, 3, J, ST) AP_B(0, 1, 0, 0), AP_RV(1, 0, J, ST) U(0, 1, 0, 1, J),                      \
    AP_RV(1, 1, J, ST) AP_RV(1, 2, J, ST) AP_B(0, 1, 0, 1), AP_RV(1, 3, J, ST) U(0, 1, 0, 2, J),                      \
    AP_RV(2, 0, J, ST) AP_RV(2, 1, J, ST) AP_B(0, 1, 0, 2), AP_RV(2, 2, J, ST) U(0, 1, 0, 3, J),                      \
    AP_RV(2, 3, J, ST) AP_RV(3, 0, J, ST) AP_B(0, 1, 0, 3), AP_RV(3, 1, J, ST) U(0, 1, 1, 0, J),                      \
    AP_RV(3, 2, J, ST) AP_RV(3, 3, J, ST) AP_B(0, 1, 1, 0), U(0, 1, 1, 1, J), AP_B(0, 1, 1, 1), U(0, 1, 1, 2, J),     \
    AP_B(0, 1, 1, 2), U(0, 1, 1, 3, J), AP_B(0, 1, 1, 3) AP_FIN(0)
// Phase 4: K reads (tile KJ of stage KS), block 1's softmax of half 0, and
// the loads of the tiles two groups ahead (AP_L4(ST) into stage ST, or
// AP_LNONE(ST)).
#define AP_X4(KJ, KS, U, J, L0, L1, L2, L3, L4, L5, L6, L7)                                                         \
    AP_RK(0, 0, KJ, KS) AP_RK(0, 1, KJ, KS) U(1, 0, 0, 0, J), AP_RK(1, 0, KJ, KS) L0 AP_B(1, 0, 0, 0),                \
    AP_RK(1, 1, KJ, KS) AP_RK(2, 0, KJ, KS) U(1, 0, 0, 1, J), AP_RK(2, 1, KJ, KS) L1 AP_B(1, 0, 0, 1),                \
    AP_RK(3, 0, KJ, KS) AP_RK(3, 1, KJ, KS) U(1, 0, 0, 2, J), AP_RK(4, 0, KJ, KS) L2 AP_B(1, 0, 0, 2),                \
    AP_RK(4, 1, KJ, KS) AP_RK(5, 0, KJ, KS) U(1, 0, 0, 3, J), AP_RK(5, 1, KJ, KS) L3 AP_B(1, 0, 0, 3),                \
    AP_RK(6, 0, KJ, KS) AP_RK(6, 1, KJ, KS) U(1, 0, 1, 0, J), AP_RK(7, 0, KJ, KS) L4 AP_B(1, 0, 1, 0),                \
    AP_RK(7, 1, KJ, KS) U(1, 0, 1, 1, J), L5 AP_B(1, 0, 1, 1), U(1, 0, 1, 2, J), L6 AP_B(1, 0, 1, 2),                 \
    U(1, 0, 1, 3, J), L7 AP_B(1, 0, 1, 3)
// The loads of one tile J (eight 1 KB blocks per wave: four of K, four of
// V^T) as eight slots. A group's two tiles are loaded in two phases: tile 0
// in its last phase (AP_L4), tile 1 in the next group's first (AP_LB), so
// that the four waves, which leave the barrier together, do not queue
// sixteen loads each at once behind the texture unit. The next group's
// barrier waits for both.
#define AP_LT(ST, J) AP_LTILE AP_LK(ST, J, 0, tl0), AP_LV(ST, J, 0), AP_LK(ST, J, 1, tl1), AP_LV(ST, J, 1),               \
    AP_LK(ST, J, 2, tl0), AP_LV(ST, J, 2), AP_LK(ST, J, 3, tl1), AP_LV(ST, J, 3)
#define AP_L4(ST) AP_LT(ST, 0)
#define AP_LB(ST) AP_LT(ST, 1)
#define AP_L4_NONE "", "", "", "", "", "", "", ""
#define AP_LNONE(ST) AP_L4_NONE
#define AP_X4_EXP(...) AP_X4(__VA_ARGS__)

#define AP_WAIT_LDS "s_waitcnt lgkmcnt(0)\n"

// One group (sub-tiles 0 and 1) in stage ST, the next group in stage OT. U0 /
// U1: the part-A macro for the softmax of sub-tiles 0 and 1 (AP_MA masks with
// lim0 / lim1), UP: for block 1's previous sub-tile in phase 1 of sub-tile 0
// (the last sub-tile of the previous group); LD: AP_L4 or AP_LNONE; LP: AP_LB
// (the previous group's second tile, loaded in the first phase) or AP_LNONE.
#define AP_GROUP(UP, JP, U0, U1, L, ST, OT, LD, LP)                                                               \
    AP_PH_EXP(AP_SMFMA(0), AP_X1L_EXP(UP, JP, LP(OT)))                                                            \
    AP_PH_EXP(AP_PVMFMA(1), AP_X2(AP_GEND(0, L##a), U0, 0))                                                       \
    AP_PH_EXP(AP_SMFMA(1), AP_X3(AP_GEND(1, L##b), U0, 0, ST))                                                    \
    AP_WAIT_LDS                                                                                                   \
    AP_PH_EXP(AP_PVMFMA(0), AP_X4_EXP(1, ST, U0, 0, AP_L4_NONE))                                                  \
    AP_WAIT_LDS                                                                                                   \
    AP_PH_EXP(AP_SMFMA(0), AP_X1(U0, 0))                                                                          \
    AP_PH_EXP(AP_PVMFMA(1), AP_X2("", U1, 1))                                                                     \
    AP_PH_EXP(AP_SMFMA(1), AP_X3("", U1, 1, ST))                                                                  \
    "s_waitcnt vmcnt(0) lgkmcnt(0)\n"                                                                             \
    "s_barrier\n"                                                                                                 \
    AP_PH_EXP(AP_PVMFMA(0), AP_X4_EXP(0, OT, U1, 1, LD(ST)))                                                      \
    AP_WAIT_LDS
#define AP_GROUP_FIRST                                                                                            \
    AP_PH_EXP(AP_SMFMA(0), AP_X1_NONE)                                                                            \
    "s_nop 7\n s_nop 7\n s_nop 7\n"                                                                               \
    AP_CHUNK(0, 0, 0, AP_UA, 0) AP_CHUNK(0, 0, 1, AP_UA, 0)                                                       \
    AP_PH_EXP(AP_SMFMA(1), AP_X3("", AP_UA, 0, 0))                                                                \
    AP_WAIT_LDS                                                                                                   \
    AP_PH_EXP(AP_PVMFMA(0), AP_X4_EXP(1, 0, AP_UA, 0, AP_L4_NONE))                                                \
    AP_WAIT_LDS                                                                                                   \
    AP_PH_EXP(AP_SMFMA(0), AP_X1(AP_UA, 0))                                                                       \
    AP_PH_EXP(AP_PVMFMA(1), AP_X2("", AP_UA, 1))                                                                  \
    AP_PH_EXP(AP_SMFMA(1), AP_X3("", AP_UA, 1, 0))                                                                \
    "s_waitcnt vmcnt(0) lgkmcnt(0)\n"                                                                             \
    "s_barrier\n"                                                                                                 \
    AP_PH_EXP(AP_PVMFMA(0), AP_X4_EXP(0, 1, AP_UA, 1, AP_L4(0)))                                                  \
    AP_WAIT_LDS
// Moves the fragment bases from stage 0 to stage 1, for a last group in
// stage 1 (its code is written for stage 0).
#define AP_BASE1 "v_add_u32 %[kb0], 0x8000, %[kb0]\n v_add_u32 %[kb1], 0x8000, %[kb1]\n"                              \
    "v_add_u32 %[kb2], 0x8000, %[kb2]\n v_add_u32 %[kb3], 0x8000, %[kb3]\n v_add_u32 %[kb4], 0x8000, %[kb4]\n"         \
    "v_add_u32 %[kb5], 0x8000, %[kb5]\n v_add_u32 %[kb6], 0x8000, %[kb6]\n v_add_u32 %[kb7], 0x8000, %[kb7]\n"         \
    "v_add_u32 %[vb0], 0x8000, %[vb0]\n v_add_u32 %[vb1], 0x8000, %[vb1]\n v_add_u32 %[vb2], 0x8000, %[vb2]\n"         \
    "v_add_u32 %[vb3], 0x8000, %[vb3]\n"
// Last sub-tile of the last group: block 1's softmax (masked with lim1) and
// P.V, both blocks' group ends, and a wait for every MFMA result before the
// accumulators leave the asm block.
#define AP_TAIL                                                                                                   \
    AP_CHUNK(1, 1, 0, AP_MA, 1) AP_CHUNK(1, 1, 1, AP_MA, 1) AP_FIN(1)                                             \
    AP_GEND(0, e0)                                                                                                \
    AP_PH_EXP(AP_PVMFMA(1), AP_X1_NONE)                                                                           \
    AP_GEND(1, e1)                                                                                                \
    "s_waitcnt vmcnt(0) lgkmcnt(0)\n"                                                                             \
    "s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n"

#define AP_CL10(p, x) #p #x "0", #p #x "1", #p #x "2", #p #x "3", #p #x "4", #p #x "5", #p #x "6", #p #x "7",          \
    #p #x "8", #p #x "9"
#define AP_CLOBBERS                                                                                               \
    "v0", "v1", "v2", "v3", "v4", "v5", "v6", "v7", "v8", "v9", AP_CL10(v, 1), AP_CL10(v, 2), AP_CL10(v, 3),           \
    AP_CL10(v, 4), AP_CL10(v, 5), "v60", "v61", "v62", "v63",                                                      \
    "a0", "a1", "a2", "a3", "a4", "a5", "a6", "a7", "a8", "a9", AP_CL10(a, 1), AP_CL10(a, 2), AP_CL10(a, 3),           \
    AP_CL10(a, 4), AP_CL10(a, 5), AP_CL10(a, 6), AP_CL10(a, 7), AP_CL10(a, 8), AP_CL10(a, 9), AP_CL10(a, 10),          \
    AP_CL10(a, 11), "a120", "a121", "a122", "a123", "a124", "a125", "a126", "a127",                               \
    "m0", "vcc", "scc", "memory"

__global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
void attn_bf16_pipe(Args a) {
    constexpr int WAVES = 4, BM = 256;
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    const unsigned tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / 64), lane = tid % 64;
    const unsigned n = lane % 32, hf = lane / 32;
    const unsigned nqb = (a.seq + BM - 1) / BM;
    const unsigned id = xcd_remap(blockIdx.x, gridDim.x);
    const unsigned head = __builtin_amdgcn_readfirstlane(id / nqb), qb = __builtin_amdgcn_readfirstlane(id % nqb);
    const unsigned q0 = qb * BM;
    uint8_t *const retry = a.retry + ((size_t)head * nqb + qb) * 8;
    const size_t stride = (size_t)a.heads * D;
    const uint16_t *qh = a.q + (size_t)head * D;
    const float c = a.scale_log2;
    const unsigned count = (a.seq + BN - 1) / BN;        // 64-key tiles
    const unsigned groups = (count + 1) / 2;             // the launcher ensures groups >= 3

    // Q fragments of both blocks (rows past S repeat the last row).
    bf16x8 qf[2][8];
    {
        bool bad = false;
#pragma unroll
        for (int b = 0; b < 2; b++) {
            unsigned row = q0 + wave * 64 + b * 32 + n;
            row = row < a.seq ? row : a.seq - 1;
            const uint16_t *p = qh + (size_t)row * stride + hf * 8;
#pragma unroll
            for (int ks = 0; ks < 8; ks++) {
                qf[b][ks] = *reinterpret_cast<const bf16x8 *>(p + ks * 16);
                bad |= bf16_vec_nonfinite(qf[b][ks]);
            }
        }
        if (bad) a.fault[0] = 1u;
    }

    // Tile loads (the layout of the wide kernel at four waves): K block
    // wave + 4 t holds keys 16 t + 4 wave + lane / 16, V^T block wave + 4 t
    // channels 32 t + 8 wave + lane / 8. Buffer offsets: K from the head's
    // first channel, V^T from its first row; keys past S load zeros.
    const unsigned kstride = (unsigned)(stride * 2);
    const unsigned lk = 4 * wave + lane / 16, ld = 8 * wave + lane / 8;
    const unsigned koff = lk * kstride + k_chunk(lk, lane % 16) * 16;
    const unsigned ko1 = koff + 16 * kstride, ko2 = koff + 32 * kstride, ko3 = koff + 48 * kstride;
    const unsigned voff = (ld * a.padded + v_chunk(ld, lane % 8) * 8) * 2;
    const i32x4 kr = {(int)__builtin_amdgcn_readfirstlane((unsigned)(uint64_t)a.k),
                      (int)__builtin_amdgcn_readfirstlane((unsigned)((uint64_t)a.k >> 32)),
                      (int)__builtin_amdgcn_readfirstlane((unsigned)((size_t)a.seq * stride * 2)), 0x00020000};
    const i32x4 vr = {(int)__builtin_amdgcn_readfirstlane((unsigned)(uint64_t)a.vt),
                      (int)__builtin_amdgcn_readfirstlane((unsigned)((uint64_t)a.vt >> 32)),
                      (int)__builtin_amdgcn_readfirstlane((unsigned)((size_t)a.heads * D * a.padded * 2)), 0x00020000};
    const unsigned hk = __builtin_amdgcn_readfirstlane(head * D * 2);
    const unsigned hv = __builtin_amdgcn_readfirstlane(head * D * a.padded * 2);
    const unsigned k64 = __builtin_amdgcn_readfirstlane(64 * kstride);
    const unsigned v32 = __builtin_amdgcn_readfirstlane(32 * a.padded * 2);
    const unsigned tmax = count - 1;
    // Tiles 0..3 (groups 0 and 1) into stages 0 and 1.
#pragma unroll
    for (int t4 = 0; t4 < 4; t4++) {
        const unsigned tile = min((unsigned)t4, tmax);
        uint8_t *base = smem + (t4 / 2) * 2 * K_BYTES + (t4 % 2) * K_BYTES;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const unsigned key = tile * BN + 16 * t + lk;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                *reinterpret_cast<const __amdgpu_buffer_rsrc_t *>(&kr),
                (__attribute__((address_space(3))) void *)(base + (wave + 4 * t) * 1024), 16,
                key < a.seq ? koff : BUFFER_OOB, hk + (tile * BN + 16 * t) * kstride, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                *reinterpret_cast<const __amdgpu_buffer_rsrc_t *>(&vr),
                (__attribute__((address_space(3))) void *)(base + PIPE_STAGE + (wave + 4 * t) * 1024), 16, voff,
                hv + 32 * t * a.padded * 2 + tile * BN * 2, 0, 0);
        }
    }
    wait_vm_loads();
    __syncthreads();

    // Fragment bases (stage 0, tile 0): K fragment (ks, mb) at kb + 8 KB mb,
    // V^T fragment (kk, md) at vb + 4 KB md.
    unsigned kc[8], vc[4];
#pragma unroll
    for (int ks = 0; ks < 8; ks++) kc[ks] = n * 256 + k_chunk(n, 2 * ks + hf) * 16;
#pragma unroll
    for (int kk = 0; kk < 4; kk++) vc[kk] = PIPE_STAGE + n * 128 + v_chunk(n, 2 * kk + hf) * 16;

    // The running max of each block: the first group's score max (as the
    // wide kernel's first group sets it from m = -1e30).
    float nm[2];
#pragma unroll
    for (int b = 0; b < 2; b++) {
        float mx0 = -INFINITY, mx1 = -INFINITY;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            f32x16 s0 = f32x16{}, s1 = f32x16{};
#pragma unroll
            for (int ks = 0; ks < 8; ks++) {
                const bf16x8 k0 = *reinterpret_cast<const bf16x8 *>(smem + j * K_BYTES + kc[ks]);
                const bf16x8 k1 = *reinterpret_cast<const bf16x8 *>(smem + j * K_BYTES + kc[ks] + 8192);
                s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k0, qf[b][ks], s0, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k1, qf[b][ks], s1, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                mx0 = fmaxf(fmaxf(mx0, s0[r]), s0[r + 1]);
                mx1 = fmaxf(fmaxf(mx1, s1[r]), s1[r + 1]);
            }
        }
        const float mx = half_max_swap(fmaxf(mx0, mx1)) * c;
        nm[b] = -fmaxf(-1e30f, mx);
    }

    f32x16 o0[4], o1[4];
#pragma unroll
    for (int md = 0; md < 4; md++) { o0[md] = f32x16{}; o1[md] = f32x16{}; }
    float l0 = 0.f, l1 = 0.f, ps0 = 0.f, ps1 = 0.f;
    int r0 = 0, r1 = 0, f0 = 0, f1 = 0;
    const unsigned mc = __builtin_amdgcn_readfirstlane(wave * 1024);   // this wave's 1 KB load blocks
    unsigned lt = 4, gl = groups - 2;                                    // gl: groups between the first and last
    const unsigned last_stage = (groups - 1) & 1;
    const unsigned last0 = 2 * (groups - 1) * BN;
    const int lim0 = (int)a.seq - (int)last0 - 4 * (int)hf, lim1 = lim0 - BN;
    const float ninf = -INFINITY;
    float t0, t1, u0, u1;
    unsigned tl0, tl1, tt, sk, sv;
    // Group 0 in stage 0; the middle groups in a loop of two groups (stages
    // 1, 0) left after its first half when their count is odd; the last group
    // (no loads) in stage-0 code, its bases moved to stage 1 when it is there.
    asm volatile(
        AP_RK(0, 0, 0, 0) AP_RK(0, 1, 0, 0) AP_RK(1, 0, 0, 0) AP_RK(1, 1, 0, 0) AP_RK(2, 0, 0, 0) AP_RK(2, 1, 0, 0)
        AP_RK(3, 0, 0, 0) AP_RK(3, 1, 0, 0) AP_RK(4, 0, 0, 0) AP_RK(4, 1, 0, 0) AP_RK(5, 0, 0, 0) AP_RK(5, 1, 0, 0)
        AP_RK(6, 0, 0, 0) AP_RK(6, 1, 0, 0) AP_RK(7, 0, 0, 0) AP_RK(7, 1, 0, 0)
        AP_WAIT_LDS
        AP_GROUP_FIRST
        "s_cmp_eq_u32 %[gl], 0\n"
        "s_cbranch_scc1 ap_loop_end_%=\n"
        "ap_loop_%=:\n"
        AP_GROUP(AP_UA, 0, AP_UA, AP_UA, gp, 1, 0, AP_L4, AP_LB)
        "s_sub_u32 %[gl], %[gl], 1\n"
        "s_cmp_eq_u32 %[gl], 0\n"
        "s_cbranch_scc1 ap_loop_end_%=\n"
        AP_GROUP(AP_UA, 0, AP_UA, AP_UA, gq, 0, 1, AP_L4, AP_LB)
        "s_sub_u32 %[gl], %[gl], 1\n"
        "s_cmp_lg_u32 %[gl], 0\n"
        "s_cbranch_scc1 ap_loop_%=\n"
        "ap_loop_end_%=:\n"
        "s_cmp_eq_u32 %[ls], 0\n"
        "s_cbranch_scc1 ap_last0_%=\n"
        AP_BASE1
        "ap_last0_%=:\n"
        AP_GROUP(AP_UA, 0, AP_MA, AP_MA, gl, 0, 1, AP_LNONE, AP_LNONE)
        AP_TAIL
        : [o00] "+{v[64:79]}"(o0[0]), [o01] "+{v[80:95]}"(o0[1]), [o02] "+{v[96:111]}"(o0[2]),
          [o03] "+{v[112:127]}"(o0[3]), [o10] "+{v[128:143]}"(o1[0]), [o11] "+{v[144:159]}"(o1[1]),
          [o12] "+{v[160:175]}"(o1[2]), [o13] "+{v[176:191]}"(o1[3]),
          [nm0] "+v"(nm[0]), [nm1] "+v"(nm[1]), [l0] "+v"(l0), [l1] "+v"(l1), [ps0] "+v"(ps0), [ps1] "+v"(ps1),
          [r0] "+v"(r0), [r1] "+v"(r1), [f0] "+v"(f0), [f1] "+v"(f1),
          [kb0] "+v"(kc[0]), [kb1] "+v"(kc[1]), [kb2] "+v"(kc[2]), [kb3] "+v"(kc[3]), [kb4] "+v"(kc[4]),
          [kb5] "+v"(kc[5]), [kb6] "+v"(kc[6]), [kb7] "+v"(kc[7]), [vb0] "+v"(vc[0]), [vb1] "+v"(vc[1]),
          [vb2] "+v"(vc[2]), [vb3] "+v"(vc[3]),
          [lt] "+s"(lt), [gl] "+s"(gl),
          [t0] "=&v"(t0), [t1] "=&v"(t1), [u0] "=&v"(u0), [u1] "=&v"(u1), [tl0] "=&v"(tl0), [tl1] "=&v"(tl1),
          [tt] "=&s"(tt), [sk] "=&s"(sk), [sv] "=&s"(sv)
        : [q00] "{a[128:131]}"(qf[0][0]), [q01] "{a[132:135]}"(qf[0][1]), [q02] "{a[136:139]}"(qf[0][2]),
          [q03] "{a[140:143]}"(qf[0][3]), [q04] "{a[144:147]}"(qf[0][4]), [q05] "{a[148:151]}"(qf[0][5]),
          [q06] "{a[152:155]}"(qf[0][6]), [q07] "{a[156:159]}"(qf[0][7]), [q10] "{a[160:163]}"(qf[1][0]),
          [q11] "{a[164:167]}"(qf[1][1]), [q12] "{a[168:171]}"(qf[1][2]), [q13] "{a[172:175]}"(qf[1][3]),
          [q14] "{a[176:179]}"(qf[1][4]), [q15] "{a[180:183]}"(qf[1][5]), [q16] "{a[184:187]}"(qf[1][6]),
          [q17] "{a[188:191]}"(qf[1][7]),
          [c] "s"(c), [kr] "s"(kr), [vr] "s"(vr), [tmax] "s"(tmax), [k64] "s"(k64), [hk] "s"(hk),
          [hv] "s"(hv), [v32] "s"(v32), [mc] "s"(mc), [ls] "s"(last_stage),
          [ko0] "v"(koff), [ko1] "v"(ko1), [ko2] "v"(ko2), [ko3] "v"(ko3), [vo] "v"(voff), [ninf] "v"(ninf),
          [lim0] "v"(lim0), [lim1] "v"(lim1)
        : AP_CLOBBERS);

    // Output: O^T / l for each block; rows whose row sum overflowed (or whose
    // output is not finite) are left to the recomputation launch.
#pragma unroll
    for (int b = 0; b < 2; b++) {
        const f32x16 *o = b ? o1 : o0;
        const float total = half_sum_swap(b ? l1 : l0);
        const float inv = total > 0.f ? 1.f / total : 0.f;
        const unsigned q = q0 + wave * 64 + b * 32 + n;
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
                        float x = o[md][g4 * 4 + i] * inv;
                        bad |= !finite_f32(x);
                        w[i] = f32_to_bf16(x);
                    }
                    *reinterpret_cast<u16x4 *>(dst + md * 32 + g4 * 8 + hf * 4) = w;
                }
        }
        const bool failed = (b ? f1 : f0) != 0 || bad;
        const bool any = __builtin_amdgcn_ballot_w64(failed) != 0;
        if (lane == 0) retry[2 * wave + b] = any ? 1 : 0;
    }
}

int launch_pipe_attention(h3_gpu *g, const Args &a) {
    constexpr size_t shared = 2 * PIPE_STAGE;
    static bool configured = false;
    if (!configured) {
        if (!h3_hip_check(g, hipFuncSetAttribute((const void *)attn_bf16_pipe, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)shared), "attention shared memory"))
            return 0;
        configured = true;
    }
    if (!configure_wide<2, false, false, false, 8>(g)) return 0;
    const unsigned groups = (a.seq + 255) / 256 * a.heads;
    hipEvent_t timing = h3_kernel_timing_begin(g);
    hipLaunchKernelGGL(attn_bf16_pipe, dim3(groups), dim3(256), shared, g->compute, a);
    if (!h3_launch_status(g, "BF16 attention")) {
        h3_kernel_timing_end(g, timing);
        return 0;
    }
    // The recomputation launch: the wide kernel with a per-tile max over the
    // 32-query blocks flagged above (same retry bytes, 256 queries per workgroup).
    hipLaunchKernelGGL((attn_bf16_wide<2, false, false, false, 8>), dim3(groups), dim3(512), 2 * 2 * STAGE_BYTES,
                       g->compute, a);
    h3_kernel_timing_end(g, timing);
    return h3_launch_status(g, "BF16 attention");
}


// Ping-pong: waves w and w + 4 of a workgroup share a SIMD, so the two wave
// groups (0-3 and 4-7) run opposite phases of the key sweep. Each barrier
// interval is a half-step: one group computes the scores of a KT x 64-key
// group (MFMA only) while the other runs the softmax and P.V of the previous
// group (VALU exponentials under the other group's MFMAs). K and V^T have
// separate two-slot rings: K(t) is read in half-steps 2t (group 0) and 2t+1
// (group 1), V^T(t) in 2t+1 and 2t+2, and each is loaded two half-steps
// ahead. Running max, overflow handling, retry bytes and output as the NOMAX
// wide kernel (one retry byte per wave, 256 queries per workgroup).
template <int KT>
__global__ __attribute__((amdgpu_flat_work_group_size(512, 512), amdgpu_waves_per_eu(2, 2)))
void attn_bf16_pingpong(Args a) {
    constexpr int WAVES = 8;
    constexpr int BM = 256;
    constexpr int KSLOT = KT * K_BYTES, VSLOT = KT * V_BYTES;
    constexpr int LOADS = (K_BYTES / 1024) / WAVES;
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];

    // wave and head are read as uniform values so that LDS destinations and
    // buffer offsets stay scalar (no waterfall loops around the loads).
    const unsigned tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / 64), lane = tid % 64;
    const unsigned n = lane % 32, hf = lane / 32;
    const int grp = (int)__builtin_amdgcn_readfirstlane(wave / 4);
    const unsigned qrows = a.qrows ? a.qrows : a.seq;
    const unsigned nqb = (qrows + BM - 1) / BM;
    const unsigned id = xcd_remap(blockIdx.x, gridDim.x);
    const unsigned head = __builtin_amdgcn_readfirstlane(id / nqb), qb = __builtin_amdgcn_readfirstlane(id % nqb);
    const unsigned q0 = qb * BM;
    uint8_t *const retry = a.retry + ((size_t)head * nqb + qb) * 8;
    const size_t stride = (size_t)a.heads * D;
    const uint16_t *qh = a.q + (size_t)head * D;
    const uint16_t *kh = a.k + (size_t)head * D;
    const uint16_t *vth = a.vt + (size_t)head * D * a.padded;
    const float c = a.scale_log2;
    const unsigned count = (a.seq + BN - 1) / BN;
    const unsigned groups = (count + KT - 1) / KT;

    bf16x8 qf[8];
    {
        unsigned row = q0 + wave * 32 + n;
        row = row < qrows ? row : qrows - 1;
        const uint16_t *p = qh + (size_t)row * stride + hf * 8;
        bool bad = false;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            qf[ks] = *reinterpret_cast<const bf16x8 *>(p + ks * 16);
            bad |= bf16_vec_nonfinite(qf[ks]);
        }
        if (bad) a.fault[0] = 1u;
    }
    uint32_t koff, voff;
    {
        const unsigned key = 4 * wave + lane / 16, d = 8 * wave + lane / 8;
        koff = (key * (uint32_t)stride + k_chunk(key, lane % 16) * 8) * 2;
        voff = (d * a.padded + v_chunk(d, lane % 8) * 8) * 2;
    }
    // Group g's K tiles into K slot g % 2, V^T tiles into V slot g % 2, with
    // buffer loads straight to LDS: a uniform byte offset per load plus one
    // per-lane offset (koff / voff). In the last tile, lanes whose key is at
    // or past seq take BUFFER_OOB and load zeros (their scores are masked);
    // tile ids past the end are clamped (such loads refill a slot no step
    // reads).
    const __amdgpu_buffer_rsrc_t krsrc =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.k, (short)0, (int)((size_t)a.seq * stride * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t vrsrc =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.vt, (short)0, (int)((size_t)a.heads * D * a.padded * 2), 0x00020000);
    auto load_k = [&](unsigned g) {
        uint8_t *base = smem + (g & 1) * KSLOT;
#pragma unroll
        for (int j = 0; j < KT; j++) {
            const unsigned key0 = min(g * KT + j, count - 1) * BN;
            const bool tail = key0 + BN > a.seq;
#pragma unroll
            for (int t = 0; t < LOADS; t++) {
                const unsigned so = (unsigned)(((size_t)head * D + ((size_t)key0 + 4 * WAVES * t) * stride) * 2);
                auto *dst = (__attribute__((address_space(3))) void *)(base + j * K_BYTES + (wave + WAVES * t) * 1024);
                if (tail) {
                    const unsigned key = key0 + 4 * WAVES * t + 4 * wave + lane / 16;
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(krsrc, dst, 16, key < a.seq ? koff : BUFFER_OOB, so, 0, 0);
                } else {
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(krsrc, dst, 16, koff, so, 0, 0);
                }
            }
        }
    };
    auto load_v = [&](unsigned g) {
        uint8_t *base = smem + 2 * KSLOT + (g & 1) * VSLOT;
#pragma unroll
        for (int j = 0; j < KT; j++) {
            const unsigned key0 = min(g * KT + j, count - 1) * BN;
#pragma unroll
            for (int t = 0; t < LOADS; t++) {
                const unsigned so = (unsigned)(((size_t)head * D * a.padded + (size_t)8 * WAVES * t * a.padded + key0) * 2);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    vrsrc, (__attribute__((address_space(3))) void *)(base + j * V_BYTES + (wave + WAVES * t) * 1024), 16,
                    voff, so, 0, 0);
            }
        }
    };

    f32x16 o[4];
#pragma unroll
    for (int md = 0; md < 4; md++) o[md] = f32x16{};
    float m = -1e30f, l = 0.f;
    bool failed = false;
    f32x16 s[KT][2];

    load_k(0);
    load_v(0);
    wait_vm_loads();
    __syncthreads();
    const int halves = 2 * (int)groups;
    for (int h = 0; h <= halves; h++) {
        if ((h & 1) == 0) load_k((unsigned)h / 2 + 1);
        else load_v((unsigned)h / 2 + 1);
        const int hh = h - grp;
        if (hh >= 0 && hh < halves) {
            const unsigned t = (unsigned)hh / 2;
            if ((hh & 1) == 0) {
                // Scores of group t (MFMA only).
                const uint8_t *base = smem + (t & 1) * KSLOT;
                // Fragment addresses are recomputed per half-step (one VALU
                // op each) rather than kept live across the loop.
                unsigned nr = n;
                asm volatile("" : "+v"(nr));
#pragma unroll
                for (int j = 0; j < KT; j++) {
                    const uint8_t *ks = base + j * K_BYTES;
                    bf16x8 kfr[16];
#pragma unroll
                    for (int x = 0; x < 16; x++) {
                        const unsigned key = (x % 2) * 32 + nr;
                        kfr[x] = *reinterpret_cast<const bf16x8 *>(ks + key * 256 + k_chunk(key, (x / 2) * 2 + hf) * 16);
                    }
                    s[j][0] = f32x16{};
                    s[j][1] = f32x16{};
#pragma unroll
                    for (int kstep = 0; kstep < 8; kstep++)
#pragma unroll
                        for (int mb = 0; mb < 2; mb++)
                            s[j][mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kfr[kstep * 2 + mb], qf[kstep], s[j][mb], 0, 0, 0);
                }
#pragma unroll
                for (int j = 0; j < KT; j++) {
                    const unsigned tile = t * KT + j;
                    if (tile >= count || tile * BN + BN > a.seq) {
#pragma unroll
                        for (int mb = 0; mb < 2; mb++)
#pragma unroll
                            for (int r = 0; r < 16; r++) {
                                unsigned key = tile * BN + mb * 32 + (r / 4) * 8 + hf * 4 + (r % 4);
                                if (tile >= count || key >= a.seq) s[j][mb][r] = -INFINITY;
                            }
                    }
                }
                if (t == 0) {
                    float mx = -INFINITY;
#pragma unroll
                    for (int j = 0; j < KT; j++)
#pragma unroll
                        for (int mb = 0; mb < 2; mb++)
#pragma unroll
                            for (int r = 0; r < 16; r++) mx = fmaxf(mx, s[j][mb][r]);
                    m = fmaxf(m, half_max_swap(mx) * c);
                }
            } else {
                // Softmax and P.V of group t.
                const uint8_t *base = smem + 2 * KSLOT + (t & 1) * VSLOT;
                const float neg = -m;
                int raise = 0;
                unsigned nr = n;
                asm volatile("" : "+v"(nr));
#pragma unroll
                for (int j = 0; j < KT; j++) {
                    const uint8_t *vs = base + j * V_BYTES;
                    bf16x8 pb[4];
                    float psum = 0.f;
#pragma unroll
                    for (int mb = 0; mb < 2; mb++)
#pragma unroll
                        for (int r = 0; r < 16; r += 2) {
                            float p0 = exp2f_fast(fmaf(s[j][mb][r], c, neg));
                            float p1 = exp2f_fast(fmaf(s[j][mb][r + 1], c, neg));
                            psum += p0 + p1;
                            pb[mb * 2 + r / 8][r % 8] = (__bf16)p0;
                            pb[mb * 2 + r / 8][r % 8 + 1] = (__bf16)p1;
                        }
                    if (!(psum <= PSUM_LIMIT)) raise = max(raise, (int)((__builtin_bit_cast(uint32_t, psum) >> 23) & 0xFF) - 127);
                    l += psum;
                    // V^T fragments in two halves of eight (32 VGPRs live).
#pragma unroll
                    for (int half = 0; half < 2; half++) {
                        bf16x8 vfr[8];
#pragma unroll
                        for (int y = 0; y < 8; y++) {
                            const int x = half * 8 + y;
                            const unsigned d = (x % 4) * 32 + nr;
                            vfr[y] = *reinterpret_cast<const bf16x8 *>(vs + d * 128 + v_chunk(d, (x / 4) * 2 + hf) * 16);
                        }
#pragma unroll
                        for (int k2 = 0; k2 < 2; k2++)
#pragma unroll
                            for (int md = 0; md < 4; md++)
                                o[md] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vfr[k2 * 4 + md], pb[half * 2 + k2], o[md], 0, 0, 0);
                    }
                }
                if (__builtin_amdgcn_ballot_w64(raise != 0)) {
                    raise = (int)half_max_swap((float)raise);
                    failed |= raise >= RETRY_EXP;
                    if (raise >= RETRY_EXP) raise = 0;
                    const float alpha = ldexpf(1.f, -raise);
                    m += (float)raise;
                    l *= alpha;
#pragma unroll
                    for (int md = 0; md < 4; md++) o[md] *= alpha;
                }
            }
        }
        // The loads of the previous half-step have landed; this half-step's
        // (needed two half-steps on) stay in flight.
        __builtin_amdgcn_s_waitcnt(0x0F70 | (KT * LOADS));
        __syncthreads();
    }
    wait_vm_loads();

    const float total = half_sum_swap(l);
    const float inv = total > 0.f ? 1.f / total : 0.f;
    const unsigned q = q0 + wave * 32 + n;
    bool bad = false;
    if (q < qrows) {
        uint16_t *dst = a.out + (a.head_major ? ((size_t)head * a.seq + q) * D : ((size_t)q * a.heads + head) * D);
#pragma unroll
        for (int md = 0; md < 4; md++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                u16x4 w;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    float x = o[md][g4 * 4 + i] * inv;
                    bad |= !finite_f32(x);
                    w[i] = f32_to_bf16(x);
                }
                *reinterpret_cast<u16x4 *>(dst + md * 32 + g4 * 8 + hf * 4) = w;
            }
    }
    const bool any = __builtin_amdgcn_ballot_w64(failed || bad) != 0;
    if (lane == 0) retry[wave] = any ? 1 : 0;
    if (!any && a.lse && hf == 0 && q < qrows) a.lse[(size_t)head * qrows + q] = (m + log2f(total)) * 0.6931471805599453f;
}

template <int KT>
int launch_pingpong(h3_gpu *g, const Args &a, unsigned groups) {
    constexpr size_t shared = 2 * KT * STAGE_BYTES;
    static bool configured = false;
    if (!configured) {
        if (!h3_hip_check(g, hipFuncSetAttribute((const void *)attn_bf16_pingpong<KT>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)shared),
                          "attention shared memory"))
            return 0;
        configured = true;
    }
    if (!configure_wide<2, false, false, false>(g)) return 0;
    hipEvent_t timing = h3_kernel_timing_begin(g);
    hipLaunchKernelGGL(attn_bf16_pingpong<KT>, dim3(groups), dim3(512), shared, g->compute, a);
    if (!h3_launch_status(g, "BF16 attention")) return 0;
    hipLaunchKernelGGL((attn_bf16_wide<2, false, false, false>), dim3(groups), dim3(512), 2 * 2 * STAGE_BYTES,
                       g->compute, a);
    h3_kernel_timing_end(g, timing);
    return h3_launch_status(g, "BF16 attention");
}

// Listed sparse attention: one workgroup of QW waves per (32 * QW-query block,
// head) walks that block's own list of kept 64-key tiles (ascending tile ids,
// a list per head and query block): SubBlock routes (QW 2) and SOL exact tiles
// (QW 1 or 2).
//  * CENT (SOL): after the exact tiles, centroid tiles: tile t holds the
//    centroids of key blocks 64t .. 64t+63 (K centroids in K's row layout, V
//    centroids transposed like V^T); only the approximate blocks of the query
//    block (a 64-bit mask per tile and half) take part, each with the bias
//    ln 64 (6 in the kernel's log2 units), in the same online softmax. SOL
//    entries carry a bit per 32-query half (HALF_BIT << wave): a wave skips
//    the entries its half's query block does not route.
//  * SPLIT: 32 KB of LDS hold one K tile and one V^T tile; the phases are
//    offset so that the next K tile loads during this tile's softmax and P.V,
//    and the next V^T tile during the next scores. Barriers: one after the
//    scores (K free, V^T ready), one after P.V (V^T free, next K ready).
//  * otherwise two full stages (64 KB): the next tile loads during this one.
// The list lengths and tile ids are read as wave-uniform values one iteration
// ahead: a vector load used at once would make the compiler wait for every
// outstanding load, the tile loads included. Fragments are read from LDS as
// they are consumed (requesting all 16 ahead, as the dense kernel does, costs
// 42 more VGPRs and spills here). Row sums of P are VALU adds.
constexpr uint32_t CENT_BIT = 0x80000000u, HALF_BIT = 1u << 29, TILE_BITS = HALF_BIT - 1;

template <bool SPLIT, int OCC, int QW, bool CENT>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * QW, 64 * QW), amdgpu_waves_per_eu(OCC, OCC)))
void attn_bf16_listed(Args a) {
    constexpr int BLOCKS = K_BYTES / 1024;
    constexpr unsigned QROWS = 32 * QW;
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    // wave is read as a wave-uniform value so that per-wave loops and LDS
    // addresses stay scalar.
    const unsigned tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid / 64), lane = tid % 64;
    const unsigned n = lane % 32, hf = lane / 32;
    const unsigned nqb = a.qslab ? a.qslab : (a.seq + QROWS - 1) / QROWS;
    const unsigned id = xcd_remap(blockIdx.x, gridDim.x);
    const unsigned head = __builtin_amdgcn_readfirstlane(id / nqb), qb = __builtin_amdgcn_readfirstlane(id % nqb);
    const unsigned q0 = (a.qb0 + qb) * QROWS;
    const size_t stride = (size_t)a.heads * D;
    const uint16_t *qh = a.q + (size_t)head * D;
    const uint16_t *kh = a.k + (size_t)head * D;
    const uint16_t *vth = a.vt + (size_t)head * D * a.padded;
    const uint16_t *kch = CENT ? a.kc + (size_t)head * D : nullptr;
    const uint16_t *vcth = CENT ? a.vct + (size_t)head * D * a.kc_padded : nullptr;
    const float c = a.scale_log2;
    const size_t lq = (size_t)head * nqb + qb;
    const unsigned count = __builtin_amdgcn_readfirstlane(a.kv_count[lq]);
    const unsigned ccount = CENT ? __builtin_amdgcn_readfirstlane(a.cent_count[lq]) : 0u;
    const unsigned total = count + ccount;
    const uint32_t *list = a.kv_list + lq * a.list_stride;
    const uint32_t *clist = CENT ? a.cent_list + lq * a.cent_stride : nullptr;
    const uint64_t *cmask = CENT ? a.cent_mask + lq * a.cent_stride * 2 : nullptr;
    const uint32_t half_bit = HALF_BIT << wave;     // SOL: this wave's query block routes the entry

    bf16x8 qf[8];
    {
        unsigned row = min(q0 + wave * 32 + n, a.seq - 1);
        const uint16_t *p = qh + (size_t)row * stride + hf * 8;
        bool bad = false;
#pragma unroll
        for (int k8 = 0; k8 < 8; k8++) {
            qf[k8] = *reinterpret_cast<const bf16x8 *>(p + k8 * 16);
            bad |= bf16_vec_nonfinite(qf[k8]);
        }
        if (bad) a.fault[0] = 1u;
    }
    f32x16 o[4];
#pragma unroll
    for (int md = 0; md < 4; md++) o[md] = f32x16{};
    float m = -1e30f, l = 0.f;

    // Byte offsets, inside a full tile, of this lane's 16-byte load t (LDS
    // block wave + QW t): a full exact tile is then a uniform base plus these,
    // with no per-load address arithmetic.
    constexpr int LOADS = BLOCKS / QW;
    uint32_t koff[LOADS], voff[LOADS];
#pragma unroll
    for (int t = 0; t < LOADS; t++) {
        const unsigned b = wave + QW * t;
        const unsigned key = 4 * b + lane / 16, d = 8 * b + lane / 8;
        koff[t] = (key * (uint32_t)stride + k_chunk(key, lane % 16) * 8) * 2;
        voff[t] = (d * a.padded + v_chunk(d, lane % 8) * 8) * 2;
    }

    // Entry i of the walk: an exact tile id, or a centroid tile (CENT_BIT | t).
    auto entry_at = [&](unsigned i) -> uint32_t {
        if (!CENT || i < count) return list[i];
        return clist[i - count] | CENT_BIT;
    };
    // Buffered exact tiles: a uniform byte offset per load plus one of four
    // (K) or two (V) lane offsets (load t's swizzle repeats with t mod 4 / 2).
    const __amdgpu_buffer_rsrc_t krsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)a.k, (short)0, (int)(uint32_t)((size_t)a.seq * stride * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t vrsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)a.vt, (short)0, (int)(uint32_t)((size_t)a.heads * D * a.padded * 2), 0x00020000);
    uint32_t kl[4], vl[2];
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const unsigned key = 4 * wave + 4 * QW * t + lane / 16;
        kl[t] = ((4 * wave + lane / 16) * (uint32_t)stride + k_chunk(key, lane % 16) * 8) * 2;
    }
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const unsigned d = 8 * wave + 8 * QW * t + lane / 8;
        vl[t] = ((8 * wave + lane / 8) * a.padded + v_chunk(d, lane % 8) * 8) * 2;
    }
    // FULL (key tiles only, every key < seq): no tail or centroid code, and
    // with a load mode fixed by the caller (BUF: buffer loads, else global
    // loads), only that mode's code.
    auto load_k = [&](uint32_t e, uint8_t *ks, auto full_tag, auto buf_tag) {
        constexpr bool FULL = decltype(full_tag)::value, BUF = decltype(buf_tag)::value;
        const bool cent = !FULL && CENT && (e & CENT_BIT);
        const unsigned key0 = (CENT ? e & TILE_BITS : e) * BN, limit = cent ? a.key_blocks : a.seq;
        const uint16_t *base = cent ? kch : kh;
        if ((FULL ? BUF : a.buffered) && !cent && (FULL || key0 + BN <= limit)) {
#pragma unroll
            for (int t = 0; t < LOADS; t++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    krsrc, (__attribute__((address_space(3))) void *)(ks + (wave + QW * t) * 1024), 16, kl[t % 4],
                    (unsigned)(((size_t)head * D + ((size_t)key0 + 4 * QW * t) * stride) * 2), 0, 0);
            return;
        }
        if (FULL || (!cent && key0 + BN <= limit)) {
            const __attribute__((address_space(1))) char *tile =
                (const __attribute__((address_space(1))) char *)(base + (size_t)key0 * stride);
#pragma unroll
            for (int t = 0; t < LOADS; t++)
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(tile + koff[t]),
                                                 (__attribute__((address_space(3))) void *)(ks + (wave + QW * t) * 1024),
                                                 16, 0, 0);
            return;
        }
#pragma unroll
        for (unsigned b = wave; b < BLOCKS; b += QW) {
            unsigned key = 4 * b + lane / 16, phys = lane % 16;
            unsigned row = min(key0 + key, limit - 1);
            const uint16_t *src = base + (size_t)row * stride + k_chunk(key, phys) * 8;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                             (__attribute__((address_space(3))) void *)(ks + b * 1024), 16, 0, 0);
        }
    };
    auto load_v = [&](uint32_t e, uint8_t *vs, auto full_tag, auto buf_tag) {
        constexpr bool FULL = decltype(full_tag)::value, BUF = decltype(buf_tag)::value;
        const bool cent = !FULL && CENT && (e & CENT_BIT);
        const unsigned padded = cent ? a.kc_padded : a.padded;
        const unsigned col = min((CENT ? e & TILE_BITS : e) * BN, padded - BN);
        const uint16_t *base = cent ? vcth : vth;
        if ((FULL ? BUF : a.buffered) && !cent) {
#pragma unroll
            for (int t = 0; t < LOADS; t++)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    vrsrc, (__attribute__((address_space(3))) void *)(vs + (wave + QW * t) * 1024), 16, vl[t % 2],
                    (unsigned)(((size_t)head * D * a.padded + (size_t)8 * QW * t * a.padded + col) * 2), 0, 0);
            return;
        }
        if (!cent) {                               // exact tiles: col + BN <= padded always
            const __attribute__((address_space(1))) char *tile =
                (const __attribute__((address_space(1))) char *)(base + col);
#pragma unroll
            for (int t = 0; t < LOADS; t++)
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(tile + voff[t]),
                                                 (__attribute__((address_space(3))) void *)(vs + (wave + QW * t) * 1024),
                                                 16, 0, 0);
            return;
        }
#pragma unroll
        for (unsigned b = wave; b < BLOCKS; b += QW) {
            unsigned d = 8 * b + lane / 8, vph = lane % 8;
            const uint16_t *src = base + (size_t)d * padded + col + v_chunk(d, vph) * 8;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                             (__attribute__((address_space(3))) void *)(vs + b * 1024), 16, 0, 0);
        }
    };
    // Scores S^T = K Q^T for a tile's 64 keys.
    auto scores = [&](const uint8_t *ks, f32x16 (&s)[2]) {
        s[0] = f32x16{}; s[1] = f32x16{};
#pragma unroll
        for (int kstep = 0; kstep < 8; kstep++)
#pragma unroll
            for (int mb = 0; mb < 2; mb++) {
                const unsigned key = mb * 32 + n;
                const bf16x8 kf = *reinterpret_cast<const bf16x8 *>(ks + key * 256 + k_chunk(key, kstep * 2 + hf) * 16);
                s[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kstep], s[mb], 0, 0, 0);
            }
    };
    // Online softmax of the tile and O^T += V^T P^T. bits: for a centroid
    // tile, bit mb * 16 + r says whether the key of accumulator element
    // s[mb][r] takes part; the bias is added in log2 units.
    auto softmax_pv = [&](f32x16 (&s)[2], const uint8_t *vs, uint32_t e, uint32_t bits, auto full_tag) {
        constexpr bool FULL = decltype(full_tag)::value;
        const bool cent = !FULL && CENT && (e & CENT_BIT);
        const unsigned tile = CENT ? e & TILE_BITS : e;
        const float bias = cent ? 6.0f : 0.0f;      // log2(64)
        // A centroid tile is masked in the P domain below (its max may then
        // include excluded centroids: an upper bound, harmless to the softmax);
        // a key tile crossing the sequence end masks keys >= seq here.
        if (!FULL && !cent && tile * BN + BN > a.seq) {
#pragma unroll
            for (int mb = 0; mb < 2; mb++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    unsigned key = tile * BN + mb * 32 + (r / 4) * 8 + hf * 4 + (r % 4);
                    if (key >= a.seq) s[mb][r] = -INFINITY;
                }
        }
        float mx0 = fmaxf(s[0][0], s[0][1]), mx1 = fmaxf(s[1][0], s[1][1]);
#pragma unroll
        for (int r = 2; r < 16; r += 2) {
            mx0 = fmaxf(fmaxf(mx0, s[0][r]), s[0][r + 1]);
            mx1 = fmaxf(fmaxf(mx1, s[1][r]), s[1][r + 1]);
        }
        const float mx = fmaf(half_max_swap(fmaxf(mx0, mx1)), c, bias);
        if (__builtin_amdgcn_ballot_w64(mx > m + RESCALE_SLACK)) {
            const float mnew = fmaxf(m, mx);
            const float alpha = exp2f_fast(m - mnew);
            m = mnew;
            l *= alpha;
#pragma unroll
            for (int md = 0; md < 4; md++) o[md] *= alpha;
        }
        const float neg = bias - m;
        bf16x8 pb[4];
        float psum = 0.f;
#pragma unroll
        for (int mb = 0; mb < 2; mb++)
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                float p0 = exp2f_fast(fmaf(s[mb][r], c, neg));
                float p1 = exp2f_fast(fmaf(s[mb][r + 1], c, neg));
                if (cent) {
                    p0 = (bits >> (mb * 16 + r)) & 1u ? p0 : 0.f;
                    p1 = (bits >> (mb * 16 + r + 1)) & 1u ? p1 : 0.f;
                }
                psum += p0 + p1;
                pb[mb * 2 + r / 8][r % 8] = (__bf16)p0;
                pb[mb * 2 + r / 8][r % 8 + 1] = (__bf16)p1;
            }
        l += psum;
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
#pragma unroll
            for (int md = 0; md < 4; md++) {
                const unsigned d = md * 32 + n;
                const bf16x8 vf = *reinterpret_cast<const bf16x8 *>(vs + d * 128 + v_chunk(d, kk * 2 + hf) * 16);
                o[md] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pb[kk], o[md], 0, 0, 0);
            }
    };
    // The approximate-block mask of entry i for this wave's half (centroid
    // entries only), read with the ids, one entry ahead; wave-uniform.
    auto mask_at = [&](unsigned i) -> uint64_t {
        if (!CENT || i >= total || i < count) return 0ull;
        return cmask[2 * (i - count) + wave];
    };
    auto uniform64 = [](uint64_t w) -> uint64_t {
        // readfirstlane returns int: widen through uint32_t, or the low word
        // sign-extends over the high one.
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(w >> 32));
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)w);
        return ((uint64_t)hi << 32) | lo;
    };
    // This lane's 32 bits of a mask: keys mb * 32 + g * 8 + hf * 4 + (0..3)
    // -> bits mb * 16 + g * 4 + (0..3), the accumulator element order.
    auto lane_bits = [&](uint64_t w) -> uint32_t {
        uint32_t bits = 0;
#pragma unroll
        for (int mb = 0; mb < 2; mb++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                bits |= (uint32_t)((w >> (mb * 32 + g * 8 + hf * 4)) & 0xfu) << (mb * 16 + g * 4);
        return bits;
    };

    uint32_t tile = 0, next = 0;
    uint64_t mask = 0;
    if (total) tile = __builtin_amdgcn_readfirstlane(entry_at(0));
    if (total > 1) next = __builtin_amdgcn_readfirstlane(entry_at(1));
    if (CENT) mask = uniform64(mask_at(0));
    if constexpr (SPLIT) {
        uint8_t *ks = smem, *vs = smem + K_BYTES;
        if (total) { load_k(tile, ks, std::false_type{}, std::false_type{}); load_v(tile, vs, std::false_type{}, std::false_type{}); }
        wait_vm_loads();
        __syncthreads();
        auto step = [&](unsigned it, auto full_tag, auto buf_tag) {
            constexpr bool FULL = decltype(full_tag)::value;   // this and the next entry: full exact tiles
            const bool has_next = it + 1 < total;
            f32x16 s[2];
            if (!CENT || (tile & half_bit)) scores(ks, s);
            wait_vm_loads();               // this tile's V^T (own share)
            __syncthreads();               // K free; every share of V^T landed
            if (has_next) load_k(next, ks, full_tag, buf_tag);
            const uint32_t later = it + 2 < total ? entry_at(it + 2) : 0u;
            const uint64_t mask_after = FULL ? 0ull : mask_at(it + 1);
            if (!CENT || (tile & half_bit)) softmax_pv(s, vs, tile, CENT && !FULL ? lane_bits(mask) : 0u, full_tag);
            wait_vm_loads();               // next K, the id after it and the next mask (own share)
            __syncthreads();               // V^T free; every share of the next K landed
            if (has_next) load_v(next, vs, full_tag, buf_tag);
            tile = next;
            next = __builtin_amdgcn_readfirstlane(later);
            if (CENT && !FULL) mask = uniform64(mask_after);
        };
        // Exact tiles come first and ascending, so only the last exact entry
        // can cross the sequence end (centroid entries follow), and a step
        // loads the entry after its own. Steps whose own and next entries are
        // exact and not the last exact one run in a loop of their own with no
        // tail or centroid code (a compact loop).
        unsigned it0 = 0;
        const unsigned exact = CENT ? count : total;
        if (a.buffered)
            for (; it0 + 2 < exact; it0++) step(it0, std::true_type{}, std::true_type{});
        else
            for (; it0 + 2 < exact; it0++) step(it0, std::true_type{}, std::false_type{});
        for (unsigned it = it0; it < total; it++) step(it, std::false_type{}, std::false_type{});
    } else {
        if (total) {
            load_k(tile, smem, std::false_type{}, std::false_type{});
            load_v(tile, smem + K_BYTES, std::false_type{}, std::false_type{});
        }
        wait_vm_loads();
        __syncthreads();
        for (unsigned it = 0; it < total; it++) {
            const int cur = it & 1;
            uint8_t *ks = smem + cur * STAGE_BYTES;
            if (it + 1 < total) {
                uint8_t *nk = smem + (cur ^ 1) * STAGE_BYTES;
                load_k(next, nk, std::false_type{}, std::false_type{});
                load_v(next, nk + K_BYTES, std::false_type{}, std::false_type{});
            }
            const uint32_t later = it + 2 < total ? entry_at(it + 2) : 0u;
            const uint64_t mask_after = mask_at(it + 1);
            if (!CENT || (tile & half_bit)) {
                f32x16 s[2];
                scores(ks, s);
                softmax_pv(s, ks + K_BYTES, tile, CENT ? lane_bits(mask) : 0u, std::false_type{});
            }
            wait_vm_loads();
            __syncthreads();
            tile = next;
            next = __builtin_amdgcn_readfirstlane(later);
            if (CENT) mask = uniform64(mask_after);
        }
    }

    const float sum = half_sum_swap(l);
    const float inv = sum > 0.f ? 1.f / sum : 0.f;
    const unsigned q = q0 + wave * 32 + n;
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
                    float x = o[md][g4 * 4 + i] * inv;
                    bad |= !finite_f32(x);
                    w[i] = f32_to_bf16(x);
                }
                *reinterpret_cast<u16x4 *>(dst + md * 32 + g4 * 8 + hf * 4) = w;
            }
    }
    if (bad) a.fault[0] = 1u;
}

template <bool SPLIT, int OCC, int QW, bool CENT>
int launch_listed(h3_gpu *g, const Args &a, unsigned groups) {
    constexpr size_t shared = SPLIT ? STAGE_BYTES : 2 * STAGE_BYTES;
    static bool configured = false;
    auto kernel = attn_bf16_listed<SPLIT, OCC, QW, CENT>;
    if (!configured) {
        if (!h3_hip_check(g, hipFuncSetAttribute((const void *)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shared),
                          "attention shared memory"))
            return 0;
        configured = true;
    }
    hipEvent_t timing = h3_kernel_timing_begin(g);
    hipLaunchKernelGGL(kernel, dim3(groups), dim3(64 * QW), shared, g->compute, a);
    h3_kernel_timing_end(g, timing);
    return h3_launch_status(g, CENT ? "SOL attention" : "routed BF16 attention");
}

}  // namespace

// V^T, then (256-byte aligned) one retry byte per (head, 256-query block, wave).
static size_t retry_offset(uint32_t seq, uint32_t heads) {
    return ((size_t)heads * D * ((seq + 63) / 64 * 64) * sizeof(uint16_t) + 255) / 256 * 256;
}

size_t h3_attention_bf16_workspace(uint32_t seq, uint32_t heads) {
    return retry_offset(seq, heads) + (size_t)heads * ((seq + 255) / 256) * 8;
}

int h3_launch_attention_bf16(h3_gpu *g, void *workspace, uint16_t *out, const uint16_t *q, const uint16_t *k,
                             const uint16_t *v, uint32_t seq, uint32_t heads, float scale, bool head_major,
                             const uint32_t *kv_list, const uint32_t *kv_count, uint32_t list_stride) {
    Args a{};
    a.out = out; a.q = q; a.k = k; a.vt = (const uint16_t *)workspace;
    a.seq = seq; a.heads = heads; a.padded = (seq + 63) / 64 * 64;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.head_major = head_major ? 1 : 0;
    a.kv_list = kv_list; a.kv_count = kv_count; a.list_stride = list_stride;
    a.fault = g->fault;
    // Variant 13: the global-load path that tensors of 4 GiB and more take.
    a.buffered = fits_buffer(a) && g->attention_variant != 13;
    hipLaunchKernelGGL(transpose_v, dim3(a.padded / BN, heads), dim3(256), 0, g->compute, v, k, (uint16_t *)workspace,
                       seq, heads, a.padded, g->fault);
    if (!h3_launch_status(g, "V transpose")) return 0;
    // Sparse lists are per 128-query block: 4 waves per workgroup, two
    // workgroups per CU. Dense: 8 waves x 32 queries, two waves per SIMD, 128
    // keys per barrier interval (measured fastest of the shapes kept here).
    if (kv_list) return launch<4, 1, 2, true, true>(g, a, (seq + 127) / 128 * heads);
    if (g->attention_variant == 1) return launch<8, 1, 2, false, true>(g, a, (seq + 255) / 256 * heads);
    if (g->attention_variant == 2) return launch<12, 1, 3, false, false>(g, a, (seq + 383) / 384 * heads);
    // Variant 3: a tile max every 128 keys instead of the row-sum test.
    if (g->attention_variant == 3) return launch_wide<2, false, false, false>(g, a, (seq + 255) / 256 * heads);
    a.retry = (uint8_t *)workspace + retry_offset(seq, heads);
    // Variant 4: four waves (128 queries) per workgroup and two workgroups per
    // CU, whose barriers are independent, 64 keys per interval (6% slower).
    if (g->attention_variant == 4) return launch_wide<1, false, false, true, 4>(g, a, (seq + 127) / 128 * heads);
    // Variant 9: ping-pong wave groups (21.7 ms against 18.3 at S = 32400, H = 40).
    if (g->attention_variant == 9 && a.buffered) return launch_pingpong<1>(g, a, (seq + 255) / 256 * heads);
    // The hand-scheduled kernel needs at least three 128-key groups; variant
    // 14 keeps the wide kernel.
    if (a.buffered && seq > 256 && g->attention_variant != 14) return launch_pipe_attention(g, a);
    return launch_wide<2, false, false, true>(g, a, (seq + 255) / 256 * heads);
}

// Dense attention of query rows [first, first + qrows) (q and out already
// offset to the first row) over all seq keys, with the FP32 log-sum-exp per
// (head, query row) written to lse [heads, qrows]: the fast kernel and its
// recomputation launch, whatever the variant selector says.
int h3_launch_attention_flash(h3_gpu *g, void *workspace, uint16_t *out, const uint16_t *q, const uint16_t *k,
                              const uint16_t *v, float *lse, uint32_t seq, uint32_t qrows, uint32_t heads,
                              float scale, bool head_major) {
    Args a{};
    a.out = out; a.q = q; a.k = k; a.vt = (const uint16_t *)workspace;
    a.seq = seq; a.qrows = qrows; a.heads = heads; a.padded = (seq + 63) / 64 * 64;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.head_major = head_major ? 1 : 0;
    a.lse = lse;
    a.fault = g->fault;
    a.buffered = fits_buffer(a);
    hipLaunchKernelGGL(transpose_v, dim3(a.padded / BN, heads), dim3(256), 0, g->compute, v, k, (uint16_t *)workspace,
                       seq, heads, a.padded, g->fault);
    if (!h3_launch_status(g, "V transpose")) return 0;
    a.retry = (uint8_t *)workspace + retry_offset(seq, heads);
    return launch_wide<2, false, false, true>(g, a, (qrows + 255) / 256 * heads);
}

int h3_launch_attention_routed(h3_gpu *g, void *workspace, uint16_t *out, const uint16_t *q, const uint16_t *k,
                               const uint16_t *v, uint32_t seq, uint32_t heads, float scale, bool head_major,
                               const uint32_t *lists, const uint32_t *counts, uint32_t list_stride,
                               uint32_t head0, uint32_t group, uint32_t qb0, uint32_t qslab, bool transpose) {
    // One head group [head0, head0 + group) and query-block slab: pointers
    // move to the group's first head (strides stay those of all heads), the
    // transposed V holds the group's heads only, and lists are slab-relative.
    Args a{};
    a.out = out + (head_major ? (size_t)head0 * seq * D : (size_t)head0 * D);
    a.q = q + (size_t)head0 * D; a.k = k + (size_t)head0 * D; a.vt = (const uint16_t *)workspace;
    a.seq = seq; a.heads = heads; a.padded = (seq + 63) / 64 * 64;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.head_major = head_major ? 1 : 0;
    a.kv_list = lists; a.kv_count = counts; a.list_stride = list_stride;
    a.qb0 = qb0; a.qslab = qslab;
    a.fault = g->fault;
    // Global loads: with buffer loads the split-phase kernel spills SGPRs and
    // ran 7% slower (7.20 against 6.69 ms at S = 32400, H = 40, 25% density).
    a.buffered = 0;
    if (transpose) {
        hipLaunchKernelGGL(transpose_v, dim3(a.padded / BN, group), dim3(256), 0, g->compute, v + (size_t)head0 * D,
                           a.k, (uint16_t *)workspace, seq, heads, a.padded, g->fault);
        if (!h3_launch_status(g, "V transpose")) return 0;
    }
    const unsigned groups = qslab * group;
    // Split K/V phases, two waves per SIMD (measured fastest); variant 12:
    // two full 64 KB stages at one wave per SIMD.
    if (g->attention_variant == 12) return launch_listed<false, 1, 2, false>(g, a, groups);
    return launch_listed<true, 2, 2, false>(g, a, groups);
}

int h3_launch_attention_sol(h3_gpu *g, void *workspace, uint16_t *out, const uint16_t *q, const uint16_t *k,
                            const uint16_t *v, uint32_t seq, uint32_t heads, float scale, bool head_major,
                            uint32_t q_block, const h3_sol_lists *lists, uint32_t head0, uint32_t group) {
    // Heads [head0, head0 + group): Q, K, output and the centroid arrays move
    // to the group's first head (strides stay those of all heads); the lists
    // and the transposed V hold the group's heads only.
    Args a{};
    a.out = out + (head_major ? (size_t)head0 * seq * D : (size_t)head0 * D);
    a.q = q + (size_t)head0 * D; a.k = k + (size_t)head0 * D; a.vt = (const uint16_t *)workspace;
    a.seq = seq; a.heads = heads; a.padded = (seq + 63) / 64 * 64;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.head_major = head_major ? 1 : 0;
    a.kv_list = lists->exact; a.kv_count = lists->exact_count; a.list_stride = lists->exact_stride;
    a.cent_list = lists->cent; a.cent_count = lists->cent_count; a.cent_mask = lists->cent_mask;
    a.cent_stride = lists->cent_stride; a.key_blocks = lists->key_blocks; a.kc_padded = lists->kc_padded;
    a.kc = lists->kc + (size_t)head0 * D; a.vct = lists->vct + (size_t)head0 * D * lists->kc_padded;
    a.fault = g->fault;
    a.buffered = fits_buffer(a) && g->attention_variant != 13;
    hipLaunchKernelGGL(transpose_v, dim3(a.padded / BN, group), dim3(256), 0, g->compute, v + (size_t)head0 * D, a.k,
                       (uint16_t *)workspace, seq, heads, a.padded, g->fault);
    if (!h3_launch_status(g, "V transpose")) return 0;
    (void)q_block;   // 32-row blocks come paired in the lists: one 64-query workgroup either way
    return launch_listed<true, 2, 2, true>(g, a, (seq + 63) / 64 * group);
}
