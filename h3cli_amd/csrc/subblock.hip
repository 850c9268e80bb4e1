// SubBlock router kernels. The algorithm is the reference's
// (src/cuda/cuda_subblock.cu:256-324): per head, 16-row cells of Q and K are
// averaged (Q pre-scaled by scale * log2 e) and rounded to BF16; each pair of
// 64-row blocks is scored by a log-sum-exp over key cells, then over query
// cells (log2 domain, times ln 2); each query block keeps the `keep`
// highest-scoring key blocks (ties to the lower index) plus protected key
// blocks, and a protected query block keeps everything.
//
// MI355X layout: the cell dot products of one head form a [cells x cells]
// matrix product, so scoring runs on the matrix cores (32 x 32 cell tiles,
// fp32 accumulation of exact BF16 products) and the two log-sum-exps fold in
// registers. Selection writes the route bytes and, in the same pass, the
// ordered list of kept 64-key tiles per (head, 128-query block) with one route
// bit per 64-query half, which is what the sparse attention kernel walks.
#include "subblock.h"
#include "../../include/h3_policy.h"
#include <algorithm>
#include <cmath>

namespace {

constexpr unsigned D = 128;
constexpr unsigned CELL_TILE = 128;        // query cells per score workgroup (4 waves x 32)
constexpr unsigned KEY_SPLIT = 16;         // 32-cell key tiles per score workgroup

// One thread per (cell, head, channel pair): fp32 tree sum over the cell's 16
// rows (missing rows are zero), mean * scale, rounded to BF16.
__global__ __launch_bounds__(256) void sb_pool(const uint16_t *q, const uint16_t *k, uint16_t *qpool,
                                               uint16_t *kpool, unsigned seq, unsigned heads, unsigned cells,
                                               float qscale, unsigned *fault) {
    const unsigned cell = blockIdx.x * 4 + threadIdx.x / 64, pair = threadIdx.x % 64, head = blockIdx.y;
    const bool is_k = blockIdx.z != 0;
    const uint16_t *src = is_k ? k : q;
    uint16_t *dst = (is_k ? kpool : qpool) + ((size_t)head * cells + cell) * D + pair * 2;
    const float scale = is_k ? 1.f : qscale;
    const unsigned start = cell * 16, count = start < seq ? min(16u, seq - start) : 0u;
    float a[16], b[16];
#pragma unroll
    for (unsigned i = 0; i < 16; i++) {
        uint32_t w = 0;
        if (i < count) w = *reinterpret_cast<const uint32_t *>(src + ((size_t)(start + i) * heads + head) * D + pair * 2);
        a[i] = bf16_to_f32((uint16_t)(w & 0xffffu));
        b[i] = bf16_to_f32((uint16_t)(w >> 16));
    }
#pragma unroll
    for (unsigned s = 8; s; s >>= 1)
#pragma unroll
        for (unsigned i = 0; i < s; i++) { a[i] += a[i + s]; b[i] += b[i + s]; }
    float ma = 0.f, mb = 0.f;
    if (count) {
        ma = __fdiv_rn(a[0], (float)count) * scale;
        mb = __fdiv_rn(b[0], (float)count) * scale;
    }
    const uint16_t ra = f32_to_bf16(ma), rb = f32_to_bf16(mb);
    if (!finite_f32(ma) || !finite_f32(mb) || !finite_f32(bf16_to_f32(ra)) || !finite_f32(bf16_to_f32(rb)))
        fault[0] = 1u;
    *reinterpret_cast<uint32_t *>(dst) = (uint32_t)ra | ((uint32_t)rb << 16);
}

__device__ inline float quad_max(float x) {
    x = fmaxf(x, __shfl_xor(x, 1, 64));
    return fmaxf(x, __shfl_xor(x, 2, 64));
}
__device__ inline float quad_sum(float x) {
    x += __shfl_xor(x, 1, 64);
    return x + __shfl_xor(x, 2, 64);
}

// Scores for 32 query cells (8 query blocks) per wave against KEY_SPLIT tiles
// of 32 key cells (8 key blocks each). S^T = Kpool . Qpool^T on the matrix
// core: lane n holds query cell n and, for g = 0..3, the four cells of key
// block 2g + (lane / 32), so the key-cell log-sum-exp is lane-local and the
// query-cell one spans four adjacent lanes.
__global__ __launch_bounds__(256) void sb_score(const uint16_t *qpool, const uint16_t *kpool, float *scores,
                                                unsigned seq, unsigned cells, unsigned blocks, unsigned *fault) {
    const unsigned wave = threadIdx.x / 64, lane = threadIdx.x % 64, n = lane % 32, hf = lane / 32;
    const unsigned head = blockIdx.z;
    const unsigned qt = blockIdx.x * (CELL_TILE / 32) + wave;          // 32-cell query tile
    const unsigned valid = (seq + 15) / 16;                            // cells holding rows
    const unsigned qcell = qt * 32 + n, qblock = qcell / 4, a = qcell % 4;
    if (qt * 8 >= blocks) return;
    const uint16_t *qh = qpool + (size_t)head * cells * D;
    const uint16_t *kh = kpool + (size_t)head * cells * D;
    bf16x8 qf[8];
#pragma unroll
    for (int ks = 0; ks < 8; ks++) qf[ks] = *reinterpret_cast<const bf16x8 *>(qh + (size_t)qcell * D + ks * 16 + hf * 8);
    const bool q_valid = qcell < valid;
    const unsigned ktiles = cells / 32;
    const unsigned kt0 = blockIdx.y * KEY_SPLIT, kt1 = min(ktiles, kt0 + KEY_SPLIT);
    bool bad = false;
    for (unsigned kt = kt0; kt < kt1 && kt * 8 < blocks; kt++) {
        f32x16 s = f32x16{};
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            bf16x8 kf = *reinterpret_cast<const bf16x8 *>(kh + (size_t)(kt * 32 + n) * D + ks * 16 + hf * 8);
            s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], s, 0, 0, 0);
        }
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const unsigned kblock = kt * 8 + 2 * g + hf;
            const unsigned kc0 = kblock * 4;
            const unsigned nk = kc0 < valid ? min(4u, valid - kc0) : 0u;
            // Key-cell log-sum-exp (log2 units) of this query cell.
            float largest = s[4 * g];
#pragma unroll
            for (unsigned b = 1; b < 4; b++)
                if (b < nk) largest = fmaxf(largest, s[4 * g + b]);
            float sum = 0.f;
#pragma unroll
            for (unsigned b = 0; b < 4; b++)
                if (b < nk) sum += exp2f(s[4 * g + b] - largest);
            float lse = (q_valid && nk) ? largest + log2f(sum) : -INFINITY;
            // Query-cell log-sum-exp over the block's four lanes.
            const float top = quad_max(lse);
            const float total = quad_sum(q_valid && nk ? exp2f(lse - top) : 0.f);
            if (a == 0 && qblock < blocks && kblock < blocks) {
                const float score = (top + log2f(total)) * 0.6931471805599453f;
                bad |= !finite_f32(score);
                scores[((size_t)head * blocks + qblock) * blocks + kblock] = score;
            }
        }
    }
    if (bad) fault[0] = 1u;
}

// One workgroup per (128-query block p, head): query blocks 2p and 2p + 1.
// Route rule and counters of the reference's selection
// (cuda_subblock.cu:300-324): rank = #{j : s_j > s_k or (s_j == s_k and j < k)},
// kept when rank < keep, the key block is protected, the query block is
// protected or force_all is set. counters: [0] kept, [1] possible,
// [2] protected query blocks, [3] protected key blocks added beyond the top.
__global__ __launch_bounds__(256) void sb_select(const float *scores, uint8_t *routes, const uint8_t *q_protect,
                                                 const uint8_t *k_protect, unsigned blocks, unsigned keep,
                                                 int force_all, uint32_t *lists, uint32_t *counts, unsigned nqb,
                                                 unsigned long long *counters) {
    extern __shared__ float row[];         // [2][blocks]
    __shared__ unsigned wave_total[4];
    __shared__ unsigned long long red[4][4];
    const unsigned tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const unsigned p = blockIdx.x, head = blockIdx.y;
    const unsigned qa = 2 * p, rows = min(2u, blocks - qa);
    const float *src = scores + ((size_t)head * blocks + qa) * blocks;
    for (unsigned i = tid; i < rows * blocks; i += 256) row[i] = src[i];
    __syncthreads();
    bool pq[2];
    for (unsigned r = 0; r < 2; r++) pq[r] = r < rows && q_protect[qa + r];
    uint32_t *list = lists + ((size_t)head * nqb + p) * blocks;
    unsigned offset = 0;
    unsigned long long kept = 0, added = 0;
    for (unsigned base = 0; base < blocks; base += 256) {
        const unsigned k = base + tid;
        unsigned route[2] = {0, 0};
        if (k < blocks) {
            const bool protect = k_protect[k] != 0;
            for (unsigned r = 0; r < rows; r++) {
                const float *sr = row + r * blocks;
                const float score = sr[k];
                unsigned rank = 0;
                for (unsigned j = 0; j < blocks; j++) {
                    const float x = sr[j];
                    rank += (x > score) | ((x == score) & (j < k));
                }
                const bool top = rank < keep;
                const bool retain = force_all || pq[r] || top || protect;
                route[r] = retain;
                routes[((size_t)head * blocks + qa + r) * blocks + k] = (uint8_t)retain;
                kept += retain;
                added += protect && !top && !pq[r] && !force_all;
            }
        }
        // Ordered compaction of the tiles either half routes.
        const bool any = route[0] | route[1];
        const unsigned long long mask = __ballot(any);
        const unsigned before = __popcll(mask & ((1ull << lane) - 1ull));
        if (lane == 0) wave_total[wave] = __popcll(mask);
        __syncthreads();
        unsigned wave_base = offset;
        for (unsigned w = 0; w < wave; w++) wave_base += wave_total[w];
        if (any) list[wave_base + before] = k | (route[0] << 30) | (route[1] << 31);
        offset += wave_total[0] + wave_total[1] + wave_total[2] + wave_total[3];
        __syncthreads();
    }
    // Workgroup totals of the counters.
    for (int off = 32; off; off >>= 1) {
        kept += __shfl_xor(kept, off, 64);
        added += __shfl_xor(added, off, 64);
    }
    if (lane == 0) { red[wave][0] = kept; red[wave][1] = added; }
    __syncthreads();
    if (tid == 0) {
        unsigned long long k_sum = red[0][0] + red[1][0] + red[2][0] + red[3][0];
        unsigned long long a_sum = red[0][1] + red[1][1] + red[2][1] + red[3][1];
        counts[(size_t)head * nqb + p] = offset;
        atomicAdd(counters + 0, k_sum);
        atomicAdd(counters + 1, (unsigned long long)rows * blocks);
        atomicAdd(counters + 2, (unsigned long long)(pq[0] + pq[1]));
        atomicAdd(counters + 3, a_sum);
    }
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

int h3_subblock_bind(h3_gpu *g, h3_subblock_router *r, const h3_sol_layout *layout) {
    if (!layout || !layout->query || !layout->key || !layout->sequence)
        return h3_set_error(g, "SubBlock: missing layout");
    if (r->bound) return h3_set_error(g, "SubBlock: layout is already configured");
    const uint32_t seq = layout->sequence, blocks = (seq + 63) / 64;
    // Selection holds two score rows in 64 KB of LDS: at most 8192 blocks.
    if (blocks > 8192) return h3_set_error(g, "SubBlock: sequence %u exceeds the router's limit", seq);
    if (layout->query_blocks != blocks || layout->key_blocks != blocks)
        return h3_set_error(g, "SubBlock: layout geometry differs from Q64/K64");
    for (uint32_t b = 0; b < blocks; b++)
        if (layout->query[b].rows != std::min(64u, seq - b * 64) || layout->key[b].rows != layout->query[b].rows)
            return h3_set_error(g, "SubBlock: invalid true block lengths");
    r->q_protect.assign(blocks, 0); r->k_protect.assign(blocks, 0);
    r->protected_ranges = 0;
    for (uint32_t b = 0; b < blocks; b++) {
        r->q_protect[b] = layout->query[b].protect != 0;
        r->k_protect[b] = layout->key[b].protect != 0;
        if (r->q_protect[b] && (b == 0 || !r->q_protect[b - 1])) r->protected_ranges++;
    }
    if (!h3_buffer_reserve(g, &r->meta, 2 * (size_t)blocks, "SubBlock layout") ||
        !h3_hip_check(g, hipMemcpy(r->meta.ptr, r->q_protect.data(), blocks, hipMemcpyHostToDevice), "SubBlock layout") ||
        !h3_hip_check(g, hipMemcpy((uint8_t *)r->meta.ptr + blocks, r->k_protect.data(), blocks, hipMemcpyHostToDevice),
                      "SubBlock layout"))
        return 0;
    r->seq = seq; r->blocks = blocks; r->bound = true;
    return 1;
}

int h3_subblock_route(h3_gpu *g, h3_subblock_router *r, const uint16_t *q, const uint16_t *k, uint32_t seq,
                      uint32_t heads, float scale, unsigned keep, bool force_all) {
    if (!r->bound) return h3_set_error(g, "SubBlock attention needs a bound layout (h3_gpu_dit_sol_layout)");
    if (seq != r->seq) return h3_set_error(g, "SubBlock layout was bound for sequence %u, not %u", r->seq, seq);
    if (!keep || keep > r->blocks) return h3_set_error(g, "SubBlock: invalid budget %u of %u blocks", keep, r->blocks);
    const uint32_t blocks = r->blocks;
    // Cells padded to whole score workgroups (128 cells); pad cells pool to 0.
    const uint32_t cells = (blocks * 4 + CELL_TILE - 1) / CELL_TILE * CELL_TILE;
    const uint32_t nqb = (seq + 127) / 128;
    size_t off = 0;
    r->off_qpool = off; off = align256(off + (size_t)heads * cells * D * 2);
    r->off_kpool = off; off = align256(off + (size_t)heads * cells * D * 2);
    r->off_scores = off; off = align256(off + (size_t)heads * blocks * blocks * 4);
    r->off_routes = off; off = align256(off + (size_t)heads * blocks * blocks);
    r->off_list = off; off = align256(off + (size_t)heads * nqb * blocks * 4);
    r->off_count = off; off = align256(off + (size_t)heads * nqb * 4);
    r->off_counters = off; off = align256(off + 4 * 8);
    const bool fresh = r->ws.bytes < off;
    if (!h3_buffer_reserve(g, &r->ws, off, "SubBlock workspace")) return 0;
    auto *base = (uint8_t *)r->ws.ptr;
    auto *counters = (unsigned long long *)(base + r->off_counters);
    if (fresh && !h3_hip_check(g, hipMemsetAsync(counters, 0, 4 * 8, g->compute), "SubBlock counters")) return 0;
    r->heads = heads; r->cells = cells; r->nqb = nqb;
    auto *qpool = (uint16_t *)(base + r->off_qpool), *kpool = (uint16_t *)(base + r->off_kpool);
    auto *scores = (float *)(base + r->off_scores);
    const auto *meta = (const uint8_t *)r->meta.ptr;

    hipLaunchKernelGGL(sb_pool, dim3(cells / 4, heads, 2), dim3(256), 0, g->compute, q, k, qpool, kpool, seq, heads,
                       cells, scale * 1.4426950408889634f, g->fault);
    if (!h3_launch_status(g, "SubBlock pool")) return 0;
    const unsigned ktiles = cells / 32;
    hipLaunchKernelGGL(sb_score, dim3(cells / CELL_TILE, (ktiles + KEY_SPLIT - 1) / KEY_SPLIT, heads), dim3(256), 0,
                       g->compute, qpool, kpool, scores, seq, cells, blocks, g->fault);
    if (!h3_launch_status(g, "SubBlock score")) return 0;
    const size_t shared = 2 * (size_t)blocks * sizeof(float);
    if (shared > 64 * 1024) return h3_set_error(g, "SubBlock: %u blocks exceed the selection workgroup", blocks);
    static bool configured = false;
    if (!configured) {
        if (!h3_hip_check(g, hipFuncSetAttribute((const void *)sb_select, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 64 * 1024), "SubBlock select shared memory"))
            return 0;
        configured = true;
    }
    hipLaunchKernelGGL(sb_select, dim3(nqb, heads), dim3(256), shared, g->compute, scores, base + r->off_routes, meta,
                       meta + blocks, blocks, keep, force_all ? 1 : 0, (uint32_t *)(base + r->off_list),
                       (uint32_t *)(base + r->off_count), nqb, counters);
    if (!h3_launch_status(g, "SubBlock select")) return 0;
    r->counters_pending = true;
    g->stats.subblock_router_calls++;
    return 1;
}

const uint32_t *h3_subblock_lists(const h3_subblock_router *r) {
    return (const uint32_t *)((const uint8_t *)r->ws.ptr + r->off_list);
}
const uint32_t *h3_subblock_counts(const h3_subblock_router *r) {
    return (const uint32_t *)((const uint8_t *)r->ws.ptr + r->off_count);
}

void h3_subblock_collect(h3_gpu *g, h3_subblock_router *r) {
    if (!r->counters_pending) return;
    unsigned long long c[4] = {0, 0, 0, 0};
    void *counters = (uint8_t *)r->ws.ptr + r->off_counters;
    if (hipMemcpy(c, counters, sizeof(c), hipMemcpyDeviceToHost) != hipSuccess) return;
    if (hipMemset(counters, 0, sizeof(c)) != hipSuccess) return;
    g->stats.subblock_selected += c[0];
    g->stats.subblock_possible += c[1];
    r->counters_pending = false;
}

void h3_subblock_free(h3_subblock_router *r) {
    h3_buffer_free(&r->ws);
    h3_buffer_free(&r->meta);
    r->bound = false;
}

// Route capture for tests and audits (the reference's h3_cuda_subblock_routes,
// cuda_subblock.cu): the last call's routes [heads][blocks][blocks], scores
// (same shape) and pooled cells [heads][cells][128] (cells = 4 * blocks; the
// padding cells are not copied). Any output may be null; counts must match.
extern "C" int h3_hip_subblock_routes(h3_gpu *g, uint8_t *routes, float *scores, size_t route_count,
                                      uint16_t *q_pool, uint16_t *k_pool, size_t pool_count) {
    if (!g) return 0;
    auto *r = h3_attention_router(g);
    if (!r || !r->heads) return h3_set_error(g, "SubBlock routes: no routed call yet");
    const size_t nr = (size_t)r->heads * r->blocks * r->blocks, cells = (size_t)r->blocks * 4;
    if ((routes || scores) && route_count != nr) return h3_set_error(g, "SubBlock routes: expected %zu routes", nr);
    if ((q_pool || k_pool) && pool_count != r->heads * cells * D)
        return h3_set_error(g, "SubBlock routes: expected %zu pooled values", r->heads * cells * D);
    if (!h3_hip_check(g, hipStreamSynchronize(g->compute), "SubBlock routes")) return 0;
    const auto *base = (const uint8_t *)r->ws.ptr;
    if (routes && !h3_hip_check(g, hipMemcpy(routes, base + r->off_routes, nr, hipMemcpyDeviceToHost), "routes")) return 0;
    if (scores && !h3_hip_check(g, hipMemcpy(scores, base + r->off_scores, nr * 4, hipMemcpyDeviceToHost), "scores"))
        return 0;
    for (int which = 0; which < 2; which++) {
        uint16_t *dst = which ? k_pool : q_pool;
        if (!dst) continue;
        const auto *src = (const uint16_t *)(base + (which ? r->off_kpool : r->off_qpool));
        if (!h3_hip_check(g, hipMemcpy2D(dst, cells * D * 2, src, (size_t)r->cells * D * 2, cells * D * 2, r->heads,
                                         hipMemcpyDeviceToHost), "pooled cells"))
            return 0;
    }
    return 1;
}
