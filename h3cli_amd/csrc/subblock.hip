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

// One thread per (cell, head, 8 channels): fp32 tree sum over the cell's 16
// rows (missing rows are zero), mean * scale, rounded to BF16. 16-byte loads;
// a workgroup covers 16 cells of one head.
__global__ __launch_bounds__(256) void sb_pool(const uint16_t *q, const uint16_t *k, uint16_t *qpool,
                                               uint16_t *kpool, unsigned seq, unsigned heads, unsigned cells,
                                               float qscale, unsigned *fault) {
    const unsigned cell = blockIdx.x * 16 + threadIdx.x / 16, part = threadIdx.x % 16, head = blockIdx.y;
    const bool is_k = blockIdx.z != 0;
    const uint16_t *src = is_k ? k : q;
    uint16_t *dst = (is_k ? kpool : qpool) + ((size_t)head * cells + cell) * D + part * 8;
    const float scale = is_k ? 1.f : qscale;
    const unsigned start = cell * 16, count = start < seq ? min(16u, seq - start) : 0u;
    u16x8 raw[16];
#pragma unroll
    for (unsigned i = 0; i < 16; i++)
        raw[i] = i < count ? *reinterpret_cast<const u16x8 *>(src + ((size_t)(start + i) * heads + head) * D + part * 8)
                           : u16x8{};
    u16x8 result;
    bool bad = false;
#pragma unroll
    for (int c = 0; c < 8; c++) {
        float v[16];
#pragma unroll
        for (unsigned i = 0; i < 16; i++) v[i] = bf16_to_f32(raw[i][c]);
#pragma unroll
        for (unsigned s = 8; s; s >>= 1)
#pragma unroll
            for (unsigned i = 0; i < s; i++) v[i] += v[i + s];
        const float mean = count ? __fdiv_rn(v[0], (float)count) * scale : 0.f;
        result[c] = f32_to_bf16(mean);
        bad |= !finite_f32(mean) || !finite_f32(bf16_to_f32(result[c]));
    }
    if (bad) fault[0] = 1u;
    *reinterpret_cast<u16x8 *>(dst) = result;
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
// query-cell one spans four adjacent lanes. The grid covers the query blocks
// [qb0, qb0 + qslab) (qb0 a multiple of 32, so the cell tiles stay inside the
// padded pool); scores are written slab-relative, [head][qslab][blocks].
__global__ __launch_bounds__(256) void sb_score(const uint16_t *qpool, const uint16_t *kpool, float *scores,
                                                unsigned seq, unsigned cells, unsigned blocks, unsigned qb0,
                                                unsigned qslab, unsigned *fault) {
    const unsigned wave = threadIdx.x / 64, lane = threadIdx.x % 64, n = lane % 32, hf = lane / 32;
    const unsigned head = blockIdx.z;
    const unsigned qt = blockIdx.x * (CELL_TILE / 32) + wave;          // 32-cell query tile in the slab
    const unsigned valid = (seq + 15) / 16;                            // cells holding rows
    const unsigned qcell = qb0 * 4 + qt * 32 + n, qblock = qcell / 4, a = qcell % 4;
    const unsigned qend = min(blocks, qb0 + qslab);
    if (qt * 8 >= qslab) return;
    const uint16_t *qh = qpool + (size_t)head * cells * D;
    const uint16_t *kh = kpool + (size_t)head * cells * D;
    bf16x8 qf[8];
#pragma unroll
    for (int ks = 0; ks < 8; ks++) qf[ks] = *reinterpret_cast<const bf16x8 *>(qh + (size_t)qcell * D + ks * 16 + hf * 8);
    const bool q_valid = qcell < valid;
    const unsigned ktiles = cells / 32;
    const unsigned kt0 = blockIdx.y * KEY_SPLIT, kt1 = min(ktiles, kt0 + KEY_SPLIT);
    bool bad = false;
    const unsigned kend = min(kt1, (blocks + 7) / 8);
    bf16x8 kf[8];
    auto load_k = [&](unsigned kt) {
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
            kf[ks] = *reinterpret_cast<const bf16x8 *>(kh + (size_t)(kt * 32 + n) * D + ks * 16 + hf * 8);
    };
    if (kt0 < kend) load_k(kt0);
    for (unsigned kt = kt0; kt < kend; kt++) {
        f32x16 s = f32x16{};
#pragma unroll
        for (int ks = 0; ks < 8; ks++) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks], qf[ks], s, 0, 0, 0);
        if (kt + 1 < kend) load_k(kt + 1);     // next tile's fragments load during the reductions
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
                if (b < nk) sum += __builtin_amdgcn_exp2f(s[4 * g + b] - largest);
            float lse = (q_valid && nk) ? largest + __builtin_amdgcn_logf(sum) : -INFINITY;
            // Query-cell log-sum-exp over the block's four lanes.
            const float top = quad_max(lse);
            const float total = quad_sum(q_valid && nk ? __builtin_amdgcn_exp2f(lse - top) : 0.f);
            if (a == 0 && qblock < qend && kblock < blocks) {
                const float score = (top + __builtin_amdgcn_logf(total)) * 0.6931471805599453f;
                bad |= !finite_f32(score);
                scores[((size_t)head * qslab + (qblock - qb0)) * blocks + kblock] = score;
            }
        }
    }
    if (bad) fault[0] = 1u;
}

// Order-preserving key of a score: larger float, larger key; -0 and +0 map to
// the same key, so keys tie exactly when the scores compare equal.
__device__ inline uint32_t score_key(float f) {
    uint32_t u = __float_as_uint(f == 0.f ? 0.f : f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// One workgroup per (query block of the slab [qb0, qb0 + qslab), head); rows
// of scores, routes, lists and counts are slab-relative. Route rule and counters of the
// reference's selection (cuda_subblock.cu:300-324): with
// rank(k) = #{j : s_j > s_k} + #{j < k : s_j == s_k}, key block k is kept
// when rank < keep, when it is protected, when the query block is protected
// or with force_all. rank(k) is k's position when the row is sorted by
// descending score and ascending index, so a bitonic sort of
// (key << 32 | ~index) in LDS gives every rank at once (P = next power of two
// of B; padding sorts last). The kept blocks are then compacted in ascending
// order into the row's tile list; counts[row] is its length and
// added_blocks[row] the protected key blocks kept beyond the top.
__global__ __launch_bounds__(256) void sb_select(const float *scores, uint8_t *routes, const uint8_t *q_protect,
                                                 const uint8_t *k_protect, unsigned blocks, unsigned padded,
                                                 unsigned keep, int force_all, unsigned qb0, unsigned qslab,
                                                 uint32_t *lists, uint32_t *counts, uint32_t *added_blocks) {
    extern __shared__ unsigned long long sortbuf[];   // [padded], then top flags [blocks]
    uint8_t *top_flag = reinterpret_cast<uint8_t *>(sortbuf + padded);
    __shared__ unsigned wave_total[4];
    __shared__ unsigned red[4];
    const unsigned tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const unsigned qb = qb0 + blockIdx.x, head = blockIdx.y;
    const size_t row = (size_t)head * qslab + blockIdx.x;
    const float *src = scores + row * blocks;
    for (unsigned i = tid; i < padded; i += 256)
        sortbuf[i] = i < blocks ? ((unsigned long long)score_key(src[i]) << 32) | (0xffffffffu - i) : 0ull;
    __syncthreads();
    // Descending bitonic sort.
    for (unsigned size = 2; size <= padded; size <<= 1)
        for (unsigned step = size >> 1; step; step >>= 1) {
            for (unsigned t = tid; t < padded / 2; t += 256) {
                const unsigned i = 2 * step * (t / step) + (t % step), j = i + step;
                const unsigned long long x = sortbuf[i], y = sortbuf[j];
                const bool descending = (i & size) == 0;
                if (descending ? x < y : x > y) { sortbuf[i] = y; sortbuf[j] = x; }
            }
            __syncthreads();
        }
    for (unsigned i = tid; i < blocks; i += 256) top_flag[i] = 0;
    __syncthreads();
    for (unsigned p = tid; p < keep; p += 256) top_flag[0xffffffffu - (uint32_t)sortbuf[p]] = 1;
    __syncthreads();

    const bool pq = q_protect[qb] != 0;
    uint32_t *list = lists + row * blocks;
    uint8_t *route_row = routes + row * blocks;
    unsigned offset = 0;
    unsigned added = 0;
    for (unsigned base = 0; base < blocks; base += 256) {
        const unsigned k = base + tid;
        bool retain = false;
        if (k < blocks) {
            const bool top = top_flag[k] != 0;
            const bool protect = k_protect[k] != 0;
            retain = force_all || pq || top || protect;
            route_row[k] = (uint8_t)retain;
            added += protect && !top && !pq && !force_all;
        }
        const unsigned long long mask = __ballot(retain);
        const unsigned before = __popcll(mask & ((1ull << lane) - 1ull));
        if (lane == 0) wave_total[wave] = __popcll(mask);
        __syncthreads();
        unsigned pos = offset + before;
        for (unsigned w = 0; w < wave; w++) pos += wave_total[w];
        if (retain) list[pos] = k;
        offset += wave_total[0] + wave_total[1] + wave_total[2] + wave_total[3];
        __syncthreads();
    }
    for (int off = 32; off; off >>= 1) added += __shfl_xor(added, off, 64);
    if (lane == 0) red[wave] = added;
    __syncthreads();
    if (tid == 0) {
        counts[row] = offset;
        added_blocks[row] = red[0] + red[1] + red[2] + red[3];
    }
}

// One workgroup: folds a call's per-row list lengths and added protected
// blocks into the running counters ([0] kept, [1] protected key blocks added
// beyond the top).
__global__ __launch_bounds__(1024) void sb_count(const uint32_t *counts, const uint32_t *added, size_t rows,
                                                 unsigned long long *counters) {
    __shared__ unsigned long long red[16][2];
    unsigned long long k = 0, a = 0;
    for (size_t i = threadIdx.x; i < rows; i += 1024) { k += counts[i]; a += added[i]; }
    for (int off = 32; off; off >>= 1) { k += __shfl_xor(k, off, 64); a += __shfl_xor(a, off, 64); }
    if (threadIdx.x % 64 == 0) { red[threadIdx.x / 64][0] = k; red[threadIdx.x / 64][1] = a; }
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long kept = 0, extra = 0;
        for (int w = 0; w < 16; w++) { kept += red[w][0]; extra += red[w][1]; }
        counters[0] += kept;
        counters[1] += extra;
    }
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

int h3_subblock_bind(h3_gpu *g, h3_subblock_router *r, const h3_sol_layout *layout) {
    if (!layout || !layout->query || !layout->key || !layout->sequence)
        return h3_set_error(g, "SubBlock: missing layout");
    if (r->bound) return h3_set_error(g, "SubBlock: layout is already configured");
    const uint32_t seq = layout->sequence, blocks = (seq + 63) / 64;
    // Selection sorts a row of 8-byte keys in LDS: at most 8192 blocks.
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

namespace {
// Byte layout of one chunk's router workspace; offsets into r when r is set.
size_t router_layout(uint32_t blocks, uint32_t cells, uint32_t group, uint32_t qslab, h3_subblock_router *r) {
    size_t off = 0, o[7];
    o[0] = off; off = align256(off + (size_t)group * cells * D * 2);           // Q pool
    o[1] = off; off = align256(off + (size_t)group * cells * D * 2);           // K pool
    o[2] = off; off = align256(off + (size_t)group * qslab * blocks * 4);      // scores
    o[3] = off; off = align256(off + (size_t)group * qslab * blocks);          // routes
    o[4] = off; off = align256(off + (size_t)group * qslab * blocks * 4);      // lists
    o[5] = off; off = align256(off + (size_t)group * qslab * 4);               // counts
    o[6] = off; off = align256(off + (size_t)group * qslab * 4);               // protected added
    if (r) {
        r->off_qpool = o[0]; r->off_kpool = o[1]; r->off_scores = o[2]; r->off_routes = o[3];
        r->off_list = o[4]; r->off_count = o[5]; r->off_added = o[6];
    }
    return off;
}
uint32_t cells_of(uint32_t blocks) { return (blocks * 4 + CELL_TILE - 1) / CELL_TILE * CELL_TILE; }
}  // namespace

int h3_subblock_plan(h3_gpu *g, const h3_subblock_router *r, uint32_t seq, uint32_t heads, h3_subblock_chunking *out) {
    if (!r->bound) return h3_set_error(g, "SubBlock attention needs a bound layout (h3_gpu_dit_sol_layout)");
    if (seq != r->seq) return h3_set_error(g, "SubBlock layout was bound for sequence %u, not %u", r->seq, seq);
    const uint32_t blocks = (seq + 63) / 64, cells = cells_of(blocks);
    for (uint32_t group = heads;; group = std::max(1u, group / 2)) {
        const uint32_t g_eff = std::min(group, heads);
        uint32_t slab = blocks;
        for (;;) {
            const size_t router = router_layout(blocks, cells, g_eff, slab, nullptr);
            const size_t vt = h3_attention_bf16_workspace(seq, g_eff);
            if (router + vt <= r->cap) {
                out->group = g_eff; out->slab = slab;
                out->router_bytes = router; out->vt_bytes = vt; out->bytes = router + vt;
                return 1;
            }
            // Next slab: the largest multiple of 32 below the current one, halving.
            uint32_t next = slab == blocks ? (blocks - 1) / 32 * 32 : slab / 2 / 32 * 32;
            if (next < 32 || next >= slab) break;
            slab = next;
        }
        if (group == 1) break;
    }
    return h3_set_error(g, "SubBlock: S=%u H=%u workspace plan exceeds its fixed budget of %zu bytes", seq, heads,
                        r->cap);
}

int h3_subblock_route(h3_gpu *g, h3_subblock_router *r, const uint16_t *q, const uint16_t *k, uint32_t seq,
                      uint32_t heads, uint32_t head0, uint32_t group, uint32_t qb0, uint32_t qslab, float scale,
                      unsigned keep, bool force_all, bool pool) {
    if (!r->bound) return h3_set_error(g, "SubBlock attention needs a bound layout (h3_gpu_dit_sol_layout)");
    if (seq != r->seq) return h3_set_error(g, "SubBlock layout was bound for sequence %u, not %u", r->seq, seq);
    if (!keep || keep > r->blocks) return h3_set_error(g, "SubBlock: invalid budget %u of %u blocks", keep, r->blocks);
    const uint32_t blocks = r->blocks;
    if (!group || head0 + group > heads || qb0 % 32 || !qslab || qb0 + qslab > blocks)
        return h3_set_error(g, "SubBlock: invalid chunk (heads %u+%u of %u, blocks %u+%u of %u)", head0, group, heads,
                            qb0, qslab, blocks);
    // Cells padded to whole score workgroups (128 cells); pad cells pool to 0.
    const uint32_t cells = cells_of(blocks);
    const size_t bytes = router_layout(blocks, cells, group, qslab, r);
    if (!pool && (r->group != group || r->head0 != head0 || r->ws.bytes < bytes))
        return h3_set_error(g, "SubBlock: chunk without pooled cells of its head group");
    if (!h3_buffer_reserve(g, &r->ws, bytes, "SubBlock workspace")) return 0;
    if (!r->counters.ptr) {
        if (!h3_buffer_reserve(g, &r->counters, 4 * 8, "SubBlock counters") ||
            !h3_hip_check(g, hipMemsetAsync(r->counters.ptr, 0, 4 * 8, g->compute), "SubBlock counters"))
            return 0;
    }
    auto *base = (uint8_t *)r->ws.ptr;
    auto *counters = (unsigned long long *)r->counters.ptr;
    r->heads = heads; r->cells = cells; r->group = group; r->head0 = head0; r->qb0 = qb0; r->qslab = qslab;
    auto *qpool = (uint16_t *)(base + r->off_qpool), *kpool = (uint16_t *)(base + r->off_kpool);
    auto *scores = (float *)(base + r->off_scores);
    const auto *meta = (const uint8_t *)r->meta.ptr;

    if (pool) {
        hipLaunchKernelGGL(sb_pool, dim3(cells / 16, group, 2), dim3(256), 0, g->compute, q + (size_t)head0 * D,
                           k + (size_t)head0 * D, qpool, kpool, seq, heads, cells, scale * 1.4426950408889634f,
                           g->fault);
        if (!h3_launch_status(g, "SubBlock pool")) return 0;
    }
    const unsigned ktiles = cells / 32;
    hipLaunchKernelGGL(sb_score, dim3((qslab * 4 + CELL_TILE - 1) / CELL_TILE, (ktiles + KEY_SPLIT - 1) / KEY_SPLIT, group),
                       dim3(256), 0, g->compute, qpool, kpool, scores, seq, cells, blocks, qb0, qslab, g->fault);
    if (!h3_launch_status(g, "SubBlock score")) return 0;
    unsigned padded = 1;
    while (padded < blocks) padded <<= 1;
    const size_t shared = (size_t)padded * 8 + blocks;
    static bool configured = false;
    if (!configured) {
        if (!h3_hip_check(g, hipFuncSetAttribute((const void *)sb_select, hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)(8192 * 8 + 8192)), "SubBlock select shared memory"))
            return 0;
        configured = true;
    }
    hipLaunchKernelGGL(sb_select, dim3(qslab, group), dim3(256), shared, g->compute, scores, base + r->off_routes,
                       meta, meta + blocks, blocks, padded, keep, force_all ? 1 : 0, qb0, qslab,
                       (uint32_t *)(base + r->off_list), (uint32_t *)(base + r->off_count),
                       (uint32_t *)(base + r->off_added));
    if (!h3_launch_status(g, "SubBlock select")) return 0;
    hipLaunchKernelGGL(sb_count, dim3(1), dim3(1024), 0, g->compute, (const uint32_t *)(base + r->off_count),
                       (const uint32_t *)(base + r->off_added), (size_t)group * qslab, counters);
    if (!h3_launch_status(g, "SubBlock counters")) return 0;
    r->possible += (uint64_t)group * qslab * blocks;
    r->counters_pending = true;
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
    void *counters = r->counters.ptr;
    if (hipMemcpy(c, counters, sizeof(c), hipMemcpyDeviceToHost) != hipSuccess) return;
    if (hipMemset(counters, 0, sizeof(c)) != hipSuccess) return;
    g->stats.subblock_selected += c[0];
    g->stats.subblock_possible += r->possible;
    r->possible = 0;
    r->counters_pending = false;
}

void h3_subblock_free(h3_subblock_router *r) {
    h3_buffer_free(&r->ws);
    h3_buffer_free(&r->counters);
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
    if (r->chunked) return h3_set_error(g, "SubBlock routes: the last call ran in chunks; only whole calls are kept");
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
