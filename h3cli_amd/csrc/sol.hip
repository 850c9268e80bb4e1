// SOL routed attention on HIP. The recipe is the reference's
// (src/cuda/cuda_sol.cu:92-310): per head, BF16 centroids of Q blocks (32 or
// 64 rows) and of K and V blocks (64 rows); per-channel mean and variance of
// the K centroids; per query block a threshold mean + tau * sigma of the
// centroid logit (log2 units); a key block is exact when it is protected,
// local in frames, on the minimum-exact floor, non-finite, a short tail block,
// or scores above the threshold, and is otherwise replaced by its centroid
// with weight 64 (bias ln 64) in the same softmax.
//
// MI355X layout: the K centroids are written in K's own row layout and the V
// centroids transposed and key-permuted exactly like the V^T workspace, so a
// "centroid tile" (64 consecutive key blocks) loads and multiplies with the
// same code as a key tile. Routing writes, per (head, query block), the
// ascending exact tile list, the list of centroid tiles that hold at least one
// approximate block, and each such tile's 64-bit approximate-block mask.
#include "sol.h"
#include <algorithm>
#include <cmath>

namespace {

constexpr unsigned D = 128;

__host__ __device__ inline unsigned vt_position(unsigned j) {   // key order of a V^T tile (attn_bf16.hip)
    unsigned k16 = j & 15;
    return (j & ~15u) + ((k16 >> 2) & 1) * 8 + (k16 >> 3) * 4 + (k16 & 3);
}

enum { SUM_Q = 0, SUM_K = 1, SUM_V = 2 };

// Centroid of block b, head h, channel d: fp32 sum of the block's rows in
// order, divided by the row count, rounded to BF16. Q -> qc [heads][qblocks][128];
// K -> kc [kblocks][heads][128]; V -> vct [heads][128][kpad] at the V^T key
// position (blocks kblocks .. kpad-1 write zeros). A workgroup covers one
// block of 16 heads: 16 lanes per head, 8 channels (one 16-byte load per row)
// per lane.
template <int WHICH>
__global__ __launch_bounds__(256) void sol_summary(const uint16_t *x, uint16_t *out, unsigned seq, unsigned heads,
                                                   unsigned block, unsigned blocks, unsigned kpad, unsigned *fault) {
    const unsigned b = blockIdx.x, h = blockIdx.y * 16 + threadIdx.x / 16, d0 = (threadIdx.x % 16) * 8;
    if (h >= heads) return;
    u16x8 value = {};
    if (b < blocks) {
        const unsigned start = b * block, len = min(block, seq - start);
        float sum[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        const uint16_t *p = x + ((size_t)start * heads + h) * D + d0;
        for (unsigned i = 0; i < len; i++) {
            const u16x8 v = *reinterpret_cast<const u16x8 *>(p + (size_t)i * heads * D);
#pragma unroll
            for (int c = 0; c < 8; c++) sum[c] = __fadd_rn(sum[c], bf16_to_f32(v[c]));
        }
        bool bad = false;
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const float mean = __fdiv_rn(sum[c], (float)len);
            value[c] = f32_to_bf16(mean);
            bad |= !finite_f32(mean) || !finite_f32(bf16_to_f32(value[c]));
        }
        if (bad) fault[0] = 1u;
    }
    if (WHICH == SUM_Q) *reinterpret_cast<u16x8 *>(out + ((size_t)h * blocks + b) * D + d0) = value;
    else if (WHICH == SUM_K) *reinterpret_cast<u16x8 *>(out + ((size_t)b * heads + h) * D + d0) = value;
    else {
#pragma unroll
        for (int c = 0; c < 8; c++) out[((size_t)h * D + d0 + c) * kpad + (b & ~63u) + vt_position(b & 63u)] = value[c];
    }
}

// Per head and channel: mean and variance of the K centroids over the key
// blocks, each product and sum rounded separately. out: [heads][256].
__global__ __launch_bounds__(128) void sol_moments(const uint16_t *kc, float *out, unsigned heads, unsigned blocks) {
    const unsigned h = blockIdx.x, d = threadIdx.x;
    float sum = 0.f, sq = 0.f;
    const uint16_t *p = kc + (size_t)h * D + d;
    const size_t stride = (size_t)heads * D;
    unsigned b = 0;
    // Sixteen loads in flight ahead of the in-order sums.
    for (; b + 16 <= blocks; b += 16) {
        float x[16];
#pragma unroll
        for (int j = 0; j < 16; j++) x[j] = bf16_to_f32(p[(size_t)(b + j) * stride]);
#pragma unroll
        for (int j = 0; j < 16; j++) {
            sum = __fadd_rn(sum, x[j]);
            sq = __fadd_rn(sq, __fmul_rn(x[j], x[j]));
        }
    }
    for (; b < blocks; b++) {
        const float x = bf16_to_f32(p[(size_t)b * stride]);
        sum = __fadd_rn(sum, x);
        sq = __fadd_rn(sq, __fmul_rn(x, x));
    }
    const float mean = __fdiv_rn(sum, (float)blocks);
    const float var = __fsub_rn(__fdiv_rn(sq, (float)blocks), __fmul_rn(mean, mean));
    out[h * 256 + d] = mean;
    out[h * 256 + 128 + d] = var > 0.f ? var : 0.f;
}

// Units: a pair of 32-row query blocks, or one 64-row block: the 64 queries a
// listed-kernel workgroup covers. One workgroup routes UPW consecutive units
// of one head. Per 256-key-block chunk each thread loads its key block's
// centroid row once into registers and scores it against every unit's query
// blocks (their centroids broadcast from LDS). For each query block, m, v and
// each dot are fmaf chains over the 128 channels in order (the oracle's order;
// see oracle_sol_route). Lists, per unit: exact tiles either block routes,
// with HALF_BIT << i set when block i routes the tile; then centroid tiles
// holding an approximate block of either, with the same half bits and one
// 64-bit approximate mask per half (for 64-row blocks both halves are the block).
constexpr uint32_t HALF_BIT = 1u << 29;
constexpr unsigned UPW = 8;

template <int PAIR>
__global__ __launch_bounds__(256) void sol_route(const uint16_t *qc, const uint16_t *kc, const float *moments,
                                                 const h3_sol_block *qmeta, const h3_sol_block *kmeta,
                                                 uint8_t *routes, uint32_t *exact_list, uint32_t *exact_count,
                                                 uint32_t *cent_list, uint32_t *cent_count, uint64_t *cent_mask,
                                                 unsigned heads, unsigned qblocks, unsigned kblocks, unsigned tiles,
                                                 unsigned units, unsigned radius, unsigned minimum, float scale,
                                                 float tau, int force_exact, uint32_t *row_counts, unsigned head0) {
    __shared__ float q[UPW][PAIR][D];
    __shared__ float limit[UPW][PAIR];
    __shared__ unsigned wave_total[1][4][2];
    __shared__ uint32_t wave_tally[4][7];
    const unsigned tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    // Head h of all heads (centroids, moments); outputs are indexed by the
    // head's place hl in the routed group [head0, head0 + gridDim.y).
    const unsigned h = head0 + blockIdx.y, hl = blockIdx.y, u0 = blockIdx.x * UPW, nu = min(UPW, units - u0);
    const float a = __fmul_rn(scale, 1.4426950408889634f);
    for (unsigned i = tid; i < UPW * PAIR * D; i += 256) {
        const unsigned u = i / (PAIR * D), qb = (u0 + u) * PAIR + (i / D) % PAIR;
        (&q[0][0][0])[i] = u < nu && qb < qblocks ? bf16_to_f32(qc[((size_t)h * qblocks + qb) * D + i % D]) : 0.f;
    }
    __syncthreads();
    if (tid < UPW * PAIR) {
        const unsigned u = tid / PAIR, pi = tid % PAIR;
        float m = 0.f, v = 0.f;
        for (unsigned d = 0; d < D; d++) {
            m = fmaf(q[u][pi][d], moments[h * 256 + d], m);
            v = fmaf(__fmul_rn(q[u][pi][d], q[u][pi][d]), moments[h * 256 + 128 + d], v);
        }
        const float mean = __fmul_rn(m, a), var = __fmul_rn(__fmul_rn(v > 0.f ? v : 0.f, a), a);
        limit[u][pi] = __fadd_rn(mean, __fmul_rn(tau, __fsqrt_rn(__fadd_rn(var, 1e-6f))));
    }
    __syncthreads();
    // Running list lengths per unit (exact, centroid).
    __shared__ unsigned lengths[UPW][2];
    if (tid < UPW * 2) (&lengths[0][0])[tid] = 0;
    // This thread's pair counts over all units: exact, approximate, protected,
    // local (not protected), floor, recovery, tail (the reference's
    // h3_cuda_sol_stats.pairs); summed per workgroup into its first unit's row.
    uint32_t tally[7] = {0, 0, 0, 0, 0, 0, 0};
    __syncthreads();
    for (unsigned base = 0; base < kblocks; base += 256) {
        const unsigned b = base + tid;
        const bool valid = b < kblocks;
        u16x8 kr[D / 8];
        h3_sol_block km = {};
        if (valid) {
            const uint16_t *row = kc + ((size_t)b * heads + h) * D;
#pragma unroll
            for (unsigned c8 = 0; c8 < D / 8; c8++) kr[c8] = *reinterpret_cast<const u16x8 *>(row + c8 * 8);
            km = kmeta[b];
        }
        const bool floor_ = valid && (uint64_t)(b + 1) * minimum / kblocks != (uint64_t)b * minimum / kblocks;
        const bool tail = valid && km.rows < 64;
#pragma unroll 1
        for (unsigned u = 0; u < nu; u++) {
            const unsigned qb0 = (u0 + u) * PAIR;
            const unsigned present = min((unsigned)PAIR, qblocks - qb0);
            bool exact[2] = {false, false};
            if (valid) {
                float dot[PAIR];
#pragma unroll
                for (int i = 0; i < PAIR; i++) dot[i] = 0.f;
#pragma unroll
                for (unsigned c8 = 0; c8 < D / 8; c8++)
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        const float kv = bf16_to_f32(kr[c8][j]);
#pragma unroll
                        for (int i = 0; i < PAIR; i++) dot[i] = fmaf(q[u][i][c8 * 8 + j], kv, dot[i]);
                    }
#pragma unroll
                for (int i = 0; i < PAIR; i++) {
                    if ((unsigned)i >= present) break;
                    const h3_sol_block qm = qmeta[qb0 + i];
                    const float di = __fmul_rn(dot[i], a), t = limit[u][i];
                    const bool protect = qm.protect || km.protect;
                    const bool local = qm.first_frame >= 0 && km.first_frame >= 0 &&
                                       qm.first_frame <= km.last_frame + (int)radius &&
                                       km.first_frame <= qm.last_frame + (int)radius;
                    const bool recovery = !finite_f32(di) || !finite_f32(t);
                    exact[i] = force_exact || protect || local || floor_ || recovery || tail || di > t;
                    routes[((size_t)hl * qblocks + qb0 + i) * kblocks + b] = (uint8_t)exact[i];
                    tally[exact[i] ? 0 : 1]++;
                    tally[2] += protect;
                    tally[3] += local && !protect;
                    tally[4] += floor_;
                    tally[5] += recovery;
                    tally[6] += tail;
                }
            }
            if (PAIR == 1) exact[1] = exact[0];
            // Ordered compaction of the tiles either block routes exactly; wave
            // w's approximate blocks are the masks of centroid tile base / 64 + w.
            const bool any = exact[0] || exact[1];
            const unsigned long long ex = __ballot(any);
            const unsigned long long m0 = __ballot(valid && !exact[0]);
            const unsigned long long m1 = PAIR == 1 ? m0 : __ballot(valid && present > 1 && !exact[1]);
            if (lane == 0) { wave_total[0][wave][0] = __popcll(ex); wave_total[0][wave][1] = (m0 | m1) != 0; }
            __syncthreads();
            const size_t row = (size_t)hl * units + u0 + u;
            unsigned pos = lengths[u][0] + __popcll(ex & ((1ull << lane) - 1ull)), cpos = lengths[u][1];
            unsigned add_exact = 0, add_cent = 0;
            for (unsigned w = 0; w < 4; w++) {
                if (w < wave) { pos += wave_total[0][w][0]; cpos += wave_total[0][w][1]; }
                add_exact += wave_total[0][w][0];
                add_cent += wave_total[0][w][1];
            }
            if (any) exact_list[row * kblocks + pos] = b | (exact[0] ? HALF_BIT : 0u) | (exact[1] ? HALF_BIT << 1 : 0u);
            if (lane == 0 && (m0 | m1)) {
                cent_list[row * tiles + cpos] = (base / 64 + wave) | (m0 ? HALF_BIT : 0u) | (m1 ? HALF_BIT << 1 : 0u);
                cent_mask[(row * tiles + cpos) * 2] = m0;
                cent_mask[(row * tiles + cpos) * 2 + 1] = m1;
            }
            __syncthreads();           // lengths[u] and wave_total read by everyone
            if (tid == 0) { lengths[u][0] += add_exact; lengths[u][1] += add_cent; }
        }
    }
    __syncthreads();
    if (tid < nu) {
        exact_count[(size_t)hl * units + u0 + tid] = lengths[tid][0];
        cent_count[(size_t)hl * units + u0 + tid] = lengths[tid][1];
    }
#pragma unroll
    for (int j = 0; j < 7; j++) {
        uint32_t x = tally[j];
        for (int off = 32; off; off >>= 1) x += __shfl_xor(x, off, 64);
        if (lane == 0) wave_tally[wave][j] = x;
    }
    __syncthreads();
    if (tid < 8) {
        const size_t row = (size_t)hl * units + u0;
        // The workgroup's counts land in its first unit's row; the others hold zeros.
        for (unsigned u = 0; u < nu; u++)
            row_counts[(row + u) * 8 + tid] =
                u == 0 && tid < 7 ? wave_tally[0][tid] + wave_tally[1][tid] + wave_tally[2][tid] + wave_tally[3][tid] : 0u;
    }
}

// Sums the per-unit pair counts of one call into the router's u64 counters
// (one workgroup: tens of thousands of same-address atomics would serialize).
__global__ __launch_bounds__(1024) void sol_count(const uint32_t *row_counts, size_t rows,
                                                  unsigned long long *counters) {
    __shared__ unsigned long long red[16][7];
    unsigned long long c[7] = {0, 0, 0, 0, 0, 0, 0};
    for (size_t r = threadIdx.x; r < rows; r += 1024)
#pragma unroll
        for (int j = 0; j < 7; j++) c[j] += row_counts[r * 8 + j];
#pragma unroll
    for (int j = 0; j < 7; j++) {
        for (int off = 32; off; off >>= 1) c[j] += __shfl_xor(c[j], off, 64);
        if (threadIdx.x % 64 == 0) red[threadIdx.x / 64][j] = c[j];
    }
    __syncthreads();
    if (threadIdx.x < 7) {
        unsigned long long t = 0;
        for (int w = 0; w < 16; w++) t += red[w][threadIdx.x];
        counters[threadIdx.x] += t;
    }
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace

int h3_sol_bind(h3_gpu *g, h3_sol_router *r, const h3_sol_layout *layout, const h3_cuda_sol_options &o) {
    if (r->bound || !layout || !layout->query || !layout->key || !layout->sequence)
        return h3_set_error(g, "SOL: missing or already configured layout");
    const uint32_t seq = layout->sequence, qblock = (uint32_t)o.q_block;
    const uint32_t qblocks = (seq + qblock - 1) / qblock, kblocks = (seq + 63) / 64;
    if (layout->query_blocks != qblocks || layout->key_blocks != kblocks)
        return h3_set_error(g, "SOL: layout block counts disagree with policy");
    for (int which = 0; which < 2; which++) {
        const uint32_t count = which ? kblocks : qblocks, block = which ? 64 : qblock;
        const h3_sol_block *m = which ? layout->key : layout->query;
        for (uint32_t i = 0; i < count; i++)
            if (m[i].rows != std::min(block, seq - i * block) || m[i].first_frame < -1 ||
                m[i].last_frame < m[i].first_frame || m[i].last_frame > 10000000)
                return h3_set_error(g, "SOL: invalid protection metadata");
    }
    const size_t qbytes = (size_t)qblocks * sizeof(h3_sol_block), kbytes = (size_t)kblocks * sizeof(h3_sol_block);
    if (!h3_buffer_reserve(g, &r->meta, qbytes + kbytes, "SOL layout") ||
        !h3_hip_check(g, hipMemcpy(r->meta.ptr, layout->query, qbytes, hipMemcpyHostToDevice), "SOL layout") ||
        !h3_hip_check(g, hipMemcpy((uint8_t *)r->meta.ptr + qbytes, layout->key, kbytes, hipMemcpyHostToDevice),
                      "SOL layout"))
        return 0;
    if (!h3_buffer_reserve(g, &r->counters, 64, "SOL counters") ||
        !h3_hip_check(g, hipMemset(r->counters.ptr, 0, 64), "SOL counters"))
        return 0;
    r->options = o;
    r->seq = seq; r->qblocks = qblocks; r->kblocks = kblocks;
    r->bound = true;
    return 1;
}

namespace {
// Workspace of a SOL call: the centroids and moments of all heads, then the
// routes and lists of one head group. Offsets into r when r is set.
size_t sol_layout(uint32_t seq, uint32_t heads, uint32_t group, uint32_t QB, uint32_t KB, h3_sol_router *r) {
    const uint32_t kpad = (KB + 63) / 64 * 64, tiles = kpad / 64, units = (seq + 63) / 64;
    size_t off = 0, o[11];
    o[0] = off; off = align256(off + (size_t)heads * QB * D * 2);          // qc
    o[1] = off; off = align256(off + (size_t)KB * heads * D * 2);          // kc
    o[2] = off; off = align256(off + (size_t)heads * D * kpad * 2);        // vct
    o[3] = off; off = align256(off + (size_t)heads * 256 * 4);             // moments
    o[4] = off; off = align256(off + (size_t)group * QB * KB);             // routes
    o[5] = off; off = align256(off + (size_t)group * units * KB * 4);      // exact lists
    o[6] = off; off = align256(off + (size_t)group * units * 4);
    o[7] = off; off = align256(off + (size_t)group * units * tiles * 4);   // centroid lists
    o[8] = off; off = align256(off + (size_t)group * units * 4);
    o[9] = off; off = align256(off + (size_t)group * units * tiles * 16);  // approximate masks
    o[10] = off; off = align256(off + (size_t)group * units * 8 * 4);      // pair counts
    if (r) {
        r->off_qc = o[0]; r->off_kc = o[1]; r->off_vct = o[2]; r->off_moments = o[3]; r->off_routes = o[4];
        r->off_exact = o[5]; r->off_exact_count = o[6]; r->off_cent = o[7]; r->off_cent_count = o[8];
        r->off_cent_mask = o[9]; r->off_row_counts = o[10];
        r->kpad = kpad; r->tiles = tiles;
    }
    return off;
}
}  // namespace

int h3_sol_plan(h3_gpu *g, const h3_sol_router *r, uint32_t seq, uint32_t heads, uint32_t *group, size_t *bytes) {
    if (!r->bound) return h3_set_error(g, "SOL attention needs a bound layout (h3_gpu_dit_sol_layout)");
    if (seq != r->seq) return h3_set_error(g, "SOL layout was bound for sequence %u, not %u", r->seq, seq);
    for (uint32_t gr = heads;; gr = std::max(1u, gr / 2)) {
        const size_t need = sol_layout(seq, heads, gr, r->qblocks, r->kblocks, nullptr) +
                            h3_attention_bf16_workspace(seq, gr);
        if (need <= r->cap) { *group = gr; *bytes = need; return 1; }
        if (gr == 1) break;
    }
    return h3_set_error(g, "SOL: S=%u H=%u workspace plan exceeds its fixed budget of %zu bytes", seq, heads, r->cap);
}

int h3_sol_prepare(h3_gpu *g, h3_sol_router *r, const uint16_t *q, const uint16_t *k, const uint16_t *v, uint32_t seq,
                   uint32_t heads, uint32_t group) {
    const uint32_t QB = r->qblocks, KB = r->kblocks;
    const size_t bytes = sol_layout(seq, heads, group, QB, KB, r);
    if (!h3_buffer_reserve(g, &r->ws, bytes, "SOL workspace")) return 0;
    r->heads = heads; r->group = group;
    auto *base = (uint8_t *)r->ws.ptr;
    auto *qc = (uint16_t *)(base + r->off_qc), *kc = (uint16_t *)(base + r->off_kc);
    auto *vct = (uint16_t *)(base + r->off_vct);
    auto *moments = (float *)(base + r->off_moments);
    const uint32_t qblock = (uint32_t)r->options.q_block, kpad = r->kpad;
    const unsigned head_groups = (heads + 15) / 16;
    hipLaunchKernelGGL(sol_summary<SUM_Q>, dim3(QB, head_groups), dim3(256), 0, g->compute, q, qc, seq, heads, qblock, QB,
                       kpad, g->fault);
    hipLaunchKernelGGL(sol_summary<SUM_K>, dim3(KB, head_groups), dim3(256), 0, g->compute, k, kc, seq, heads, 64u, KB,
                       kpad, g->fault);
    hipLaunchKernelGGL(sol_summary<SUM_V>, dim3(kpad, head_groups), dim3(256), 0, g->compute, v, vct, seq, heads, 64u, KB,
                       kpad, g->fault);
    hipLaunchKernelGGL(sol_moments, dim3(heads), dim3(128), 0, g->compute, kc, moments, heads, KB);
    if (!h3_launch_status(g, "SOL summaries")) return 0;
    r->calls++;
    return 1;
}

int h3_sol_route(h3_gpu *g, h3_sol_router *r, uint32_t seq, uint32_t heads, uint32_t head0, uint32_t group,
                 float scale) {
    // The workspace is laid out for r->group heads; the last group of a split
    // may hold fewer (the reference runs min(head_group, heads - first),
    // cuda_sol.cu:388-389).
    if (!group || group > r->group || head0 + group > heads) return h3_set_error(g, "SOL: invalid head group");
    const uint32_t QB = r->qblocks, KB = r->kblocks, tiles = r->tiles;
    auto *base = (uint8_t *)r->ws.ptr;
    const auto *qc = (const uint16_t *)(base + r->off_qc), *kc = (const uint16_t *)(base + r->off_kc);
    const auto *moments = (const float *)(base + r->off_moments);
    const auto *qmeta = (const h3_sol_block *)r->meta.ptr;
    const auto *kmeta = qmeta + QB;
    const uint32_t qblock = (uint32_t)r->options.q_block;
    const unsigned minimum = (unsigned)std::ceil((double)r->options.min_exact * KB);
    const uint32_t units = (seq + 63) / 64;     // lists are per 64-query unit
    // Lists per 64-query unit: pairs of 32-row blocks, or single 64-row blocks.
    auto route = qblock == 32 ? sol_route<2> : sol_route<1>;
    hipLaunchKernelGGL(route, dim3((units + UPW - 1) / UPW, group), dim3(256), 0, g->compute, qc, kc, moments, qmeta,
                       kmeta, base + r->off_routes, (uint32_t *)(base + r->off_exact),
                       (uint32_t *)(base + r->off_exact_count), (uint32_t *)(base + r->off_cent),
                       (uint32_t *)(base + r->off_cent_count), (uint64_t *)(base + r->off_cent_mask), heads, QB, KB,
                       tiles, units, (unsigned)r->options.local_radius, minimum, scale, r->options.tau,
                       r->force_exact ? 1 : 0, (uint32_t *)(base + r->off_row_counts), head0);
    if (!h3_launch_status(g, "SOL route")) return 0;
    hipLaunchKernelGGL(sol_count, dim3(1), dim3(1024), 0, g->compute, (const uint32_t *)(base + r->off_row_counts),
                       (size_t)group * units, (unsigned long long *)r->counters.ptr);
    if (!h3_launch_status(g, "SOL counters")) return 0;
    r->pending = true;
    return 1;
}

void h3_sol_collect(h3_gpu *g, h3_sol_router *r) {
    (void)g;
    if (!r->pending) return;
    unsigned long long c[7];
    if (hipMemcpy(c, r->counters.ptr, sizeof(c), hipMemcpyDeviceToHost) != hipSuccess) return;
    if (hipMemset(r->counters.ptr, 0, sizeof(c)) != hipSuccess) return;
    for (int j = 0; j < 7; j++) r->pairs[j] += c[j];
    r->pending = false;
}

h3_sol_lists h3_sol_lists_of(const h3_sol_router *r) {
    const auto *base = (const uint8_t *)r->ws.ptr;
    h3_sol_lists l{};
    l.exact = (const uint32_t *)(base + r->off_exact);
    l.exact_count = (const uint32_t *)(base + r->off_exact_count);
    l.exact_stride = r->kblocks;       // per 64-query unit (ceil(seq / 64) per head)
    l.cent = (const uint32_t *)(base + r->off_cent);
    l.cent_count = (const uint32_t *)(base + r->off_cent_count);
    l.cent_mask = (const uint64_t *)(base + r->off_cent_mask);
    l.cent_stride = r->tiles;
    l.key_blocks = r->kblocks;
    l.kc_padded = r->kpad;
    l.kc = (const uint16_t *)(base + r->off_kc);
    l.vct = (const uint16_t *)(base + r->off_vct);
    return l;
}

void h3_sol_free(h3_sol_router *r) {
    h3_buffer_free(&r->ws);
    h3_buffer_free(&r->meta);
    h3_buffer_free(&r->counters);
    r->bound = false;
}

// Route and centroid capture for tests, the counterpart of the reference's
// h3_cuda_sol_routes (cuda_sol.cu:418-423): the last call's routes u8
// [heads][qblocks][kblocks] and centroids BF16 qc [heads][qblocks][128], kc and
// vc [heads][kblocks][128]. Any output may be null; counts must match.
extern "C" int h3_hip_sol_routes(h3_gpu *g, uint8_t *routes, size_t route_count, uint16_t *qc, size_t qc_count,
                                 uint16_t *kc, uint16_t *vc, size_t kv_count) {
    if (!g) return 0;
    auto *r = h3_attention_sol(g);
    if (!r || !r->heads) return h3_set_error(g, "SOL routes: no routed call yet");
    if (r->group != r->heads) return h3_set_error(g, "SOL routes: the last call ran in head groups; only whole calls are kept");
    const size_t H = r->heads, QB = r->qblocks, KB = r->kblocks;
    if (routes && route_count != H * QB * KB) return h3_set_error(g, "SOL routes: expected %zu routes", H * QB * KB);
    if (qc && qc_count != H * QB * D) return h3_set_error(g, "SOL routes: expected %zu query centroids", H * QB * D);
    if ((kc || vc) && kv_count != H * KB * D) return h3_set_error(g, "SOL routes: expected %zu key centroids", H * KB * D);
    if (!h3_hip_check(g, hipStreamSynchronize(g->compute), "SOL routes")) return 0;
    const auto *base = (const uint8_t *)r->ws.ptr;
    if (routes && !h3_hip_check(g, hipMemcpy(routes, base + r->off_routes, H * QB * KB, hipMemcpyDeviceToHost), "routes"))
        return 0;
    if (qc && !h3_hip_check(g, hipMemcpy(qc, base + r->off_qc, H * QB * D * 2, hipMemcpyDeviceToHost), "centroids"))
        return 0;
    if (kc) {
        std::vector<uint16_t> rows(KB * H * D);
        if (!h3_hip_check(g, hipMemcpy(rows.data(), base + r->off_kc, rows.size() * 2, hipMemcpyDeviceToHost), "centroids"))
            return 0;
        for (size_t h = 0; h < H; h++)
            for (size_t b = 0; b < KB; b++)
                std::copy_n(&rows[(b * H + h) * D], D, kc + (h * KB + b) * D);
    }
    if (vc) {
        const size_t kpad = r->kpad;
        std::vector<uint16_t> t(H * D * kpad);
        if (!h3_hip_check(g, hipMemcpy(t.data(), base + r->off_vct, t.size() * 2, hipMemcpyDeviceToHost), "centroids"))
            return 0;
        for (size_t h = 0; h < H; h++)
            for (size_t b = 0; b < KB; b++)
                for (size_t d = 0; d < D; d++)
                    vc[(h * KB + b) * D + d] = t[(h * D + d) * kpad + (b & ~(size_t)63) + vt_position((unsigned)(b & 63))];
    }
    return 1;
}
