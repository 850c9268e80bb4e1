// SubBlock router (reference src/cuda/cuda_subblock.cu:256-324): pooled 16-row
// cells, 64 x 64 block scores, exact top-k selection with protected blocks,
// compacted into the per-head sparse lists the BF16 attention kernel walks.
#pragma once
#include "common.h"
#include "internal.h"
#include "../../include/h3_gpu_surface.h"
#include <vector>

// Fixed budget of a routed call's device workspace (router buffers plus the
// transposed V of one head group): the reference's attention workspace cap
// (src/denoise/attention.h:12).
constexpr size_t H3_SUBBLOCK_WORKSPACE_CAP = (size_t)512 << 20;

// How a routed call is split: heads in groups of `group`, 64-query blocks in
// slabs of `slab` (a multiple of 32 unless it covers the sequence); `bytes` is
// the router workspace plus the transposed V of one group.
struct h3_subblock_chunking {
    uint32_t group = 0, slab = 0;
    size_t router_bytes = 0, vt_bytes = 0, bytes = 0;
};

struct h3_subblock_router {
    bool bound = false;                    // a layout was bound for this context
    uint32_t seq = 0, blocks = 0;          // 64-row blocks of the bound layout
    uint32_t protected_ranges = 0;         // runs of protected query blocks
    std::vector<uint8_t> q_protect, k_protect;
    h3_device_buffer meta;                 // device copy: q_protect then k_protect
    h3_device_buffer ws;                   // pools, scores, routes, lists of one chunk
    h3_device_buffer counters;             // u64 [4]: kept, protected added (reset at collect)
    size_t cap = H3_SUBBLOCK_WORKSPACE_CAP;
    h3_subblock_chunking plan;             // of the last routed call
    // Geometry of the workspace for the last routed chunk.
    uint32_t heads = 0, cells = 0, group = 0, head0 = 0, qb0 = 0, qslab = 0;
    bool chunked = false;                  // the last call ran in more than one chunk
    size_t off_qpool = 0, off_kpool = 0, off_scores = 0, off_routes = 0, off_list = 0, off_count = 0, off_added = 0;
    bool counters_pending = false;
    uint64_t possible = 0;                 // route slots of the calls since the last collect
};

// Validates and stores a layout: query_blocks == key_blocks == ceil(seq / 64),
// block rows min(64, seq - 64 b) (reference cuda_subblock.cu:352-361).
int h3_subblock_bind(h3_gpu *g, h3_subblock_router *r, const h3_sol_layout *layout);
// Largest head group (heads, halved down to 1), then largest query slab (all
// blocks, else multiples of 32 blocks halving), whose chunk workspace fits
// r->cap. The loop shape is the reference's (src/denoise/subblock.c:18-42:
// head group outer, query slab inner), the slab sequence is not: the reference
// tries slabs 128, 64, ..., 1 and clamps the cap to 512 MiB, while the routed
// kernels here take slabs of whole 32-block rows and the cap is whatever
// h3_hip_subblock_workspace_cap set (512 MiB by default). The budget covers
// one chunk's router buffers and transposed V only; buffers the context
// already holds from earlier calls (its grow-only BF16 workspace) are not
// counted. Outputs do not depend on the split.
int h3_subblock_plan(h3_gpu *g, const h3_subblock_router *r, uint32_t seq, uint32_t heads, h3_subblock_chunking *out);
// One chunk: with pool set, pools Q and K of heads [head0, head0 + group)
// (q, k point at head 0; strides are those of `heads`); then scores the query
// blocks [qb0, qb0 + qslab) against every key block, selects `keep` key blocks
// per query block (plus protected ones) and writes, per (head, query block) of
// the slab, the ascending list of kept key blocks [group][qslab][blocks] and
// its length [group][qslab]. Enqueued on g->compute; valid until the next call.
int h3_subblock_route(h3_gpu *g, h3_subblock_router *r, const uint16_t *q, const uint16_t *k, uint32_t seq,
                      uint32_t heads, uint32_t head0, uint32_t group, uint32_t qb0, uint32_t qslab, float scale,
                      unsigned keep, bool force_all, bool pool);
const uint32_t *h3_subblock_lists(const h3_subblock_router *r);
const uint32_t *h3_subblock_counts(const h3_subblock_router *r);
// Folds the device route counters into g->stats (after the stream is idle).
void h3_subblock_collect(h3_gpu *g, h3_subblock_router *r);
void h3_subblock_free(h3_subblock_router *r);
