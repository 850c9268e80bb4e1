// SubBlock router (reference src/cuda/cuda_subblock.cu:256-324): pooled 16-row
// cells, 64 x 64 block scores, exact top-k selection with protected blocks,
// compacted into the per-head sparse lists the BF16 attention kernel walks.
#pragma once
#include "common.h"
#include "internal.h"
#include "../../include/h3_gpu_surface.h"
#include <vector>

struct h3_subblock_router {
    bool bound = false;                    // a layout was bound for this context
    uint32_t seq = 0, blocks = 0;          // 64-row blocks of the bound layout
    uint32_t protected_ranges = 0;         // runs of protected query blocks
    std::vector<uint8_t> q_protect, k_protect;
    h3_device_buffer meta;                 // device copy: q_protect then k_protect
    h3_device_buffer ws;                   // pools, scores, routes, lists, counters
    // Geometry of the workspace for the last routed call.
    uint32_t heads = 0, cells = 0;
    size_t off_qpool = 0, off_kpool = 0, off_scores = 0, off_routes = 0, off_list = 0, off_count = 0, off_added = 0,
           off_counters = 0;
    bool counters_pending = false;
    uint64_t possible = 0;                 // route slots of the calls since the last collect
};

// Validates and stores a layout: query_blocks == key_blocks == ceil(seq / 64),
// block rows min(64, seq - 64 b) (reference cuda_subblock.cu:352-361).
int h3_subblock_bind(h3_gpu *g, h3_subblock_router *r, const h3_sol_layout *layout);
// Pools Q and K, scores every block pair, selects `keep` key blocks per query
// block (plus protected ones) and writes, per (head, query block), the
// ascending list of kept key blocks [heads][B][B] and its length [heads][B]. Enqueued on
// g->compute; the lists stay valid until the next call.
int h3_subblock_route(h3_gpu *g, h3_subblock_router *r, const uint16_t *q, const uint16_t *k, uint32_t seq,
                      uint32_t heads, float scale, unsigned keep, bool force_all);
const uint32_t *h3_subblock_lists(const h3_subblock_router *r);
const uint32_t *h3_subblock_counts(const h3_subblock_router *r);
// Folds the device route counters into g->stats (after the stream is idle).
void h3_subblock_collect(h3_gpu *g, h3_subblock_router *r);
void h3_subblock_free(h3_subblock_router *r);
