// SOL routed attention (reference src/cuda/cuda_sol.cu:92-310): block centroids,
// threshold routing of exact vs centroid-approximated key blocks, and the
// per-(head, query block) lists the listed attention kernel walks.
#pragma once
#include "common.h"
#include "internal.h"
#include "../../include/h3_gpu_surface.h"
#include "../../include/h3_sol_policy.h"
#include <vector>

struct h3_sol_router {
    bool bound = false;
    h3_cuda_sol_options options = H3_CUDA_SOL_DEFAULT;
    bool force_exact = false;              // every key block exact (operator tests)
    uint32_t seq = 0, qblocks = 0, kblocks = 0;
    h3_device_buffer meta;                 // h3_sol_block query [qblocks], key [kblocks]
    h3_device_buffer ws;
    h3_device_buffer counters;             // u64 [7] pair counts, summed on the device per call
    // Collected counters (the reference's h3_cuda_sol_stats calls and pairs)
    // and the calls the dense bypass rules took.
    uint64_t calls = 0, bypass = 0, pairs[7] = {0, 0, 0, 0, 0, 0, 0};
    bool pending = false;
    // Workspace budget (centroids of all heads, routes and lists of one head
    // group, the group's transposed V) and the geometry of the last call.
    size_t cap = (size_t)512 << 20;
    uint32_t heads = 0, group = 0, kpad = 0, tiles = 0;
    size_t plan_bytes = 0;
    size_t off_qc = 0, off_kc = 0, off_vct = 0, off_moments = 0, off_routes = 0, off_exact = 0, off_exact_count = 0,
           off_cent = 0, off_cent_count = 0, off_cent_mask = 0, off_row_counts = 0;
};

// Validates a layout as the reference's configure (cuda_sol.cu:356-364):
// query_blocks = ceil(seq / q_block), key_blocks = ceil(seq / 64), true block
// rows, frames -1 <= first <= last <= 1e7.
int h3_sol_bind(h3_gpu *g, h3_sol_router *r, const h3_sol_layout *layout, const h3_cuda_sol_options &options);
// Largest head group (all heads, halved down to 1) whose workspace, with the
// group's transposed V, fits r->cap; bytes is that total.
int h3_sol_plan(h3_gpu *g, const h3_sol_router *r, uint32_t seq, uint32_t heads, uint32_t *group, size_t *bytes);
// Centroids of Q, K and V and the K moments of every head (enqueued on
// g->compute), in a workspace laid out for head groups of `group`.
int h3_sol_prepare(h3_gpu *g, h3_sol_router *r, const uint16_t *q, const uint16_t *k, const uint16_t *v, uint32_t seq,
                   uint32_t heads, uint32_t group);
// Routes and lists of heads [head0, head0 + group) for one call; scale is the
// call's (BF16-rounded) softmax scale. The lists hold the group's heads.
int h3_sol_route(h3_gpu *g, h3_sol_router *r, uint32_t seq, uint32_t heads, uint32_t head0, uint32_t group,
                 float scale);
h3_sol_lists h3_sol_lists_of(const h3_sol_router *r);
// Folds the device pair counters of the calls since the last collect into
// r->pairs (after the compute stream has drained).
void h3_sol_collect(h3_gpu *g, h3_sol_router *r);
void h3_sol_free(h3_sol_router *r);
