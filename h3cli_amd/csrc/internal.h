// Cross-translation-unit hooks inside the backend (not exported).
#pragma once
#include "common.h"

int h3_attention_init(h3_gpu *g);
void h3_attention_destroy(h3_gpu *g);
void h3_attention_collect_timing(h3_gpu *g);
struct h3_subblock_router *h3_attention_router(h3_gpu *g);
int h3_attention_mode(h3_gpu *g);
struct h3_sol_router *h3_attention_sol(h3_gpu *g);          // configured DiT attention mode (0 when unconfigured)
void h3_streaming_destroy(h3_gpu *g);
int h3_tensor_events(h3_gpu *g, h3_gpu_tensor *t);
int h3_tensor_acquire(h3_gpu *g, const h3_gpu_tensor *t);
int h3_tensor_release(h3_gpu *g, const h3_gpu_tensor *t);

// Launch helpers of the kernel translation units (all enqueue on g->compute).
size_t h3_attention_bf16_workspace(uint32_t seq, uint32_t heads);
int h3_launch_attention_bf16(h3_gpu *g, void *workspace, uint16_t *out, const uint16_t *q, const uint16_t *k,
                             const uint16_t *v, uint32_t seq, uint32_t heads, float scale,
                             bool head_major, const uint32_t *kv_list, const uint32_t *kv_count,
                             uint32_t list_stride);
// Dense attention of qrows query rows (q, out offset to the first) over seq
// keys with the FP32 natural-log LSE per (head, query row) into lse [heads, qrows].
int h3_launch_attention_flash(h3_gpu *g, void *workspace, uint16_t *out, const uint16_t *q, const uint16_t *k,
                              const uint16_t *v, float *lse, uint32_t seq, uint32_t qrows, uint32_t heads,
                              float scale, bool head_major);
// Routed attention of heads [head0, head0 + group) and 64-query blocks
// [qb0, qb0 + qslab) over lists of kept 64-key tiles, slab-relative:
// lists [group][qslab][list_stride], counts [group][qslab]. workspace holds
// the group's transposed V (written first when transpose is set).
int h3_launch_attention_routed(h3_gpu *g, void *workspace, uint16_t *out, const uint16_t *q, const uint16_t *k,
                               const uint16_t *v, uint32_t seq, uint32_t heads, float scale, bool head_major,
                               const uint32_t *lists, const uint32_t *counts, uint32_t list_stride,
                               uint32_t head0, uint32_t group, uint32_t qb0, uint32_t qslab, bool transpose);

// SOL attention lists (see csrc/sol.hip): exact tiles per (head, query block),
// centroid tiles with their approximate-block masks, and the centroid arrays.
struct h3_sol_lists {
    const uint32_t *exact, *exact_count;
    uint32_t exact_stride;
    const uint32_t *cent, *cent_count;
    const uint64_t *cent_mask;
    uint32_t cent_stride, key_blocks, kc_padded;
    const uint16_t *kc, *vct;
};
// SOL attention of heads [head0, head0 + group): lists hold the group's heads,
// kc / vct all heads; workspace receives the group's transposed V.
int h3_launch_attention_sol(h3_gpu *g, void *workspace, uint16_t *out, const uint16_t *q, const uint16_t *k,
                            const uint16_t *v, uint32_t seq, uint32_t heads, float scale, bool head_major,
                            uint32_t q_block, const h3_sol_lists *lists, uint32_t head0, uint32_t group);

// Grow-only device buffer; growing waits for queued work that may read the old one.
// FP8 projections (quant.hip): y = FP8 GEMM of x with a packed weight; teardown.
int h3_quant_gemm(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in, const h3_gpu_tensor *w, uint32_t rows,
                  uint32_t k, uint32_t n);
void h3_quant_destroy(h3_gpu *g);
// y[M,N] = bf16(alpha[0] * x . w^T), BF16 device operands, device scalar alpha (gemm.hip).
int h3_gemm_bf16_alpha(h3_gpu *g, uint16_t *y, const uint16_t *x, const uint16_t *w, const float *alpha, uint32_t m,
                       uint32_t k, uint32_t n);

struct h3_device_buffer {
    void *ptr = nullptr;
    size_t bytes = 0;
};
int h3_buffer_reserve(h3_gpu *g, h3_device_buffer *b, size_t bytes, const char *what);
void h3_buffer_free(h3_device_buffer *b);

// Dominant-kernel timing: h3_kernel_timing_begin records a start event on the
// compute stream when timing is enabled (else returns nullptr); _end records the
// stop event and queues the pair for h3_hip_kernel_timing_read.
hipEvent_t h3_kernel_timing_begin(h3_gpu *g);
void h3_kernel_timing_end(h3_gpu *g, hipEvent_t start);
