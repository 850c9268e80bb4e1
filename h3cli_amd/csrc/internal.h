// Cross-translation-unit hooks inside the backend (not exported).
#pragma once
#include "common.h"

int h3_attention_init(h3_gpu *g);
void h3_attention_destroy(h3_gpu *g);
void h3_attention_collect_timing(h3_gpu *g);
void h3_streaming_destroy(h3_gpu *g);
int h3_tensor_events(h3_gpu *g, h3_gpu_tensor *t);
int h3_tensor_acquire(h3_gpu *g, const h3_gpu_tensor *t);
int h3_tensor_release(h3_gpu *g, const h3_gpu_tensor *t);

// Launch helpers of the kernel translation units (all enqueue on g->compute).
int h3_launch_attention_bf16(h3_gpu *g, uint16_t *out, const uint16_t *q, const uint16_t *k,
                             const uint16_t *v, uint32_t seq, uint32_t heads, float scale,
                             bool head_major, const uint32_t *kv_list, const uint32_t *kv_count,
                             uint32_t list_stride);
