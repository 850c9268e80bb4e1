/* h3_sglang_flash.h — FlashAttention-2-style forward with log-sum-exp on the
 * reference's stream-level interface (src/cuda/cuda_sglang_flash.h:8-16,
 * implementation src/cuda/cuda_sglang_flash.cu:14-74), which its backend
 * calls for SGLang-parity attention and, per protected query range, inside
 * SubBlock attention (src/cuda/gpu_cuda.cu:1633). Device pointers; `stream` is
 * a hipStream_t (NULL: the default stream). Returns 1 on success, 0 for
 * invalid or unsupported arguments (with a message in `error` when the shape
 * is valid but not supported here), -1 with a message when a launch fails.
 * Output and inputs are BF16 sequence-major [batch, sequence, heads, 128];
 * lse is FP32 [batch, heads, sequence] (query range: [heads, count]) holding
 * log(sum_j exp(scale * q . k_j)). */
#ifndef H3_SGLANG_FLASH_H
#define H3_SGLANG_FLASH_H
#include <stddef.h>
#ifdef __cplusplus
extern "C" {
#endif
/* cuda_sglang_flash.h:8-10. Non-causal BF16, dim 128, heads == kv_heads
 * (the main-DiT case); the reference's causal, dim-72 vision and grouped
 * K/V cases return 0 with a message. head_major_output writes [heads,
 * sequence, 128] per batch. */
int h3_sglang_flash(void *out, const void *q, const void *k, const void *v, float *lse, unsigned batch,
                    unsigned sequence, unsigned heads, unsigned kv_heads, unsigned dim, float scale, int causal,
                    int head_major_output, void *stream, char *error, size_t size);
/* cuda_sglang_flash.h:14-16. Query rows [first, first + count) against all
 * `sequence` keys, written at those rows of the full-size output (the
 * head-major output keeps the full sequence as its head stride). */
int h3_sglang_flash_query_range(void *out, const void *q, const void *k, const void *v, float *lse,
                                unsigned sequence, unsigned heads, unsigned first, unsigned count, float scale,
                                int head_major_output, void *stream, char *error, size_t size);
#ifdef __cplusplus
}
#endif
#endif
