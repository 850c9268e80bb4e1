/* h3_sol_policy.h — SOL routed-attention options (attention mode 3), the
 * reference's src/cuda/cuda_sol_policy.h:9-26 types and host rules. The
 * request's options reach the backend through the calling thread's current
 * options (h3_cuda_sol_current), read at h3_gpu_dit_attention_configure(3)
 * as the reference's gpu_cuda.cu:1553-1555 does. libh3hip.so defines the
 * functions weak, so the host's own definitions win when both are linked. */
#ifndef H3_SOL_POLICY_H
#define H3_SOL_POLICY_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* cuda_sol_policy.h:12-15 */
typedef struct {
    int q_block, kv_block, dense_layers, dense_steps, local_radius;
    float tau, min_exact, dense_sigma;
} h3_cuda_sol_options;
#define H3_CUDA_SOL_DEFAULT {32, 64, 1, 1, 1, 1.0f, 0.0f, -1.0f}
/* cuda_sol_policy.h:16-17: field masks of h3_cuda_sol_options_match. */
enum { H3_SOL_Q = 1, H3_SOL_KV = 2, H3_SOL_LAYERS = 4, H3_SOL_STEPS = 8,
       H3_SOL_RADIUS = 16, H3_SOL_TAU = 32, H3_SOL_MIN = 64, H3_SOL_SIGMA = 128 };

/* Q 32|64, KV 64, layers 0..50, steps 0..1000, radius 0..10000, tau 0..16,
 * min_exact 0..1, sigma -1 or 0..1 (cuda_sol_policy.c:12-24). */
int h3_cuda_sol_options_valid(h3_cuda_sol_options o, char *error, size_t size);
int h3_cuda_sol_options_match(h3_cuda_sol_options a, h3_cuda_sol_options b, unsigned mask);
/* "invalid-noise" | "all-exact" | "early-evaluation" | "high-noise" |
 * "early-layer" | NULL (cuda_sol_policy.c:30-37). */
const char *h3_cuda_sol_dense_reason(h3_cuda_sol_options o, unsigned block, int step, float video, float audio);
h3_cuda_sol_options h3_cuda_sol_current(void);                            /* thread-local, :9 */
h3_cuda_sol_options h3_cuda_sol_exchange(h3_cuda_sol_options o);          /* returns the previous, :10 */

#ifdef __cplusplus
}
#endif
#endif
