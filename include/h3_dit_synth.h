/* h3_dit_synth.h — the synthetic 40-block DiT denoise step that exercises the
 * whole hot path through the operator ABI (no reference counterpart: it stands
 * in for the reference's src/denoise/dit.c encode_forward / run_block loop,
 * dit.c:2286-2539 and 2577-3038, on random-init weights of the benchmark's
 * synthetic geometry). Host C; every device operation goes through h3_gpu.h. */
#ifndef H3_DIT_SYNTH_H
#define H3_DIT_SYNTH_H
#include <stddef.h>
#include <stdint.h>
#include "h3_gpu.h"
#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    uint32_t blocks;            /* 40 */
    uint32_t hidden;            /* 5120 (heads * 128) */
    uint32_t heads;             /* 40 */
    uint32_t mlp;               /* 13824, GELU-tanh MLP */
    uint32_t frames, height, width; /* video latent grid: 27 x 30 x 40 = 32400 rows */
    uint32_t audio_rows;        /* 1024 audio rows after the video rows */
    uint32_t latent;            /* latent width per row (patch embed in, head out) */
    uint32_t streamed_first;    /* blocks >= this stream from pinned host memory */
    float mask_density;         /* block-sparse density of 128x128 blocks; < 0 = dense */
    int attention_mode;         /* 1 sage2++ (int8 QK / fp8 PV), 0 BF16 */
    float eps;                  /* AdaLN RMSNorm epsilon (1e-6) */
    float time;                 /* timestep of the modulation embedding (0.5) */
    uint64_t seed;
} h3_hip_dit_synth_config;

/* The benchmark geometry. */
h3_hip_dit_synth_config h3_hip_dit_synth_default(void);

typedef struct h3_hip_dit_synth h3_hip_dit_synth;

/* Build the model on a fresh context (configures its DiT attention mode, binds
 * the block mask): seeded W8A16 projection weights (int8 U[-127,127], per-output
 * channel fp32 scales U[1e-3,1e-2]), AdaLN norms and modulation from a 256-d
 * sinusoidal timestep embedding, 3D RoPE tables, a seeded latent. Blocks from
 * streamed_first on live in pinned host memory and are copied into two device
 * slots on the copy stream one block ahead of use. */
h3_hip_dit_synth *h3_hip_dit_synth_create(h3_gpu *gpu, const h3_hip_dit_synth_config *config,
                                          char *error, size_t error_size);
void h3_hip_dit_synth_free(h3_hip_dit_synth *model);

/* One denoise evaluation and Euler update, latent += dt * velocity, inside its
 * own h3_gpu_begin / h3_gpu_submit (no command may be active). step is the
 * absolute sampler step bound for sparse attention. */
int h3_hip_dit_synth_step(h3_hip_dit_synth *model, int step, float dt);

/* Model tensors for inspection: "latent" (F32 [rows, latent]), "hidden" (BF16
 * [rows, hidden], the residual stream after the last block), "velocity",
 * "mask" (U32 kept-block count in element 0 is not provided; use the config). */
h3_gpu_tensor *h3_hip_dit_synth_tensor(h3_hip_dit_synth *model, const char *name);
uint32_t h3_hip_dit_synth_rows(const h3_hip_dit_synth *model);
/* Kept 128x128 blocks of the bound mask and the total (for FLOP accounting). */
uint64_t h3_hip_dit_synth_kept_blocks(const h3_hip_dit_synth *model, uint64_t *total);

#ifdef __cplusplus
}
#endif
#endif
