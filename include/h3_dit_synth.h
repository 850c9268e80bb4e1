/* h3_dit_synth.h — a DiT denoise step that exercises the whole hot path through
 * the operator ABI (no reference counterpart: it stands in for the reference's
 * src/denoise/dit.c encode_forward / run_block loop, dit.c:2286-2539 and
 * 2577-3038, on random-init weights). Two geometries: the benchmark's synthetic
 * 40-block model (h3_hip_dit_synth_default) and the real H3 block
 * (h3_hip_dit_synth_h3: dit.c:31-46, 50 blocks, hidden 5376, 56 heads x 128,
 * grouped QKV with per-head Q/K RMSNorm, 48 RoPE pairs, SwiGLU 14336).
 * Host C; every device operation goes through h3_gpu.h. */
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
    uint32_t hidden;            /* residual width: 5120 (H3: 5376); attention width is heads * 128 */
    uint32_t heads;             /* 40 (H3: 56) */
    uint32_t mlp;               /* 13824 GELU-tanh MLP (H3: 14336 SwiGLU) */
    uint32_t frames, height, width; /* video latent grid: 27 x 30 x 40 = 32400 rows */
    uint32_t audio_rows;        /* 1024 audio rows after the video rows */
    uint32_t latent;            /* latent width per row (patch embed in, head out) */
    uint32_t streamed_first;    /* blocks >= this stream from pinned host memory */
    float mask_density;         /* block-sparse density of 128x128 blocks; < 0 = dense */
    int attention_mode;         /* 1 sage2++ (int8 QK / fp8 PV), 0 BF16, 4 SubBlock router */
    float eps;                  /* AdaLN RMSNorm epsilon (1e-6) */
    float time;                 /* timestep of the modulation embedding (0.5) */
    uint64_t seed;
    uint32_t rope_half;         /* rotate-half pairs d <-> d + rope_half: 64 (H3: 48) */
    int swiglu;                 /* 1: fc1 -> 2 * mlp (gate rows, then up rows), SwiGLU, fc2 */
    int qk_norm;                /* 1: per-head RMSNorm of Q and K with learned [128] weights */
    int grouped_qkv;            /* 1: QKV rows grouped per head [heads, 3, 128] (H3 checkpoint layout) */
    float subblock_sparsity;    /* attention_mode 4: the request's sparsity (0.75) */
    int projection_quant;       /* 0: W8A16 q8 projections; 1: FP8 W8A8, 2: NVFP4 W4A4
                                   (h3_gpu_quant_configure mode 1/2, every block resident) */
    uint32_t trace_block;       /* 0: off; b + 1: each step keeps device copies of block b's stage
                                   tensors, read back as "trace.<stage>" (h3_hip_dit_synth_tensor) */
} h3_hip_dit_synth_config;

/* The benchmark geometry. */
h3_hip_dit_synth_config h3_hip_dit_synth_default(void);
/* The real H3 block geometry (reference dit.c:31-46): 50 blocks, hidden 5376,
 * 56 heads, SwiGLU 14336, grouped QKV, Q/K RMSNorm, 48 RoPE pairs (16 per
 * axis), eps 1e-5, BF16 attention; video grid 25 x 27 x 27 = 18225 rows (the
 * reference's 18,225-token attention case), no audio rows, all blocks resident. */
h3_hip_dit_synth_config h3_hip_dit_synth_h3(void);

/* The 256-d timestep features of reference dit_schedule.c:152-162 for rows
 * of times: features[row, i] = cos(t * f_i) for i < 128 and
 * features[row, 128 + i] = sin(t * f_i), f_i = exp(-ln(1e4) * i / 128), in
 * FP32 as the reference computes them. */
void h3_hip_dit_time_features(const float *times, uint32_t rows, float *features);

/* 3D RoPE cos/sin tables [frames * height * width + audio_rows, half] as BF16
 * bits, rows frame-major then row then column, audio rows angle 0. Pair j of
 * axis a (frame, row, column) has inv_freq theta^(-2 i / dim_a), theta 1e4,
 * i = j - first pair of the axis; half 64 splits 22/21/21 pairs (44/42/42
 * channels), a multiple of 3 below 64 splits evenly (reference dit.c:1051-1090
 * with ROPE_FREQS = half / 3). angle = position * inv_freq in FP32 (inv_freq
 * rounded to FP32, as read from the reference's rope.inv_freq weights), then
 * cosf / sinf and BF16 rounding. Returns 0 on invalid arguments. */
int h3_hip_dit_rope_tables(uint32_t frames, uint32_t height, uint32_t width, uint32_t audio_rows, uint32_t half,
                           uint16_t *cosines, uint16_t *sines);

typedef struct h3_hip_dit_synth h3_hip_dit_synth;

/* Build the model on a fresh context (configures its DiT attention mode, binds
 * the block mask): seeded W8A16 projection weights (int8 U[-127,127], per-output
 * channel fp32 scales U[1e-3,1e-2]) or, with projection_quant 1 or 2, FP8 or
 * NVFP4 weights packed from N(0, 1/k) BF16 values (the context's quantization is configured,
 * artifacts under $TMPDIR/h3cli-amd-quant), AdaLN norms and modulation from a 256-d
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

/* Replaces the block weights with those of a safetensors checkpoint that uses
 * the reference's names (dit.c:592-611): "blocks.<b>." + "norm1.weight" and
 * "norm2.weight" [hidden], "attn.qkv_proj.weight" [3 * heads * 128, hidden],
 * "attn.q_norm.weight" and "attn.k_norm.weight" [128] (loaded when qk_norm),
 * "attn.out_proj.weight" [hidden, heads * 128], "mlp.fc1.weight" [2 * mlp
 * (SwiGLU) or mlp, hidden], "mlp.fc2.weight" [hidden, mlp]; all BF16. The four
 * projections are packed to W8A16 on the device with the reference q8 recipe
 * (group 64), or with projection_quant 1 / 2 to FP8 / NVFP4 through
 * h3_gpu_quant_load and its artifact cache. Every block must be resident (streamed_first >= blocks); no
 * command may be active. Errors name the first missing or mismatched tensor. */
int h3_hip_dit_synth_load(h3_hip_dit_synth *model, const char *path, char *error, size_t error_size);

/* Model tensors for inspection: "latent" (F32 [rows, latent]), "hidden" (BF16
 * [rows, hidden], the residual stream after the last block), "velocity",
 * "latent_bf16" (the patch-embedding input), "patch" [hidden, latent], "head"
 * [latent, hidden], "head_norm", "head_mod" [2, 2, hidden], "rope_cos" and
 * "rope_sin" [rows, rope_half], "row_map" (U32 [rows]: 0 video, 1 audio), a
 * block's modulation "blocks.<b>.modulation" [2, 6, hidden], a resident
 * block's weights under the checkpoint names above
 * ("blocks.0.attn.qkv_proj.weight": a W8A16 tensor; norms BF16), and with
 * trace_block the traced block's stages "trace.x0" (block input), "xn1"
 * (AdaLN), "qkv", "q", "k", "v", "attn", "o" (out projection), "x1" (gated
 * residual), "xn2" (second AdaLN), "h" (fc1, GELU applied when fused),
 * "act" (SwiGLU or separate GELU), "f" (fc2) and "x2" (block output), and
 * the modulation chain's tensors: "time.features" (BF16 [2, 256] timestep
 * features), "time.w1" [hidden, 256], "time.t1" [2, hidden] (first
 * projection, the SiLU input), "time.w2" [6 hidden, hidden], "time.shared"
 * [2, 6, hidden] (second projection) and "trace.mod_table" [2, 6, hidden]
 * (the traced block's own table, added to time.shared). */
h3_gpu_tensor *h3_hip_dit_synth_tensor(h3_hip_dit_synth *model, const char *name);
uint32_t h3_hip_dit_synth_rows(const h3_hip_dit_synth *model);
/* Kept 128x128 blocks of the bound mask and the total (for FLOP accounting). */
uint64_t h3_hip_dit_synth_kept_blocks(const h3_hip_dit_synth *model, uint64_t *total);

#ifdef __cplusplus
}
#endif
#endif
