/* Host-side attention policy of the DiT hot path: the mode names of the
 * reference's src/denoise/attention.h:7-24 and the SubBlock budget / dense-bypass
 * rules of src/denoise/subblock.c:7-51, restated.
 *
 * These functions belong to the caller's host build in h3cli (src/denoise/).
 * They are defined weak here so that libh3hip.so works standalone and yields to
 * the host's own definitions when it is linked into h3cli as a drop-in backend. */
#include "h3_policy.h"
#include <math.h>
#include <stdio.h>
#include <string.h>

#define WEAK __attribute__((weak))

static const char *const mode_names[] = {"default", "sage2++", "sage3", "sol", "subblock"};

WEAK const char *h3_attention_name(int mode) {
    return mode >= 0 && mode < 5 ? mode_names[mode] : "invalid";
}

WEAK int h3_attention_parse(const char *text, int *mode) {
    if (!text || !mode) return 0;
    for (int i = 0; i < 5; i++)
        if (!strcmp(text, mode_names[i])) { *mode = i; return 1; }
    return 0;
}

WEAK int h3_attention_options(int mode, char *error, size_t size) {
    if (mode >= 0 && mode <= 4) return 1;
    if (error && size) snprintf(error, size, "cuda-attention must be default, sage2++, sage3, sol or subblock");
    return 0;
}

/* Modes this backend runs: default (dense BF16), sage2++, sol and subblock. */
WEAK int h3_attention_preflight(int mode, char *error, size_t size) {
    if (!h3_attention_options(mode, error, size)) return 0;
    if (mode == 2) {
        if (error && size) snprintf(error, size, "%s attention is unsupported on the HIP backend", h3_attention_name(mode));
        return 0;
    }
    return 1;
}

/* Keep budget of a row of `blocks` key blocks: 8 * ceil((1 - sparsity) * blocks / 8),
 * capped at blocks; 0 for invalid input. */
WEAK unsigned h3_subblock_budget(unsigned blocks, float sparsity) {
    if (!blocks || !(sparsity >= 0.f) || sparsity >= 1.f) return 0;
    double keep = 8.0 * ceil((1.0 - (double)sparsity) * (double)blocks / 8.0);
    return keep >= (double)blocks ? blocks : (unsigned)keep;
}

WEAK int h3_subblock_warmup(int configured) { return configured ? configured : 10; }

/* Why a SubBlock call runs dense instead (NULL: it may run sparse). */
WEAK const char *h3_subblock_dense_reason(unsigned sequence, unsigned block, int step, float sparsity, int warmup) {
    if (step < h3_subblock_warmup(warmup)) return "warmup";
    if (block == 0) return "probe";
    if (sequence < 4096) return "short";
    unsigned blocks = (sequence + 63) / 64;
    if (h3_subblock_budget(blocks, sparsity) == blocks) return "full-budget";
    return NULL;
}

/* ---- SOL options (src/cuda/cuda_sol_policy.c:9-37), restated. ---- */
#include "h3_sol_policy.h"

static _Thread_local h3_cuda_sol_options sol_current = H3_CUDA_SOL_DEFAULT;

WEAK h3_cuda_sol_options h3_cuda_sol_current(void) { return sol_current; }

WEAK h3_cuda_sol_options h3_cuda_sol_exchange(h3_cuda_sol_options o) {
    h3_cuda_sol_options previous = sol_current;
    sol_current = o;
    return previous;
}

WEAK int h3_cuda_sol_options_valid(h3_cuda_sol_options o, char *error, size_t size) {
    int ok = (o.q_block == 32 || o.q_block == 64) && o.kv_block == 64 && o.dense_layers >= 0 &&
             o.dense_layers <= 50 && o.dense_steps >= 0 && o.dense_steps <= 1000 && o.local_radius >= 0 &&
             o.local_radius <= 10000 && isfinite(o.tau) && o.tau >= 0 && o.tau <= 16 && isfinite(o.min_exact) &&
             o.min_exact >= 0 && o.min_exact <= 1 && isfinite(o.dense_sigma) &&
             (o.dense_sigma == -1 || (o.dense_sigma >= 0 && o.dense_sigma <= 1));
    if (!ok && error && size)
        snprintf(error, size, "invalid CUDA SOL policy: Q=32|64, KV=64, layers=0..50, steps=0..1000, "
                              "radius=0..10000, tau=0..16, min-exact=0..1, sigma=-1|0..1");
    return ok;
}

WEAK int h3_cuda_sol_options_match(h3_cuda_sol_options a, h3_cuda_sol_options b, unsigned m) {
    return (!(m & H3_SOL_Q) || a.q_block == b.q_block) && (!(m & H3_SOL_KV) || a.kv_block == b.kv_block) &&
           (!(m & H3_SOL_LAYERS) || a.dense_layers == b.dense_layers) &&
           (!(m & H3_SOL_STEPS) || a.dense_steps == b.dense_steps) &&
           (!(m & H3_SOL_RADIUS) || a.local_radius == b.local_radius) && (!(m & H3_SOL_TAU) || a.tau == b.tau) &&
           (!(m & H3_SOL_MIN) || a.min_exact == b.min_exact) &&
           (!(m & H3_SOL_SIGMA) || a.dense_sigma == b.dense_sigma);
}

WEAK const char *h3_cuda_sol_dense_reason(h3_cuda_sol_options o, unsigned block, int step, float video,
                                          float audio) {
    if (step < 0 || !isfinite(video) || !isfinite(audio) || video < 0 || video > 1 || audio < 0 || audio > 1)
        return "invalid-noise";
    if (o.min_exact >= 1) return "all-exact";
    if (step < o.dense_steps) return "early-evaluation";
    if (o.dense_sigma >= 0 && fmaxf(video, audio) >= o.dense_sigma) return "high-noise";
    if (block < (unsigned)o.dense_layers) return "early-layer";
    return NULL;
}
