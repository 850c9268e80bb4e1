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

/* Modes this backend runs: default (dense BF16), sage2++ and subblock. */
WEAK int h3_attention_preflight(int mode, char *error, size_t size) {
    if (!h3_attention_options(mode, error, size)) return 0;
    if (mode == 2 || mode == 3) {
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
