/* Quantized-projection policy restated from the reference's
 * src/weights/quant.c:9-65 (same names, decisions and error texts). Weak: a host
 * application that links its own src/weights/quant.c keeps its definitions. */
#define _GNU_SOURCE
#include "h3_quant.h"
#include <errno.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#define WEAK __attribute__((weak))

static _Thread_local h3_quant_scope current_scope;

WEAK int h3_quant_verify(void) {
    const char *v = getenv("H3_QUANT_VERIFY");
    return v && strcmp(v, "1") == 0;
}

WEAK const char *h3_quant_name(int mode) {
    switch (mode) {
    case H3_QUANT_OFF: return "off";
    case H3_QUANT_FP8: return "fp8";
    case H3_QUANT_NVFP4: return "nvfp4";
    default: return "invalid";
    }
}

WEAK int h3_quant_parse(const char *text, int *mode) {
    if (!text || !mode) return 0;
    for (int m = H3_QUANT_OFF; m <= H3_QUANT_NVFP4; m++)
        if (strcmp(text, h3_quant_name(m)) == 0) { *mode = m; return 1; }
    return 0;
}

/* blocks.<digits><suffix> with one of the four projection suffixes. */
WEAK int h3_quant_projection(const char *name, int requested) {
    static const char *const suffixes[] = {".attn.qkv_proj.weight", ".attn.out_proj.weight", ".mlp.fc1.weight",
                                           ".mlp.fc2.weight"};
    if (!name || strncmp(name, "blocks.", 7) != 0) return H3_QUANT_OFF;
    const char *p = name + 7;
    if (*p < '0' || *p > '9') return H3_QUANT_OFF;
    while (*p >= '0' && *p <= '9') p++;
    for (unsigned i = 0; i < sizeof(suffixes) / sizeof(suffixes[0]); i++)
        if (strcmp(p, suffixes[i]) == 0) return requested;
    return H3_QUANT_OFF;
}

WEAK unsigned h3_quant_recipe(int mode, int adaptive_cache) {
    if (!mode) return 0;
    return adaptive_cache ? H3_QUANT_ADAPTIVE_VERSION : H3_QUANT_VERSION;
}

/* Attention mode 4 is SubBlock (reference src/denoise/attention.h). */
WEAK unsigned h3_quant_execution_recipe(int mode, int adaptive_cache, int attention) {
    if (mode && attention == 4) return H3_QUANT_SUBBLOCK_VERSION;
    return h3_quant_recipe(mode, adaptive_cache);
}

WEAK int h3_quant_projection_policy(const char *name, int requested, int adaptive_cache) {
    if (adaptive_cache && name && strncmp(name, "blocks.0.", 9) == 0) return H3_QUANT_OFF;
    return h3_quant_projection(name, requested);
}

/* The nearest existing ancestor of `path` must be a writable, searchable
 * directory; nothing is created. */
static int writable_parent(const char *path) {
    char *dir = strdup(path);
    if (!dir) return 0;
    struct stat st;
    int ok = 1;
    while (stat(dir, &st) != 0) {
        if (errno != ENOENT) { ok = 0; break; }
        char *slash = strrchr(dir, '/');
        if (!slash) { strcpy(dir, "."); break; }
        if (slash == dir) { dir[1] = 0; break; }
        *slash = 0;
    }
    if (ok) ok = stat(dir, &st) == 0 && S_ISDIR(st.st_mode) && access(dir, W_OK | X_OK) == 0;
    free(dir);
    return ok;
}

WEAK int h3_quant_options(int mode, const char *cache, char *error, size_t size) {
    const char *verify = getenv("H3_QUANT_VERIFY"), *message = NULL;
    if (mode < 0 || mode > 2) message = "cuda-denoise-quant must be off, fp8 or nvfp4";
    else if (cache && (!*cache || !mode)) message = "cuda-denoise-quant-cache requires a nonempty path and quantized denoising";
    else if (mode && verify && strcmp(verify, "0") != 0 && strcmp(verify, "1") != 0) message = "H3_QUANT_VERIFY must be 0 or 1";
    if (message) {
        if (error && size) snprintf(error, size, "%s", message);
        return 0;
    }
    if (mode && cache && !writable_parent(cache)) {
        if (error && size) snprintf(error, size, "quantization cache path is not a writable directory: %s", cache);
        return 0;
    }
    return 1;
}

WEAK h3_quant_scope h3_quant_exchange(h3_quant_scope next) {
    h3_quant_scope previous = current_scope;
    current_scope = next;
    return previous;
}

WEAK h3_quant_scope h3_quant_current(void) { return current_scope; }
