/* h3_quant.h — quantized DiT projection policy, the reference's
 * src/weights/quant.h:1-36 names, constants and rules. libh3hip.so defines the
 * policy functions weak (host/quant.c), so a host that links its own
 * src/weights/quant.c keeps its definitions; h3_quant_preflight is the
 * backend's own (csrc/quant.hip), as src/cuda/cuda_quant.cuh:106-119 is. */
#ifndef H3_QUANT_H
#define H3_QUANT_H
#include <stddef.h>
#ifdef __cplusplus
extern "C" {
#endif

#define H3_QUANT_VERSION 2            /* packing recipe: tensorwide E4M3 (quant.h:7) */
#define H3_QUANT_ADAPTIVE_VERSION 3   /* quant.h:8 */
#define H3_QUANT_SUBBLOCK_VERSION 4   /* quant.h:9 */
enum { H3_QUANT_OFF = 0, H3_QUANT_FP8 = 1, H3_QUANT_NVFP4 = 2 };   /* quant.h:10 */
typedef struct { int mode; const char *cache; } h3_quant_scope;     /* quant.h:11 */

const char *h3_quant_name(int mode);                                 /* "off" | "fp8" | "nvfp4" | "invalid" */
int h3_quant_parse(const char *text, int *mode);
/* Mode 0..2; a cache path needs a nonempty value and a quantized mode and must
 * sit under a writable directory; H3_QUANT_VERIFY must be unset, 0 or 1. */
int h3_quant_options(int mode, const char *cache, char *error, size_t size);
int h3_quant_verify(void);                                           /* H3_QUANT_VERIFY=1: strict content cache */
/* The requested mode for the four per-block projections
 * blocks.<n>.{attn.qkv_proj,attn.out_proj,mlp.fc1,mlp.fc2}.weight, else off. */
int h3_quant_projection(const char *name, int requested);
unsigned h3_quant_recipe(int mode, int adaptive_cache);
unsigned h3_quant_execution_recipe(int mode, int adaptive_cache, int attention);
/* As h3_quant_projection, but block 0 stays BF16 under the adaptive cache. */
int h3_quant_projection_policy(const char *name, int requested, int adaptive_cache);
h3_quant_scope h3_quant_exchange(h3_quant_scope next);              /* thread-local; returns the previous */
h3_quant_scope h3_quant_current(void);
/* Backend capability: mode 0 always; modes 1 (FP8) and 2 (NVFP4, computed by
 * exact dequantization to BF16) on a gfx950 device. */
int h3_quant_preflight(int mode, char *error, size_t size);

#ifdef __cplusplus
}
#endif
#endif
