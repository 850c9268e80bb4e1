/* h3_quant.h — the backend's part of the reference's quantized-projection
 * interface (src/weights/quant.h): the recipe and mode constants that name
 * packed-weight artifacts, and h3_quant_preflight, which the reference's CUDA
 * backend implements (src/cuda/cuda_quant.cuh:106-119) and this library
 * implements for gfx950 (csrc/quant.hip). The host-side policy functions of
 * quant.h (names, parsing, per-tensor projection policy, the thread scope) stay
 * in the host's own src/weights/quant.c. */
#ifndef H3_QUANT_H
#define H3_QUANT_H
#include <stddef.h>
#ifdef __cplusplus
extern "C" {
#endif

#define H3_QUANT_VERSION 2            /* packing recipe: tensorwide E4M3 (quant.h:7) */
enum { H3_QUANT_OFF = 0, H3_QUANT_FP8 = 1, H3_QUANT_NVFP4 = 2 };   /* quant.h:10 */

/* quant.h:34. Mode 0 always passes; modes 1 (FP8) and 2 (NVFP4, computed by
 * exact dequantization to BF16) need a gfx950 device. */
int h3_quant_preflight(int mode, char *error, size_t size);

#ifdef __cplusplus
}
#endif
#endif
