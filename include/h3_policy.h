/* h3_policy.h — host-side DiT attention policy used by the backend's dispatch:
 * the same names and meaning as the reference's src/denoise/attention.h:7-24
 * and src/denoise/subblock.h:12-24. libh3hip.so defines them weak, so the host
 * application's own definitions take precedence when both are linked. */
#ifndef H3_POLICY_H
#define H3_POLICY_H
#include <stddef.h>
#ifdef __cplusplus
extern "C" {
#endif
/* attention.h:7 */
enum { H3_ATTENTION_DEFAULT = 0, H3_ATTENTION_SAGE2 = 1, H3_ATTENTION_SAGE3 = 2, H3_ATTENTION_SOL = 3,
       H3_ATTENTION_SUBBLOCK = 4 };
const char *h3_attention_name(int mode);                          /* attention.h:14 */
int h3_attention_parse(const char *text, int *mode);               /* attention.h:19 */
int h3_attention_options(int mode, char *error, size_t size);      /* attention.h:20 */
int h3_attention_preflight(int mode, char *error, size_t size);    /* attention.h:21 */
/* subblock.h:16. 8 * ceil((1 - sparsity) * blocks / 8), capped at blocks. */
unsigned h3_subblock_budget(unsigned blocks, float sparsity);
int h3_subblock_warmup(int configured);                             /* subblock.h:17 */
/* subblock.h:20-21. "warmup" | "probe" | "short" | "full-budget" | NULL. */
const char *h3_subblock_dense_reason(unsigned sequence, unsigned block, int step, float sparsity, int warmup);
#ifdef __cplusplus
}
#endif
#endif
