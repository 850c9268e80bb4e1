/* h3_q8.h — host-side W8A16 weight packing, same names, layout and rounding as
 * the reference's src/weights/q8.h:6-16 (implementation src/weights/q8.c:6-56). */
#ifndef H3_Q8_H
#define H3_Q8_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
#define H3_Q8_VERSION 1
#define H3_Q8_GROUP 64
/* q8.h:13. Codes int8 [rows, columns], then fp32 scales [rows, ceil(columns/64)]
 * at *scale_offset (4-byte aligned); *bytes is the total. */
int h3_q8_layout(uint32_t rows, uint32_t columns, size_t *scale_offset, size_t *bytes);
/* q8.h:15. Pack BF16 rows; returns 0 on a non-finite weight or invalid shape. */
int h3_q8_pack_rows(const uint16_t *source, int8_t *weights, float *scales,
                    uint32_t rows, uint32_t columns);
#ifdef __cplusplus
}
#endif
#endif
