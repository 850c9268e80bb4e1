/* Host-side W8A16 packing (the reference's src/weights/q8.h interface).
 *
 * Storage, which packed files share with the reference: int8 codes
 * [rows, columns] row-major, then float scales [rows, ceil(columns / 64)]
 * starting at the first 4-byte boundary after the codes. Per 64-column group:
 * scale = max|w| / 127 (1 for an all-zero group, never below FLT_MIN) and
 * code = w / scale rounded to nearest, ties to even, clamped to [-127, 127].
 * A non-finite weight refuses the whole tensor. The device packer
 * (q8_pack_kernel) computes the same bytes on the GPU. */
#include "h3_q8.h"
#include <float.h>
#include <math.h>
#include <string.h>

/* Accepted shapes: the code plane stays below 2^32 - 32 bytes, the limit of
 * the format's 32-bit addressing (a shape the reference refuses is refused
 * here too, so both sides agree on which checkpoints pack). */
#define Q8_MAX_CODES (UINT32_MAX - 31u)

int h3_q8_layout(uint32_t rows, uint32_t columns, size_t *scale_offset, size_t *bytes) {
    if (!scale_offset || !bytes || rows == 0 || columns == 0) return 0;
    if ((uint64_t)columns + (H3_Q8_GROUP - 1) > UINT32_MAX) return 0;
    const uint64_t codes = (uint64_t)rows * columns;
    if (codes > Q8_MAX_CODES) return 0;
    const uint64_t groups = ((uint64_t)columns + H3_Q8_GROUP - 1) / H3_Q8_GROUP;
    const uint64_t scales_at = (codes + 3) / 4 * 4;
    const uint64_t end = scales_at + (uint64_t)rows * groups * 4;
    if (end > SIZE_MAX) return 0;
    *scale_offset = (size_t)scales_at;
    *bytes = (size_t)end;
    return 1;
}

/* BF16 magnitude bits order like the magnitudes themselves; 0x7f80 and above
 * are infinities and NaNs. */
static float bf16_value(uint16_t bits) {
    const uint32_t word = (uint32_t)bits << 16;
    float f;
    memcpy(&f, &word, 4);
    return f;
}

/* Packs one group of n weights; 0 if any is not finite. */
static int pack_group(const uint16_t *w, uint32_t n, int8_t *codes, float *scale_out) {
    uint16_t top = 0;
    for (uint32_t i = 0; i < n; i++) {
        const uint16_t mag = w[i] & 0x7fffu;
        if (mag >= 0x7f80u) return 0;
        if (mag > top) top = mag;
    }
    const float amax = bf16_value(top);
    const float scale = top ? fmaxf(amax / 127.0f, FLT_MIN) : 1.0f;
    *scale_out = scale;
    for (uint32_t i = 0; i < n; i++) {
        /* rintf rounds half to even in the default rounding mode. */
        const float q = rintf(bf16_value(w[i]) / scale);
        codes[i] = (int8_t)(q > 127.f ? 127 : q < -127.f ? -127 : (int)q);
    }
    return 1;
}

int h3_q8_pack_rows(const uint16_t *source, int8_t *weights, float *scales, uint32_t rows, uint32_t columns) {
    size_t scale_offset, bytes;
    if (!source || !weights || !scales || !h3_q8_layout(rows, columns, &scale_offset, &bytes)) return 0;
    const uint32_t groups = (columns + H3_Q8_GROUP - 1) / H3_Q8_GROUP;
    size_t at = 0;
    for (uint32_t r = 0; r < rows; r++, at += columns)
        for (uint32_t g = 0; g < groups; g++) {
            const uint32_t first = g * H3_Q8_GROUP;
            const uint32_t n = columns - first < H3_Q8_GROUP ? columns - first : H3_Q8_GROUP;
            if (!pack_group(source + at + first, n, weights + at + first, scales + (size_t)r * groups + g)) return 0;
        }
    return 1;
}
