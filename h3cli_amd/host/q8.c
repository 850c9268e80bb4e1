/* Host-side W8A16 packing with the reference's layout and rounding
 * (src/weights/q8.h:6-16, src/weights/q8.c:6-56): int8 [rows, columns] row-major,
 * then fp32 scales [rows, ceil(columns/64)] starting at a 4-byte aligned offset.
 * Per 64-wide group: scale = max|w| / 127, or 1 when the group is all zero,
 * floored at FLT_MIN; code = round-half-to-even(w / scale) clamped to +-127. */
#include <float.h>
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define Q8_GROUP 64u

int h3_q8_layout(uint32_t rows, uint32_t columns, size_t *offset, size_t *bytes) {
    if (!rows || !columns || columns > UINT32_MAX - (Q8_GROUP - 1u) || !offset || !bytes) return 0;
    uint64_t elements = (uint64_t)rows * columns;
    uint64_t groups = ((uint64_t)columns + Q8_GROUP - 1) / Q8_GROUP;
    if (elements > UINT32_MAX - 31u) return 0;
    uint64_t start = (elements + 3) & ~UINT64_C(3);
    uint64_t total = start + (uint64_t)rows * groups * sizeof(float);
    if (total > SIZE_MAX) return 0;
    *offset = (size_t)start;
    *bytes = (size_t)total;
    return 1;
}

static float widen(uint16_t bits) {
    uint32_t word = (uint32_t)bits << 16;
    float value;
    memcpy(&value, &word, sizeof(value));
    return value;
}

/* Round half to even of v, clamped to +-127. */
static int8_t code_of(float v) {
    float lo = floorf(v), frac = v - lo;
    long q = (long)lo;
    if (frac > 0.5f || (frac == 0.5f && (q & 1))) q++;
    return (int8_t)(q < -127 ? -127 : q > 127 ? 127 : q);
}

int h3_q8_pack_rows(const uint16_t *source, int8_t *weights, float *scales, uint32_t rows, uint32_t columns) {
    size_t offset, bytes;
    if (!source || !weights || !scales || !h3_q8_layout(rows, columns, &offset, &bytes)) return 0;
    uint32_t groups = (columns + Q8_GROUP - 1) / Q8_GROUP;
    for (uint32_t r = 0; r < rows; r++) {
        const uint16_t *row = source + (size_t)r * columns;
        for (uint32_t gi = 0; gi < groups; gi++) {
            uint32_t begin = gi * Q8_GROUP, end = begin + Q8_GROUP < columns ? begin + Q8_GROUP : columns;
            float amax = 0.f;
            for (uint32_t c = begin; c < end; c++) {
                float w = widen(row[c]);
                if (!isfinite(w)) return 0;
                if (fabsf(w) > amax) amax = fabsf(w);
            }
            float scale = amax == 0.f ? 1.f : fmaxf(amax / 127.f, FLT_MIN);
            scales[(size_t)r * groups + gi] = scale;
            for (uint32_t c = begin; c < end; c++) weights[(size_t)r * columns + c] = code_of(widen(row[c]) / scale);
        }
    }
    return 1;
}
