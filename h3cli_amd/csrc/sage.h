// Sage-style quantized attention (int8 Q.K^T, fp8 e4m3 P.V) for gfx950.
#pragma once
#include "common.h"

// Device workspace for one quantized attention call, grown on demand.
struct h3_sage_workspace {
    void *base = nullptr;
    size_t bytes = 0;
};
void h3_sage_workspace_free(h3_sage_workspace *w);

// Layout of the packed operands inside a workspace (byte offsets).
struct h3_sage_layout {
    unsigned seq, heads, padded, blocks, partials;
    size_t q8, k8, v8, q_scale, k_scale, v_scale, v_recip, k_mean, sums, maxima, retry, total;
};
h3_sage_layout h3_sage_plan(unsigned seq, unsigned heads);

// Enqueue the quantizers into the given buffers (all device pointers).
int h3_sage_quantize(h3_gpu *g, const h3_sage_layout &L, char *ws, const uint16_t *q, const uint16_t *k,
                     const uint16_t *v);
int h3_sage_attention(h3_gpu *g, h3_sage_workspace *w, uint16_t *out, const uint16_t *q, const uint16_t *k,
                      const uint16_t *v, unsigned seq, unsigned heads, float scale, bool head_major,
                      const uint32_t *kv_list, const uint32_t *kv_count, unsigned list_stride);

// fp8 e4m3 (OCP, "fn": max 448, no infinities) encode, round-to-nearest-even,
// saturating at 448. NaN encodes as 0x7f with the input sign.
__host__ __device__ inline uint8_t f32_to_e4m3(float x) {
    uint32_t u = __builtin_bit_cast(uint32_t, x);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7fu;
    float f = __builtin_bit_cast(float, a);
    if (f >= 464.0f) return sign | 0x7eu;                 // beyond the 448/512 midpoint
    if (f < 0.015625f) {                                   // below 2^-6: subnormal grid of 2^-9
        float m = __builtin_rintf(f * 512.0f);             // exact scaling, RNE
        return sign | (uint8_t)m;                          // m == 8 is the smallest normal 0x08
    }
    int e = (int)(a >> 23) - 127;                          // -6 .. 8
    uint32_t mant = a & 0x7fffffu, r = mant >> 20, rem = mant & 0xfffffu;
    if (rem > 0x80000u || (rem == 0x80000u && (r & 1u))) r++;
    if (r == 8) { r = 0; e++; }
    uint32_t code = ((uint32_t)(e + 7) << 3) | r;
    if (code > 0x7eu) code = 0x7eu;
    return sign | (uint8_t)code;
}

// Position of key j (0..63) of a 64-key tile inside a packed fp8 V row: the
// order in which a lane half holds the keys of the two 32x32 score blocks.
__host__ __device__ inline unsigned sage_v_position(unsigned j) {
    unsigned mb = j / 32, j32 = j % 32, hf = (j32 % 8) / 4;
    unsigned r = (j32 / 8) * 4 + j32 % 4;
    return hf * 32 + mb * 16 + r;
}
