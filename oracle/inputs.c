/* CPU oracle — TEST INFRASTRUCTURE ONLY (see oracle.h). The reference's
 * deterministic test-input generators, restated so parity tests can reuse the
 * reference's own input patterns. */
#include "oracle.h"

/* tests/cuda_attention.c:14-18: xorshift32 (13, 17, 5) from *seed, value
 * (seed % 4097 - 2048) / 1024 rounded to BF16 (RNE). Advances *seed. */
void oracle_xorshift_bf16(uint16_t *out, size_t count, uint32_t *seed) {
    uint32_t s = *seed;
    for (size_t i = 0; i < count; i++) {
        s ^= s << 13; s ^= s >> 17; s ^= s << 5;
        float x = (float)((int)(s % 4097u) - 2048) / 1024.0f;
        out[i] = oracle_f32_to_bf16(x);
    }
    *seed = s;
}

/* tests/attention_native.c:20,56: xorshift32 from 0x5a317d6b, value
 * (state % 65537 - 32768) / 16384 rounded to BF16. Advances *state. */
void oracle_xorshift_native_bf16(uint16_t *out, size_t count, uint32_t *state) {
    uint32_t s = *state;
    for (size_t i = 0; i < count; i++) {
        s ^= s << 13; s ^= s >> 17; s ^= s << 5;
        float x = (float)((int)(s % 65537u) - 32768) / 16384.0f;
        out[i] = oracle_f32_to_bf16(x);
    }
    *state = s;
}
