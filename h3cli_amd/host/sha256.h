/* SHA-256 (FIPS 180-4) for the quantization caches: internal to libh3hip.so
 * (hidden symbols), so it never collides with a host's own digest code. */
#ifndef H3HIP_SHA256_H
#define H3HIP_SHA256_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
typedef struct {
    uint32_t h[8];
    uint64_t length;          /* bytes absorbed */
    uint8_t block[64];
} h3hip_sha256;
__attribute__((visibility("hidden"))) void h3hip_sha256_init(h3hip_sha256 *s);
__attribute__((visibility("hidden"))) void h3hip_sha256_update(h3hip_sha256 *s, const void *data, size_t bytes);
__attribute__((visibility("hidden"))) void h3hip_sha256_final(h3hip_sha256 *s, uint8_t digest[32]);
#ifdef __cplusplus
}
#endif
#endif
