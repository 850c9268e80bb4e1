/* h3_quant_cache.h — metadata-keyed packed-weight cache, the reference's
 * src/weights/quant_cache.h:1-37 API and artifact format (H3QMT002). The key
 * is a SHA-256 of the source file's identity (canonical path, device, inode,
 * size, mtime, ctime, offset, shape, mode, versions, packed size); no tensor
 * bytes are hashed. libh3hip.so defines the functions weak (host/quant_cache.c). */
#ifndef H3_QUANT_CACHE_H
#define H3_QUANT_CACHE_H
#include <stddef.h>
#include <stdint.h>
#include <sys/stat.h>
#ifdef __cplusplus
extern "C" {
#endif

#define H3_QUANT_CACHE_VERSION 2      /* quant_cache.h:11 */
#define H3_QUANT_CACHE_HEADER 128     /* quant_cache.h:12 */
typedef struct {                      /* quant_cache.h:13-21, same members and order */
    char *source, *artifact;
    struct stat stamp;
    uint64_t offset, bytes, scale, global;
    unsigned mode, rows, columns;
    unsigned char key[32];
    int lock;
} h3_quant_cache;

/* Takes <artifact>.lock exclusively until close. rows, columns: multiples of
 * 128 with rows * columns <= 2^32 - 1; mode 1 or 2; scale < global <= bytes - 16.
 * The caller creates the directory. */
h3_quant_cache *h3_quant_cache_open(const char *directory, const char *source, uint64_t offset, unsigned rows,
                                    unsigned columns, int mode, uint64_t bytes, uint64_t scale, uint64_t global,
                                    char *error, size_t size);
/* 1 hit (payload filled, cache->bytes), 0 absent, -1 malformed or error. */
int h3_quant_cache_read(h3_quant_cache *cache, void *payload, char *error, size_t size);
int h3_quant_cache_write(h3_quant_cache *cache, const void *payload, char *error, size_t size);
int h3_quant_cache_unchanged(const h3_quant_cache *cache, char *error, size_t size);
void h3_quant_cache_close(h3_quant_cache *cache);

#ifdef __cplusplus
}
#endif
#endif
