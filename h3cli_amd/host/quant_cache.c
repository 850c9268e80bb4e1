/* Metadata-keyed packed-weight cache restated from the reference's
 * src/weights/quant_cache.c:13-127: the same key, artifact name, 128-byte
 * H3QMT002 header, validation rules and error texts, so that artifacts written
 * by either build are accepted by the other. Weak: a host application that
 * links its own src/weights/quant_cache.c keeps its definitions. */
#define _GNU_SOURCE
#include "h3_quant_cache.h"
#include "h3_quant.h"
#include "sha256.h"
#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/file.h>
#include <unistd.h>

#define WEAK __attribute__((weak))

static int fail(char *error, size_t size, const char *message, const char *path) {
    if (error && size) snprintf(error, size, "%s: %s", message, path ? path : strerror(errno));
    return 0;
}

static void le(unsigned char *p, uint64_t v, unsigned n) {
    for (unsigned i = 0; i < n; i++) p[i] = (unsigned char)(v >> (8 * i));
}

/* Same regular file, unmodified: device, inode, size, mtime and ctime. */
static int same_file(const struct stat *a, const struct stat *b) {
    return S_ISREG(b->st_mode) && a->st_dev == b->st_dev && a->st_ino == b->st_ino && a->st_size == b->st_size &&
           a->st_mtim.tv_sec == b->st_mtim.tv_sec && a->st_mtim.tv_nsec == b->st_mtim.tv_nsec &&
           a->st_ctim.tv_sec == b->st_ctim.tv_sec && a->st_ctim.tv_nsec == b->st_ctim.tv_nsec;
}

static int transfer(int fd, void *data, size_t bytes, int writing) {
    unsigned char *p = (unsigned char *)data;
    while (bytes) {
        ssize_t n = writing ? write(fd, p, bytes) : read(fd, p, bytes);
        if (n < 0 && errno == EINTR) continue;
        if (n <= 0) return 0;
        p += n;
        bytes -= (size_t)n;
    }
    return 1;
}

/* Header: magic, cache and recipe versions, mode, shape, sizes, key, offset;
 * every other byte zero. */
static void encode_header(const h3_quant_cache *c, unsigned char h[H3_QUANT_CACHE_HEADER]) {
    memset(h, 0, H3_QUANT_CACHE_HEADER);
    memcpy(h, "H3QMT002", 8);
    le(h + 8, H3_QUANT_CACHE_VERSION, 4);
    le(h + 12, H3_QUANT_VERSION, 4);
    le(h + 16, c->mode, 4);
    le(h + 20, c->rows, 4);
    le(h + 24, c->columns, 4);
    le(h + 32, c->bytes, 8);
    le(h + 40, c->scale, 8);
    le(h + 48, c->global, 8);
    memcpy(h + 56, c->key, 32);
    le(h + 88, c->offset, 8);
}

WEAK int h3_quant_cache_unchanged(const h3_quant_cache *c, char *error, size_t size) {
    struct stat now;
    if (stat(c->source, &now) != 0 || !same_file(&c->stamp, &now))
        return fail(error, size, "quantization source changed during loading/preparation; retry", c->source);
    return 1;
}

WEAK void h3_quant_cache_close(h3_quant_cache *c) {
    if (!c) return;
    if (c->lock >= 0) {
        flock(c->lock, LOCK_UN);
        close(c->lock);
    }
    free(c->source);
    free(c->artifact);
    free(c);
}

WEAK h3_quant_cache *h3_quant_cache_open(const char *directory, const char *source, uint64_t offset, unsigned rows,
                                         unsigned columns, int mode, uint64_t bytes, uint64_t scale, uint64_t global,
                                         char *error, size_t size) {
    h3_quant_cache *c = (h3_quant_cache *)calloc(1, sizeof(*c));
    if (!c) {
        fail(error, size, "cannot allocate quantization metadata", NULL);
        return NULL;
    }
    c->lock = -1;
    const int shape_ok = rows && columns && rows % 128 == 0 && columns % 128 == 0 &&
                         (uint64_t)rows * columns <= UINT32_MAX;
    const int sizes_ok = bytes && bytes <= SIZE_MAX - H3_QUANT_CACHE_HEADER && scale < global && global <= bytes &&
                         bytes - global >= 16;
    if (!directory || !*directory || !source || !shape_ok || (mode != H3_QUANT_FP8 && mode != H3_QUANT_NVFP4) ||
        !sizes_ok) {
        fail(error, size, "invalid quantization metadata arguments", source);
        h3_quant_cache_close(c);
        return NULL;
    }
    c->source = realpath(source, NULL);
    if (!c->source || stat(c->source, &c->stamp) != 0 || !S_ISREG(c->stamp.st_mode) || c->stamp.st_size < 0 ||
        offset > (uint64_t)c->stamp.st_size || (uint64_t)rows * columns * 2 > (uint64_t)c->stamp.st_size - offset) {
        fail(error, size, "invalid quantized source range", source);
        h3_quant_cache_close(c);
        return NULL;
    }
    c->offset = offset; c->rows = rows; c->columns = columns; c->mode = (unsigned)mode;
    c->bytes = bytes; c->scale = scale; c->global = global;

    /* Key: SHA-256 of 14 little-endian u64 identity values (112 bytes) and the
     * canonical path with its terminating NUL. */
    const uint64_t identity[14] = {H3_QUANT_CACHE_VERSION, H3_QUANT_VERSION, (uint64_t)mode, rows, columns, offset,
                                   (uint64_t)c->stamp.st_dev, (uint64_t)c->stamp.st_ino, (uint64_t)c->stamp.st_size,
                                   (uint64_t)c->stamp.st_mtim.tv_sec, (uint64_t)c->stamp.st_mtim.tv_nsec,
                                   (uint64_t)c->stamp.st_ctim.tv_sec, (uint64_t)c->stamp.st_ctim.tv_nsec, bytes};
    unsigned char record[112];
    for (unsigned i = 0; i < 14; i++) le(record + 8 * i, identity[i], 8);
    h3hip_sha256 hash;
    h3hip_sha256_init(&hash);
    h3hip_sha256_update(&hash, record, sizeof(record));
    h3hip_sha256_update(&hash, c->source, strlen(c->source) + 1);
    h3hip_sha256_final(&hash, c->key);
    char hex[65];
    for (unsigned i = 0; i < 32; i++) snprintf(hex + 2 * i, 3, "%02x", c->key[i]);
    char *lock_path = NULL;
    if (asprintf(&c->artifact, "%s/m%d-%s-%ux%u-%s.h3q", directory, H3_QUANT_CACHE_VERSION, h3_quant_name(mode), rows,
                 columns, hex) < 0)
        c->artifact = NULL;
    if (!c->artifact || asprintf(&lock_path, "%s.lock", c->artifact) < 0) {
        fail(error, size, "cannot allocate quantization cache path", source);
        h3_quant_cache_close(c);
        return NULL;
    }
    c->lock = open(lock_path, O_CREAT | O_RDWR, 0600);
    free(lock_path);
    if (c->lock < 0 || flock(c->lock, LOCK_EX) != 0) {
        fail(error, size, "cannot lock quantization artifact", c->artifact);
        h3_quant_cache_close(c);
        return NULL;
    }
    if (!h3_quant_cache_unchanged(c, error, size)) {
        h3_quant_cache_close(c);
        return NULL;
    }
    return c;
}

WEAK int h3_quant_cache_read(h3_quant_cache *c, void *payload, char *error, size_t size) {
    int fd = open(c->artifact, O_RDONLY);
    if (fd < 0) {
        if (errno == ENOENT) return h3_quant_cache_unchanged(c, error, size) ? 0 : -1;
        fail(error, size, "cannot read quantization artifact", c->artifact);
        return -1;
    }
    unsigned char want[H3_QUANT_CACHE_HEADER], got[H3_QUANT_CACHE_HEADER];
    encode_header(c, want);
    struct stat before, after;
    int ok = fstat(fd, &before) == 0 && S_ISREG(before.st_mode) && before.st_size >= 0 &&
             (uint64_t)before.st_size == H3_QUANT_CACHE_HEADER + c->bytes && transfer(fd, got, sizeof(got), 0) &&
             memcmp(got, want, sizeof(got)) == 0 && transfer(fd, payload, (size_t)c->bytes, 0) &&
             fstat(fd, &after) == 0 && same_file(&before, &after);
    close(fd);
    if (!ok) {
        fail(error, size, "corrupt/incompatible metadata quantization artifact; remove it and prepare again",
             c->artifact);
        return -1;
    }
    return h3_quant_cache_unchanged(c, error, size) ? 1 : -1;
}

/* Written to a temporary file beside the artifact, synced, and renamed over it
 * only if the source is still unchanged. */
WEAK int h3_quant_cache_write(h3_quant_cache *c, const void *payload, char *error, size_t size) {
    if (!h3_quant_cache_unchanged(c, error, size)) return 0;
    char *staging = NULL;
    if (asprintf(&staging, "%s.tmp.XXXXXX", c->artifact) < 0)
        return fail(error, size, "cannot allocate quantization staging path", c->artifact);
    unsigned char h[H3_QUANT_CACHE_HEADER];
    encode_header(c, h);
    int fd = mkstemp(staging), ok = fd >= 0;
    if (ok) {
        ok = transfer(fd, h, sizeof(h), 1) && transfer(fd, (void *)payload, (size_t)c->bytes, 1) && fsync(fd) == 0;
        if (close(fd) != 0) ok = 0;
    }
    if (ok) ok = h3_quant_cache_unchanged(c, error, size);
    if (ok) ok = rename(staging, c->artifact) == 0;
    if (!ok) {
        unlink(staging);
        fail(error, size, "cannot publish quantization artifact (source changed or I/O failure)", c->artifact);
    }
    free(staging);
    return ok;
}
