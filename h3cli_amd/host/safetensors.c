/* safetensors reader (include/h3_safetensors.h), the reference's
 * src/weights/safetensors.c contract: the same accepted files, the same
 * validation rules and the same error texts (callers match on them), written
 * as a small recursive-descent parser over the header bytes.
 *
 * File layout (the safetensors format): u64 little-endian header length N,
 * N bytes of JSON, then the payload. The JSON object maps tensor names to
 * {"dtype", "shape", "data_offsets": [begin, end]} (offsets relative to the
 * payload) plus an optional "__metadata__" string map. */
#define _GNU_SOURCE
#include "h3_safetensors.h"
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#define MAX_HEADER_BYTES (256u * 1024u * 1024u)   /* safetensors.c:13 */

static const char *const DTYPE_NAMES[] = {"UNKNOWN", "BOOL", "I8", "U8", "I16", "U16", "F16",
                                          "BF16", "I32", "U32", "F32", "I64", "U64", "F64"};
static const unsigned char DTYPE_BYTES[] = {0, 1, 1, 1, 2, 2, 2, 2, 4, 4, 4, 8, 8, 8};

size_t h3_dtype_size(h3_dtype dtype) {
    return (unsigned)dtype < sizeof(DTYPE_BYTES) ? DTYPE_BYTES[dtype] : 0;
}

const char *h3_dtype_name(h3_dtype dtype) {
    return (unsigned)dtype < sizeof(DTYPE_BYTES) ? DTYPE_NAMES[dtype] : "UNKNOWN";
}

int h3_st_file_range(uint64_t offset, uint64_t bytes, uint64_t file_size) {
    return offset <= (uint64_t)INT64_MAX && bytes <= (uint64_t)INT64_MAX - offset && offset <= file_size &&
           bytes <= file_size - offset;
}

/* ---- parser state: the header bytes [p, end) and where errors go ---- */
typedef struct {
    const unsigned char *p, *end;
    char *error;
    size_t error_size;
} parser;

static int fail(parser *s, const char *message) {
    if (s->error && s->error_size) snprintf(s->error, s->error_size, "%s", message);
    return 0;
}

static void report(char *error, size_t size, const char *fmt, ...) {
    if (!error || !size) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(error, size, fmt, ap);
    va_end(ap);
}

static void skip_space(parser *s) {
    while (s->p < s->end && (*s->p == ' ' || *s->p == '\t' || *s->p == '\n' || *s->p == '\r')) s->p++;
}

/* Next non-space byte, or -1 at the end (not consumed). */
static int peek(parser *s) {
    skip_space(s);
    return s->p < s->end ? *s->p : -1;
}

static int expect(parser *s, char c) {
    if (peek(s) != (unsigned char)c) return fail(s, "malformed safetensors JSON header");
    s->p++;
    return 1;
}

static int hex4(const unsigned char *at) {
    int v = 0;
    for (int i = 0; i < 4; i++) {
        int c = at[i], d = c >= '0' && c <= '9' ? c - '0' : c >= 'a' && c <= 'f' ? c - 'a' + 10
                          : c >= 'A' && c <= 'F' ? c - 'A' + 10 : -1;
        if (d < 0) return -1;
        v = v * 16 + d;
    }
    return v;
}

static size_t put_utf8(char *out, unsigned cp) {
    if (cp < 0x80) { out[0] = (char)cp; return 1; }
    if (cp < 0x800) { out[0] = (char)(0xc0 | cp >> 6); out[1] = (char)(0x80 | (cp & 0x3f)); return 2; }
    if (cp < 0x10000) {
        out[0] = (char)(0xe0 | cp >> 12); out[1] = (char)(0x80 | ((cp >> 6) & 0x3f));
        out[2] = (char)(0x80 | (cp & 0x3f));
        return 3;
    }
    out[0] = (char)(0xf0 | cp >> 18); out[1] = (char)(0x80 | ((cp >> 12) & 0x3f));
    out[2] = (char)(0x80 | ((cp >> 6) & 0x3f)); out[3] = (char)(0x80 | (cp & 0x3f));
    return 4;
}

/* Length of the well-formed UTF-8 sequence that starts with lead byte c at
 * s->p - 1 (RFC 3629 table), or 0 if it is malformed. */
static int utf8_tail(const parser *s, unsigned c) {
    int extra = c >= 0xc2 && c <= 0xdf ? 1 : c >= 0xe0 && c <= 0xef ? 2 : c >= 0xf0 && c <= 0xf4 ? 3 : -1;
    if (extra < 0 || s->end - s->p < extra) return -1;
    unsigned first = s->p[0];
    if ((c == 0xe0 && first < 0xa0) || (c == 0xed && first >= 0xa0) || (c == 0xf0 && first < 0x90) ||
        (c == 0xf4 && first >= 0x90))
        return -1;
    for (int i = 0; i < extra; i++)
        if ((s->p[i] & 0xc0) != 0x80) return -1;
    return extra;
}

/* A JSON string as a NUL-terminated UTF-8 C string (malloc'd), or NULL. */
static char *read_string(parser *s) {
    if (peek(s) != '"') { fail(s, "expected JSON string"); return NULL; }
    s->p++;
    char *out = malloc((size_t)(s->end - s->p) + 1);   /* decoding never grows the text */
    if (!out) { fail(s, "out of memory parsing safetensors header"); return NULL; }
    size_t n = 0;
    for (;;) {
        if (s->p >= s->end) goto bad;
        unsigned c = *s->p++;
        if (c == '"') break;
        if (c < 0x20) goto bad;
        if (c != '\\') {
            out[n++] = (char)c;
            if (c >= 0x80) {
                int extra = utf8_tail(s, c);
                if (extra < 0) goto bad;
                memcpy(out + n, s->p, (size_t)extra);
                n += (size_t)extra;
                s->p += extra;
            }
            continue;
        }
        if (s->p >= s->end) goto bad;
        c = *s->p++;
        const char *simple = strchr("\"\\/bfnrt", (int)c);
        if (c && simple) {
            static const char decoded[] = "\"\\/\b\f\n\r\t";
            out[n++] = decoded[simple - "\"\\/bfnrt"];
            continue;
        }
        if (c != 'u' || s->end - s->p < 4) goto bad;
        int cp = hex4(s->p);
        if (cp < 0) goto bad;
        s->p += 4;
        if (cp >= 0xd800 && cp <= 0xdbff) {          /* high surrogate: a low one must follow */
            if (s->end - s->p < 6 || s->p[0] != '\\' || s->p[1] != 'u') goto bad;
            int low = hex4(s->p + 2);
            if (low < 0xdc00 || low > 0xdfff) goto bad;
            s->p += 6;
            cp = 0x10000 + ((cp - 0xd800) << 10) + (low - 0xdc00);
        } else if (cp >= 0xdc00 && cp <= 0xdfff) {
            goto bad;
        }
        if (!cp) goto bad;                           /* names are C strings */
        n += put_utf8(out + n, (unsigned)cp);
    }
    out[n] = '\0';
    char *shrunk = realloc(out, n + 1);
    return shrunk ? shrunk : out;
bad:
    free(out);
    fail(s, "malformed JSON string escape");
    return NULL;
}

static int read_u64(parser *s, uint64_t *value) {
    int c = peek(s);
    if (c < '0' || c > '9') return fail(s, "expected unsigned JSON integer");
    if (c == '0' && s->p + 1 < s->end && s->p[1] >= '0' && s->p[1] <= '9')
        return fail(s, "leading zero in JSON integer");
    uint64_t v = 0;
    while (s->p < s->end && *s->p >= '0' && *s->p <= '9') {
        unsigned d = (unsigned)(*s->p - '0');
        if (v > (UINT64_MAX - d) / 10) return fail(s, "integer overflow in safetensors header");
        v = v * 10 + d;
        s->p++;
    }
    *value = v;
    return 1;
}

static h3_dtype dtype_of(const char *name) {
    for (unsigned d = 1; d < sizeof(DTYPE_BYTES); d++)
        if (!strcmp(name, DTYPE_NAMES[d])) return (h3_dtype)d;
    return H3_DTYPE_UNKNOWN;
}

static int read_shape(parser *s, h3_st_tensor *t) {
    if (!expect(s, '[')) return 0;
    t->ndim = 0;
    if (peek(s) == ']') { s->p++; return 1; }
    for (;;) {
        if (t->ndim >= 8) return fail(s, "tensor rank exceeds 8");
        if (!read_u64(s, &t->shape[t->ndim])) return 0;
        t->ndim++;
        int c = peek(s);
        if (c < 0) return fail(s, "unterminated shape");
        s->p++;
        if (c == ']') return 1;
        if (c != ',') return fail(s, "expected shape comma");
    }
}

/* {"dtype": ..., "shape": [...], "data_offsets": [b, e]}, any order, each once. */
static int read_tensor(parser *s, h3_st_tensor *t) {
    if (!expect(s, '{')) return 0;
    int have = 0;                                   /* bits: 1 dtype, 2 shape, 4 offsets */
    while (peek(s) != '}') {
        char *key = read_string(s);
        if (!key || !expect(s, ':')) { free(key); return 0; }
        int bit = !strcmp(key, "dtype") ? 1 : !strcmp(key, "shape") ? 2 : !strcmp(key, "data_offsets") ? 4 : 0;
        free(key);
        if (!bit) return fail(s, "unknown tensor descriptor field");
        if (have & bit)
            return fail(s, bit == 1 ? "duplicate dtype" : bit == 2 ? "duplicate shape" : "duplicate data_offsets");
        if (bit == 1) {
            char *name = read_string(s);
            if (!name) return 0;
            t->dtype = dtype_of(name);
            free(name);
            if (t->dtype == H3_DTYPE_UNKNOWN) return fail(s, "unknown tensor dtype");
        } else if (bit == 2) {
            if (!read_shape(s, t)) return 0;
        } else if (!expect(s, '[') || !read_u64(s, &t->data_begin) || !expect(s, ',') ||
                   !read_u64(s, &t->data_end) || !expect(s, ']')) {
            return 0;
        }
        have |= bit;
        int c = peek(s);
        if (c < 0) return fail(s, "unterminated tensor entry");
        if (c == '}') break;
        s->p++;
        if (c != ',') return fail(s, "expected tensor comma");
        if (peek(s) == '}') return fail(s, "trailing tensor comma");
    }
    s->p++;
    if (have != 7) return fail(s, "incomplete tensor descriptor");
    return 1;
}

/* Byte range inside the file and equal to shape x dtype size; sets file_offset. */
static int check_tensor(parser *s, h3_st_tensor *t, uint64_t payload, uint64_t file_size) {
    if (payload > file_size || payload > (uint64_t)INT64_MAX || t->data_end < t->data_begin ||
        t->data_end > file_size - payload)
        return fail(s, "tensor data offsets exceed file");
    uint64_t elements = 1;
    for (int d = 0; d < t->ndim; d++) {
        if (t->shape[d] && elements > UINT64_MAX / t->shape[d]) return fail(s, "tensor element count overflow");
        elements *= t->shape[d];
    }
    uint64_t item = h3_dtype_size(t->dtype);
    if (item && elements > UINT64_MAX / item) return fail(s, "tensor byte count overflow");
    if (elements * item != t->data_end - t->data_begin) return fail(s, "tensor shape does not match byte offsets");
    t->file_offset = payload + t->data_begin;
    return 1;
}

/* Flat {"key": "value", ...}; keys unique. */
static int read_metadata(parser *s, h3_st_header *h) {
    if (!expect(s, '{')) return 0;
    if (peek(s) == '}') { s->p++; return 1; }
    size_t cap = 0;
    for (;;) {
        char *key = read_string(s);
        if (!key) return 0;
        for (size_t i = 0; i < h->metadata_count; i++)
            if (!strcmp(h->metadata_keys[i], key)) { free(key); return fail(s, "duplicate metadata key"); }
        if (h->metadata_count == cap) {
            size_t next = cap ? 2 * cap : 8;
            char **k = realloc(h->metadata_keys, next * sizeof(*k));
            if (k) h->metadata_keys = k;
            char **v = k ? realloc(h->metadata_values, next * sizeof(*v)) : NULL;
            if (v) h->metadata_values = v;
            if (!k || !v) { free(key); return fail(s, "out of memory"); }
            cap = next;
        }
        char *value = NULL;
        if (!expect(s, ':') || !(value = read_string(s))) { free(key); return 0; }
        h->metadata_keys[h->metadata_count] = key;
        h->metadata_values[h->metadata_count++] = value;
        if (peek(s) == '}') { s->p++; return 1; }
        if (!expect(s, ',')) return 0;
    }
}

static int by_name(const void *a, const void *b) {
    return strcmp((*(const h3_st_tensor *const *)a)->name, (*(const h3_st_tensor *const *)b)->name);
}

static int by_range(const void *a, const void *b) {
    const h3_st_tensor *x = *(const h3_st_tensor *const *)a, *y = *(const h3_st_tensor *const *)b;
    if (x->data_begin != y->data_begin) return x->data_begin < y->data_begin ? -1 : 1;
    return (x->data_end > y->data_end) - (x->data_end < y->data_end);
}

/* Unique names; ranges that tile [0, payload) with no gap or overlap. */
static int check_index(parser *s, const h3_st_header *h) {
    size_t n = h->tensor_count;
    const h3_st_tensor **v = malloc((n ? n : 1) * sizeof(*v));
    if (!v) return fail(s, "out of memory validating tensors");
    for (size_t i = 0; i < n; i++) v[i] = &h->tensors[i];
    int ok = 1;
    qsort(v, n, sizeof(*v), by_name);
    for (size_t i = 1; ok && i < n; i++)
        if (!strcmp(v[i - 1]->name, v[i]->name)) ok = fail(s, "duplicate tensor name");
    uint64_t covered = 0;
    if (ok) {
        qsort(v, n, sizeof(*v), by_range);
        for (size_t i = 0; ok && i < n; i++) {
            if (v[i]->data_begin != covered) ok = fail(s, "overlapping tensor ranges or unindexed payload gap");
            covered = v[i]->data_end;
        }
    }
    free(v);
    if (ok && covered != h->file_size - 8 - h->header_size)
        ok = fail(s, "unindexed trailing safetensors payload");
    return ok;
}

static int push_tensor(parser *s, h3_st_header *h, size_t *cap, const h3_st_tensor *t) {
    if (h->tensor_count == *cap) {
        size_t next = *cap ? 2 * *cap : 64;
        h3_st_tensor *grown = realloc(h->tensors, next * sizeof(*grown));
        if (!grown) return fail(s, "out of memory indexing tensors");
        h->tensors = grown;
        *cap = next;
    }
    h->tensors[h->tensor_count++] = *t;
    return 1;
}

static int parse(parser *s, h3_st_header *h) {
    if (s->p >= s->end || *s->p != '{') return fail(s, "safetensors header must begin with an object");
    s->p++;
    const uint64_t payload = 8 + h->header_size;
    size_t cap = 0;
    int have_metadata = 0;
    if (peek(s) == '}') {
        s->p++;
    } else {
        for (;;) {
            char *name = read_string(s);
            if (!name || !expect(s, ':')) { free(name); return 0; }
            if (!strcmp(name, "__metadata__")) {
                free(name);
                if (have_metadata++) return fail(s, "duplicate metadata entry");
                if (!read_metadata(s, h)) return 0;
            } else {
                h3_st_tensor t;
                memset(&t, 0, sizeof(t));
                t.name = name;
                if (!read_tensor(s, &t) || !check_tensor(s, &t, payload, h->file_size) || !push_tensor(s, h, &cap, &t)) {
                    free(name);
                    return 0;
                }
            }
            int c = peek(s);
            if (c < 0) return fail(s, "unterminated safetensors object");
            s->p++;
            if (c == '}') break;
            if (c != ',') return fail(s, "expected top-level comma");
        }
    }
    if (peek(s) >= 0) return fail(s, "trailing data in safetensors header");
    return check_index(s, h);
}

static uint64_t le64(const unsigned char b[8]) {
    uint64_t v = 0;
    for (int i = 7; i >= 0; i--) v = v << 8 | b[i];
    return v;
}

int h3_st_read_header(const char *path, h3_st_header *header, char *error, size_t error_size) {
    if (!path || !header) return 0;
    memset(header, 0, sizeof(*header));
    if (error && error_size) error[0] = '\0';
    int fd = open(path, O_RDONLY);
    if (fd < 0) { report(error, error_size, "%s: %s", path, strerror(errno)); return 0; }
    struct stat st;
    unsigned char prefix[8];
    if (fstat(fd, &st) || st.st_size < 8 || pread(fd, prefix, 8, 0) != 8) {
        report(error, error_size, "%s: invalid file", path);
        close(fd);
        return 0;
    }
    const uint64_t file_size = (uint64_t)st.st_size, header_size = le64(prefix);
    if (!header_size || header_size > MAX_HEADER_BYTES || !h3_st_file_range(8, header_size, file_size)) {
        report(error, error_size, "%s: invalid header size", path);
        close(fd);
        return 0;
    }
    unsigned char *json = malloc((size_t)header_size + 1);
    if (!json || pread(fd, json, (size_t)header_size, 8) != (ssize_t)header_size) {
        report(error, error_size, "%s: cannot read header", path);
        free(json);
        close(fd);
        return 0;
    }
    close(fd);
    header->path = strdup(path);
    header->file_size = file_size;
    header->header_size = header_size;
    if (!header->path) {
        free(json);
        report(error, error_size, "out of memory");
        return 0;
    }
    parser s = {json, json + header_size, error, error_size};
    int ok = parse(&s, header);
    free(json);
    if (!ok) h3_st_free_header(header);
    return ok;
}

void h3_st_free_header(h3_st_header *header) {
    if (!header) return;
    for (size_t i = 0; i < header->tensor_count; i++) free(header->tensors[i].name);
    for (size_t i = 0; i < header->metadata_count; i++) {
        free(header->metadata_keys[i]);
        free(header->metadata_values[i]);
    }
    free(header->metadata_keys);
    free(header->metadata_values);
    free(header->tensors);
    free(header->path);
    memset(header, 0, sizeof(*header));
}

const h3_st_tensor *h3_st_find(const h3_st_header *header, const char *name) {
    if (!header || !name) return NULL;
    for (size_t i = 0; i < header->tensor_count; i++)
        if (!strcmp(header->tensors[i].name, name)) return &header->tensors[i];
    return NULL;
}

uint64_t h3_st_tensor_elements(const h3_st_tensor *tensor) {
    if (!tensor) return 0;
    uint64_t n = 1;
    for (int d = 0; d < tensor->ndim; d++) {
        if (tensor->shape[d] && n > UINT64_MAX / tensor->shape[d]) return 0;
        n *= tensor->shape[d];
    }
    return n;
}

int h3_st_read_data(const h3_st_header *header, const h3_st_tensor *tensor, void *data, size_t bytes,
                    char *error, size_t error_size) {
    if (error && error_size) error[0] = '\0';
    if (!header || !header->path || !tensor || (!data && bytes)) {
        report(error, error_size, "invalid tensor read request");
        return 0;
    }
    if (tensor->data_end < tensor->data_begin || !h3_st_file_range(tensor->file_offset, bytes, header->file_size)) {
        report(error, error_size, "invalid tensor file range");
        return 0;
    }
    const uint64_t want = tensor->data_end - tensor->data_begin;
    const char *name = tensor->name ? tensor->name : "tensor";
    if (want != bytes) {
        report(error, error_size, "%s: expected %llu bytes, got %zu", name, (unsigned long long)want, bytes);
        return 0;
    }
    int fd = open(header->path, O_RDONLY);
    if (fd < 0) { report(error, error_size, "%s: %s", header->path, strerror(errno)); return 0; }
    struct stat st;
    if (fstat(fd, &st) || st.st_size < 0 || !h3_st_file_range(tensor->file_offset, bytes, (uint64_t)st.st_size)) {
        report(error, error_size, "%s: tensor range exceeds current file", header->path);
        close(fd);
        return 0;
    }
    for (size_t done = 0; done < bytes;) {
        size_t chunk = bytes - done < ((size_t)1 << 30) ? bytes - done : ((size_t)1 << 30);
        ssize_t got = pread(fd, (unsigned char *)data + done, chunk, (off_t)(tensor->file_offset + done));
        if (got < 0 && errno == EINTR) continue;
        if (got <= 0) {
            report(error, error_size, "%s: cannot read %s: %s", header->path, name,
                   got < 0 ? strerror(errno) : "unexpected end of file");
            close(fd);
            return 0;
        }
        done += (size_t)got;
    }
    close(fd);
    return 1;
}
