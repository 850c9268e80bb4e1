/* h3_safetensors.h — safetensors checkpoint reader, the reference's
 * src/weights/safetensors.h API (types and names as safetensors.h:8-61; the
 * Metal zero-copy planner and the component inventory are not on this path and
 * are not provided). Host C in libh3hip.so. */
#ifndef H3_SAFETENSORS_H
#define H3_SAFETENSORS_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* safetensors.h:8-23 */
typedef enum {
    H3_DTYPE_UNKNOWN = 0,
    H3_DTYPE_BOOL,
    H3_DTYPE_I8,
    H3_DTYPE_U8,
    H3_DTYPE_I16,
    H3_DTYPE_U16,
    H3_DTYPE_F16,
    H3_DTYPE_BF16,
    H3_DTYPE_I32,
    H3_DTYPE_U32,
    H3_DTYPE_F32,
    H3_DTYPE_I64,
    H3_DTYPE_U64,
    H3_DTYPE_F64
} h3_dtype;

/* safetensors.h:25-33. data_begin/data_end are relative to the payload (the
 * byte after the header); file_offset is absolute. */
typedef struct {
    char *name;
    h3_dtype dtype;
    int ndim;
    uint64_t shape[8];
    uint64_t data_begin;
    uint64_t data_end;
    uint64_t file_offset;
} h3_st_tensor;

/* safetensors.h:35-44 */
typedef struct {
    char *path;
    uint64_t file_size;
    uint64_t header_size;
    h3_st_tensor *tensors;
    size_t tensor_count;
    char **metadata_keys;
    char **metadata_values;
    size_t metadata_count;
} h3_st_header;

/* safetensors.h:48: offset + bytes lies inside a file of file_size bytes and
 * fits off_t. */
int h3_st_file_range(uint64_t offset, uint64_t bytes, uint64_t file_size);
/* safetensors.h:53-54. Reads and validates the header: the 8-byte little-endian
 * length (1 .. 256 MiB), a JSON object starting at the first byte, string keys
 * (valid UTF-8, escapes, no NUL), an optional flat string "__metadata__" map,
 * tensor entries {dtype, shape (rank <= 8), data_offsets} each field once,
 * shape x dtype size == the byte range, unique names, and ranges that tile the
 * payload exactly (no gap, overlap or trailing bytes). Errors name the rule in
 * `error`; on failure the header is left empty. */
int h3_st_read_header(const char *path, h3_st_header *header, char *error, size_t error_size);
void h3_st_free_header(h3_st_header *header);                                   /* :55 */
const h3_st_tensor *h3_st_find(const h3_st_header *header, const char *name);   /* :56 */
uint64_t h3_st_tensor_elements(const h3_st_tensor *tensor);                      /* :57 */
/* safetensors.h:58-59: reads exactly the tensor's bytes (bytes must equal its
 * byte range) with pread. */
int h3_st_read_data(const h3_st_header *header, const h3_st_tensor *tensor, void *data, size_t bytes,
                    char *error, size_t error_size);
size_t h3_dtype_size(h3_dtype dtype);                                            /* :60 */
const char *h3_dtype_name(h3_dtype dtype);                                       /* :61 */

#ifdef __cplusplus
}
#endif
#endif
