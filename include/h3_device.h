/* h3_device.h — process-wide device selection and query of the reference's
 * src/device.h:7-13, implemented for HIP (the reference's CUDA version is
 * src/cuda/cuda_probe.c). h3_device_info has the reference's field layout
 * (src/h3.h:282-298); the cuda_* fields carry the HIP equivalents (gfx major /
 * minor, HIP driver / runtime versions) and backend is "hip". */
#ifndef H3_DEVICE_H
#define H3_DEVICE_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
typedef struct {
    char name[128];
    char architecture[128];          /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    uint64_t physical_memory;        /* host RAM */
    uint64_t recommended_working_set;
    uint64_t max_buffer_length;
    int apple_gpu_family;
    int metal4;
    int unified_memory;
    char backend[16];
    int device_index;
    int cuda_compute_major, cuda_compute_minor;
    int cuda_driver_version, cuda_runtime_version;
    uint64_t device_memory, free_device_memory;
    int multiprocessor_count;
    uint8_t cuda_uuid[16];
} h3_device_info;
/* device.h:8. Selects H3_CUDA_DEVICE (default 0); fails unless it is gfx950. */
int h3_device_query(h3_device_info *info, char *error, size_t error_size);
/* device.h:9-10. Validates and exports H3_CUDA_DEVICE / H3_CUDA_WEIGHT_MODE. */
int h3_device_configure(const char *index, const char *weight_mode, char *error, size_t error_size);
/* device.h:13. Whether `next_component_bytes` fits beside a 10% reserve. */
int h3_device_memory_fits(uint64_t next_component_bytes);
#ifdef __cplusplus
}
#endif
#endif
