/* h3_residency.h — the weight residency planner of the reference
 * (src/weights/residency.h:8-27): same types, names and meaning. libh3hip.so
 * defines the functions weak (the host application's own definitions win when
 * linked), and h3_gpu_plan_bf16_weights calls them with the device's free bytes. */
#ifndef H3_RESIDENCY_H
#define H3_RESIDENCY_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
enum { H3_WEIGHTS_AUTO, H3_WEIGHTS_RESIDENT, H3_WEIGHTS_STREAM };  /* residency.h:8 */
typedef struct {                                                      /* residency.h:9-14 */
    int mode;
    int max_resident;           /* -1: uncapped */
    uint64_t capacity_limit;    /* 0: uncapped */
    uint64_t allocation_limit;
} h3_weight_options;
typedef struct {                                                      /* residency.h:15-22 */
    h3_weight_options options;
    uint64_t active_mask, resident_mask;
    uint64_t free_bytes, live_bytes, reserve_bytes, future_bytes;
    uint64_t block_bytes, resident_bytes, slot_bytes;
    unsigned active_count, resident_count;
    int effective_mode;         /* AUTO here means partial residency */
} h3_weight_plan;
const char *h3_weight_mode_name(int mode);                                             /* residency.h:23 */
int h3_weight_options_read(h3_weight_options *out, int force_stream, char *error, size_t size);  /* :24 */
int h3_weight_options_equal(const h3_weight_options *a, const h3_weight_options *b);  /* :25 */
/* residency.h:26-28. Resident if every active block fits beside future bytes and
 * the reserve; otherwise two streaming slots plus as many resident blocks (lowest
 * index first) as fit. */
int h3_weight_plan_build(h3_weight_plan *out, h3_weight_options options, uint64_t active_mask, uint64_t block_bytes,
                         uint64_t available, uint64_t live, uint64_t future, uint64_t reserve, char *error, size_t size);
int h3_weight_retry_cap(unsigned count);                                              /* residency.h:30 */
/* residency.h:31-33: packed projection descriptor sizes (payload, 256-aligned
 * scale plane at *scale, 16-byte global slot at *global; *bytes in total).
 * mode 1 FP8, 2 NVFP4. */
int h3_weight_packed_size(uint32_t rows, uint32_t columns, int mode, uint64_t *scale, uint64_t *global,
                          uint64_t *bytes);
#ifdef __cplusplus
}
#endif
#endif
