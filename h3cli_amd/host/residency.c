/* Weight residency planner restated from the reference's
 * src/weights/residency.c:7-80 (same decisions, same error texts), for
 * h3_gpu_plan_bf16_weights. Weak: a host application that links its own
 * src/weights/residency.c keeps its definitions. */
#include "h3_residency.h"
#include <errno.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define WEAK __attribute__((weak))

static int fail(char *error, size_t size, const char *text) {
    if (error && size) snprintf(error, size, "%s", text);
    return 0;
}
static int add_u64(uint64_t a, uint64_t b, uint64_t *out) {
    if (a > UINT64_MAX - b) return 0;
    *out = a + b;
    return 1;
}
static int mul_u64(uint64_t a, uint64_t b, uint64_t *out) {
    if (a && b > UINT64_MAX / a) return 0;
    *out = a * b;
    return 1;
}

WEAK const char *h3_weight_mode_name(int mode) {
    switch (mode) {
    case H3_WEIGHTS_RESIDENT: return "resident";
    case H3_WEIGHTS_STREAM: return "stream";
    default: return "auto";
    }
}

/* Optional decimal environment value; absent leaves *value unchanged. */
static int env_u64(const char *name, uint64_t *value, char *error, size_t size) {
    const char *text = getenv(name);
    if (!text) return 1;
    if (text[0] < '0' || text[0] > '9') return fail(error, size, "invalid CUDA weight test cap");
    char *end;
    errno = 0;
    unsigned long long v = strtoull(text, &end, 10);
    if (errno || *end) return fail(error, size, "invalid CUDA weight test cap");
    *value = v;
    return 1;
}

WEAK int h3_weight_options_read(h3_weight_options *out, int force_stream, char *error, size_t size) {
    memset(out, 0, sizeof(*out));
    out->max_resident = -1;
    const char *mode = getenv("H3_CUDA_WEIGHT_MODE");
    if (mode && strcmp(mode, "auto") != 0) {
        if (!strcmp(mode, "resident")) out->mode = H3_WEIGHTS_RESIDENT;
        else if (!strcmp(mode, "stream")) out->mode = H3_WEIGHTS_STREAM;
        else return fail(error, size, "CUDA weight mode must be auto, resident, or stream");
    }
    if (force_stream && out->mode == H3_WEIGHTS_RESIDENT)
        return fail(error, size, "--ssd-streaming conflicts with CUDA resident weight mode");
    if (force_stream) out->mode = H3_WEIGHTS_STREAM;
    uint64_t cap = 50;
    if (!env_u64("H3_TEST_CUDA_RESIDENT_BLOCKS", &cap, error, size) || cap > 50)
        return fail(error, size, "H3_TEST_CUDA_RESIDENT_BLOCKS must be 0..50");
    if (getenv("H3_TEST_CUDA_RESIDENT_BLOCKS")) out->max_resident = (int)cap;
    return env_u64("H3_TEST_CUDA_CAPACITY_BYTES", &out->capacity_limit, error, size) &&
           env_u64("H3_CUDA_TEST_MEMORY_BUDGET", &out->allocation_limit, error, size);
}

WEAK int h3_weight_options_equal(const h3_weight_options *a, const h3_weight_options *b) {
    return a->mode == b->mode && a->max_resident == b->max_resident && a->capacity_limit == b->capacity_limit &&
           a->allocation_limit == b->allocation_limit;
}

WEAK int h3_weight_retry_cap(unsigned count) { return count ? (int)((count - 1) / 2) : -1; }

WEAK int h3_weight_plan_build(h3_weight_plan *p, h3_weight_options o, uint64_t mask, uint64_t block,
                              uint64_t available, uint64_t live, uint64_t future, uint64_t reserve, char *error,
                              size_t size) {
    if (!p || !mask || (mask >> 50) || !block || o.mode < 0 || o.mode > 2 || o.max_resident < -1 || o.max_resident > 50)
        return fail(error, size, "invalid weight planner input");
    memset(p, 0, sizeof(*p));
    p->options = o;
    p->active_mask = mask;
    p->live_bytes = live;
    p->future_bytes = future;
    p->reserve_bytes = reserve;
    p->block_bytes = block;
    p->active_count = (unsigned)__builtin_popcountll(mask);
    if (o.capacity_limit) {
        uint64_t capped = o.capacity_limit > live ? o.capacity_limit - live : 0;
        if (capped < available) available = capped;
    }
    p->free_bytes = available;
    uint64_t fixed, all_blocks, two_slots;
    if (!add_u64(future, reserve, &fixed) || !mul_u64(block, p->active_count, &all_blocks) || !mul_u64(block, 2, &two_slots))
        return fail(error, size, "weight planner byte overflow");
    const uint64_t budget = available >= fixed ? available - fixed : 0;
    const int uncapped = o.max_resident < 0 || (unsigned)o.max_resident >= p->active_count;
    if (o.mode != H3_WEIGHTS_STREAM && uncapped && available >= fixed && all_blocks <= budget) {
        p->resident_count = p->active_count;
        p->resident_mask = mask;
        p->resident_bytes = all_blocks;
        p->effective_mode = H3_WEIGHTS_RESIDENT;
        return 1;
    }
    if (o.mode == H3_WEIGHTS_RESIDENT)
        return fail(error, size, "resident weights need more capacity than available after future allocations/reserve or test cap");
    if (available < fixed || two_slots > budget)
        return fail(error, size, "insufficient CUDA capacity even for two-slot streaming plus future allocations/reserve");
    p->slot_bytes = two_slots;
    p->effective_mode = H3_WEIGHTS_STREAM;
    uint64_t keep = (budget - two_slots) / block;
    if (keep >= p->active_count) keep = p->active_count - 1;
    if (o.max_resident >= 0 && keep > (unsigned)o.max_resident) keep = (unsigned)o.max_resident;
    if (o.mode == H3_WEIGHTS_STREAM) keep = 0;
    p->resident_count = (unsigned)keep;
    p->resident_bytes = keep * block;
    if (keep) p->effective_mode = H3_WEIGHTS_AUTO;
    for (unsigned i = 0; keep && i < 50; i++)
        if (mask & (UINT64_C(1) << i)) { p->resident_mask |= UINT64_C(1) << i; keep--; }
    return 1;
}

/* Packed projection descriptor (reference residency.c:39-51): the payload
 * (rows x columns FP8 bytes, or half that for NVFP4), then at `scale` (next
 * 256-byte boundary) the scale plane (4 bytes for FP8; for NVFP4 one E4M3 byte
 * per 16 columns, rows padded to 128 and block columns to 4), then at `global`
 * (next 256-byte boundary) 16 bytes of global scale; bytes = global + 16. */
WEAK int h3_weight_packed_size(uint32_t rows, uint32_t columns, int mode, uint64_t *scale, uint64_t *global,
                               uint64_t *bytes) {
    uint64_t payload, plane, end;
    if (!rows || !columns || (mode != 1 && mode != 2) || !scale || !global || !bytes || (mode == 2 && columns % 16) ||
        !mul_u64(rows, columns, &payload))
        return 0;
    if (mode == 2) payload /= 2;
    if (!add_u64(payload, 255, &end)) return 0;
    *scale = end / 256 * 256;
    plane = mode == 1 ? 4 : ((uint64_t)rows + 127) / 128 * 128 * (((uint64_t)columns / 16 + 3) / 4 * 4);
    if (!add_u64(*scale, plane, &end) || !add_u64(end, 255, &end)) return 0;
    *global = end / 256 * 256;
    return add_u64(*global, 16, bytes);
}
