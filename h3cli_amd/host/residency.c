/* Weight residency planning for h3_gpu_plan_bf16_weights / h3_gpu_plan_weights
 * (the reference's src/weights/residency.h interface).
 *
 * The planner answers one question per model: with `available` device bytes,
 * of which future allocations and a reserve are spoken for, can every active
 * block stay resident, and if not, how many can stay beside the two streaming
 * slots? Resident blocks are the lowest-indexed active ones. The environment
 * names, option meanings and error texts are the reference's, because the
 * host reads and reports them; the arithmetic is checked bit for bit against
 * the reference's own compiled planner (tests/test_ref_host.py).
 *
 * The functions are weak: a host application that links its own
 * src/weights/residency.c keeps its definitions, and this backend then plans
 * with those. */
#include "h3_residency.h"
#include <errno.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define WEAK __attribute__((weak))
#define MAX_BLOCKS 50u

static int say(char *error, size_t size, const char *text) {
    if (error && size) snprintf(error, size, "%s", text);
    return 0;
}

/* Saturation-free 64-bit helpers: 0 when the exact result does not fit. */
static int sum_fits(uint64_t a, uint64_t b, uint64_t *out) { return !__builtin_add_overflow(a, b, out); }
static int product_fits(uint64_t a, uint64_t b, uint64_t *out) { return !__builtin_mul_overflow(a, b, out); }

WEAK const char *h3_weight_mode_name(int mode) {
    static const char *const names[] = {"auto", "resident", "stream"};
    return mode == H3_WEIGHTS_RESIDENT || mode == H3_WEIGHTS_STREAM ? names[mode] : names[0];
}

/* Unsigned decimal environment value; an unset variable leaves *value as is. */
static int read_count(const char *variable, uint64_t *value) {
    const char *text = getenv(variable);
    if (!text) return 1;
    if (text[0] < '0' || text[0] > '9') return 0;
    char *end = NULL;
    errno = 0;
    const unsigned long long parsed = strtoull(text, &end, 10);
    if (errno != 0 || *end != '\0') return 0;
    *value = parsed;
    return 1;
}

WEAK int h3_weight_options_read(h3_weight_options *out, int force_stream, char *error, size_t size) {
    static const char bad_cap[] = "invalid CUDA weight test cap";
    h3_weight_options *o = out;
    *o = (h3_weight_options){H3_WEIGHTS_AUTO, -1, 0, 0};
    const char *mode = getenv("H3_CUDA_WEIGHT_MODE");
    if (mode) {
        int m = -1;
        for (int i = H3_WEIGHTS_AUTO; i <= H3_WEIGHTS_STREAM; i++)
            if (strcmp(mode, h3_weight_mode_name(i)) == 0) m = i;
        if (m < 0) return say(error, size, "CUDA weight mode must be auto, resident, or stream");
        o->mode = m;
    }
    if (force_stream) {
        if (o->mode == H3_WEIGHTS_RESIDENT)
            return say(error, size, "--ssd-streaming conflicts with CUDA resident weight mode");
        o->mode = H3_WEIGHTS_STREAM;
    }
    uint64_t cap = MAX_BLOCKS;
    if (!read_count("H3_TEST_CUDA_RESIDENT_BLOCKS", &cap) || cap > MAX_BLOCKS)
        return say(error, size, "H3_TEST_CUDA_RESIDENT_BLOCKS must be 0..50");
    if (getenv("H3_TEST_CUDA_RESIDENT_BLOCKS")) o->max_resident = (int)cap;
    if (!read_count("H3_TEST_CUDA_CAPACITY_BYTES", &o->capacity_limit) ||
        !read_count("H3_CUDA_TEST_MEMORY_BUDGET", &o->allocation_limit))
        return say(error, size, bad_cap);
    return 1;
}

WEAK int h3_weight_options_equal(const h3_weight_options *a, const h3_weight_options *b) {
    const h3_weight_options x = *a, y = *b;
    return x.mode == y.mode && x.max_resident == y.max_resident && x.capacity_limit == y.capacity_limit &&
           x.allocation_limit == y.allocation_limit;
}

/* Retry n (from 1) halves the resident ceiling: 0, 0, 1, 1, 2, ...; -1 before any. */
WEAK int h3_weight_retry_cap(unsigned count) { return count == 0 ? -1 : (int)((count - 1) >> 1); }

WEAK int h3_weight_plan_build(h3_weight_plan *plan, h3_weight_options o, uint64_t active, uint64_t block,
                              uint64_t available, uint64_t live, uint64_t future, uint64_t reserve, char *error,
                              size_t size) {
    const int options_ok = o.mode >= H3_WEIGHTS_AUTO && o.mode <= H3_WEIGHTS_STREAM && o.max_resident >= -1 &&
                           o.max_resident <= (int)MAX_BLOCKS;
    if (!plan || active == 0 || (active >> MAX_BLOCKS) != 0 || block == 0 || !options_ok)
        return say(error, size, "invalid weight planner input");
    /* The plan holds the inputs even when planning fails, for the caller's report. */
    h3_weight_plan p;
    memset(&p, 0, sizeof(p));
    p.options = o;
    p.active_mask = active;
    p.live_bytes = live;
    p.future_bytes = future;
    p.reserve_bytes = reserve;
    p.block_bytes = block;
    p.active_count = (unsigned)__builtin_popcountll(active);

    /* A test capacity cap counts what is already live against it. */
    if (o.capacity_limit) {
        const uint64_t room = o.capacity_limit > live ? o.capacity_limit - live : 0;
        if (room < available) available = room;
    }
    p.free_bytes = available;
    *plan = p;

    uint64_t spoken_for, every_block, two_slots;
    if (!sum_fits(future, reserve, &spoken_for) || !product_fits(block, p.active_count, &every_block) ||
        !product_fits(block, 2, &two_slots))
        return say(error, size, "weight planner byte overflow");
    const int room_left = available >= spoken_for;
    const uint64_t budget = room_left ? available - spoken_for : 0;

    const int cap_allows_all = o.max_resident < 0 || (unsigned)o.max_resident >= p.active_count;
    if (o.mode != H3_WEIGHTS_STREAM && cap_allows_all && room_left && every_block <= budget) {
        p.effective_mode = H3_WEIGHTS_RESIDENT;
        p.resident_count = p.active_count;
        p.resident_mask = active;
        p.resident_bytes = every_block;
        *plan = p;
        return 1;
    }
    if (o.mode == H3_WEIGHTS_RESIDENT)
        return say(error, size,
                   "resident weights need more capacity than available after future allocations/reserve or test cap");
    if (!room_left || two_slots > budget)
        return say(error, size, "insufficient CUDA capacity even for two-slot streaming plus future allocations/reserve");

    /* Streaming: two slots, plus resident blocks in what is left (never all
     * of them, never above the test cap, none in forced streaming). */
    uint64_t keep = o.mode == H3_WEIGHTS_STREAM ? 0 : (budget - two_slots) / block;
    if (keep > p.active_count - 1) keep = p.active_count - 1;
    if (o.max_resident >= 0 && keep > (uint64_t)o.max_resident) keep = (uint64_t)o.max_resident;
    p.slot_bytes = two_slots;
    p.resident_count = (unsigned)keep;
    p.resident_bytes = keep * block;
    p.effective_mode = keep ? H3_WEIGHTS_AUTO : H3_WEIGHTS_STREAM;
    for (uint64_t rest = active; keep; keep--) {
        const uint64_t lowest = rest & (~rest + 1);
        p.resident_mask |= lowest;
        rest ^= lowest;
    }
    *plan = p;
    return 1;
}

/* Packed projection descriptor shared with the reference's packers: the
 * payload (rows x columns E4M3 bytes, or half that as E2M1 pairs), the scale
 * plane at the next 256-byte boundary (one fp32 for FP8; for NVFP4 one UE4M3
 * byte per 16 columns, rows padded to 128 and scale columns to 4), then the
 * 16-byte global slot at the next 256-byte boundary. */
WEAK int h3_weight_packed_size(uint32_t rows, uint32_t columns, int mode, uint64_t *scale, uint64_t *global,
                               uint64_t *bytes) {
    if (!scale || !global || !bytes || rows == 0 || columns == 0) return 0;
    if (mode != 1 && !(mode == 2 && columns % 16 == 0)) return 0;
    uint64_t payload;
    if (!product_fits(rows, columns, &payload)) return 0;
    if (mode == 2) payload >>= 1;
    const uint64_t plane = mode == 1 ? 4 : (((uint64_t)rows + 127) & ~(uint64_t)127) * ((columns / 16 + 3) & ~3u);
    uint64_t at, end;
    if (!sum_fits(payload, 255, &at)) return 0;
    at &= ~(uint64_t)255;
    if (!sum_fits(at, plane, &end) || !sum_fits(end, 255, &end)) return 0;
    *scale = at;
    *global = end & ~(uint64_t)255;
    return sum_fits(*global, 16, bytes);
}
