// Main-DiT attention boundary: mode configuration, block-sparse mask binding and
// dispatch to the BF16 or Sage kernels. Contract of the reference's
// h3_gpu_dit_sdpa_bf16 (src/cuda/gpu_cuda.cu:1599-1668): sequence-major BF16
// Q/K/V [seq, heads, 128] after norm/RoPE, disjoint output (sequence- or
// head-major), positive finite scale rounded to BF16, deferred faults.
#include "common.h"
#include "internal.h"
#include "sage.h"
#include "subblock.h"
#include "sol.h"
#include "../../include/h3_policy.h"
#include <cmath>
#include <mutex>
#include <new>
#include <vector>

enum { MODE_DEFAULT = 0, MODE_SAGE2 = 1, MODE_SAGE3 = 2, MODE_SOL = 3, MODE_SUBBLOCK = 4 };

struct h3_attention_state {
    bool configured = false;
    int mode = MODE_DEFAULT;
    int step = -1;
    float sigma_video = 0.f, sigma_audio = 0.f;
    // SubBlock bypass policy (reference src/denoise/subblock.c:44-51): the
    // request's sparsity and warmup; dense attention when a reason applies.
    float subblock_sparsity = 0.75f;
    int subblock_warmup = 0;
    // Bound block-sparse mask (128 x 128 tiles), compacted to kept 64-key tiles.
    bool masked = false;
    uint32_t mask_q_blocks = 0, mask_k_blocks = 0, mask_block = 0;
    uint32_t *kv_list = nullptr, *kv_count = nullptr;
    uint32_t list_stride = 0;
    uint64_t kept_tiles = 0, total_tiles = 0;  // over 128-query blocks x 64-key tiles
    // SubBlock router over the bound layout (used when no host mask is bound).
    h3_subblock_router router;
    // SOL router and the options read at configure (mode 3).
    h3_sol_router sol;
    h3_sage_workspace sage;
    h3_device_buffer bf16_ws;              // transposed V of the BF16 kernel
    // Per-dispatch timing (H3_PROFILE): pairs of events collected at synchronize.
    std::vector<std::pair<hipEvent_t, hipEvent_t>> pending;
};

// ---------------------------------------------------------------- no-allocation scratch
// Workspace of h3_hip_sdpa_bf16_noalloc: the transposed V and the retry bytes
// of the dense BF16 kernel, in a fixed device array instead of a grow-only
// allocation. 384 MiB holds S = 32400 x H = 40 (332 MB) and S = 18225 x
// H = 56 (261 MB). The runtime gives every device its own copy of the array
// when the code object loads, held until the process ends. Host code never
// passes the array's name to a kernel (on the host it is only a stand-in for
// the symbol): each device's address comes from hipGetSymbolAddress, taken
// once per device at context creation with that device current.
constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(384) << 20;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex scratch_mutex;
void *scratch_address[MAX_DEVICES];   // per device, once resolved
bool scratch_resolved[MAX_DEVICES];
}  // namespace

// With g->device current (h3_gpu_create runs on it). A failure is remembered
// and reported by the entry point; contexts that never use it are unaffected.
static void resolve_scratch(h3_gpu *g) {
    if (g->device < 0 || g->device >= MAX_DEVICES) return;
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (scratch_resolved[g->device]) return;
    void *ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess) {
        (void)hipGetLastError();
        ptr = nullptr;
    }
    scratch_address[g->device] = ptr;
    scratch_resolved[g->device] = true;
}

int h3_attention_init(h3_gpu *g) {
    g->attention = new (std::nothrow) h3_attention_state();
    if (!g->attention) return h3_set_error(g, "attention: out of host memory");
    resolve_scratch(g);
    return 1;
}

void h3_attention_destroy(h3_gpu *g) {
    auto *s = g->attention;
    if (!s) return;
    if (s->kv_list) hipFree(s->kv_list);
    if (s->kv_count) hipFree(s->kv_count);
    h3_sage_workspace_free(&s->sage);
    h3_subblock_free(&s->router);
    h3_sol_free(&s->sol);
    h3_buffer_free(&s->bf16_ws);
    for (auto &p : s->pending) { hipEventDestroy(p.first); hipEventDestroy(p.second); }
    delete s; g->attention = nullptr;
}

int h3_attention_mode(h3_gpu *g) { return g && g->attention && g->attention->configured ? g->attention->mode : 0; }
h3_sol_router *h3_attention_sol(h3_gpu *g) { return g && g->attention ? &g->attention->sol : nullptr; }
h3_subblock_router *h3_attention_router(h3_gpu *g) { return g && g->attention ? &g->attention->router : nullptr; }

void h3_attention_collect_timing(h3_gpu *g) {
    auto *s = g->attention;
    if (!s) return;
    h3_subblock_collect(g, &s->router);
    h3_sol_collect(g, &s->sol);
    for (auto &p : s->pending) {
        float ms = 0;
        if (hipEventElapsedTime(&ms, p.first, p.second) == hipSuccess) {
            g->stats.attention_seconds += ms * 1e-3; g->stats.main_attention_seconds += ms * 1e-3;
            g->stats.attention_timing_samples++;
        } else g->stats.attention_timing_missed++;
        hipEventDestroy(p.first); hipEventDestroy(p.second);
    }
    s->pending.clear();
}

extern "C" int h3_gpu_dit_attention_configure(h3_gpu *g, int mode) {
    if (!g) return 0;
    auto *s = g->attention;
    if (s->configured) return h3_set_error(g, "attention context is already configured");
    if (mode < 0 || mode > 4) return h3_set_error(g, "cuda-attention must be default, sage2++, sage3, sol or subblock");
    if (mode == MODE_SAGE3) return h3_set_error(g, "sage3 (NVFP4) attention is unsupported on the HIP backend");
    if (mode == MODE_SOL) {
        // The request's options, as the reference reads them (gpu_cuda.cu:1553-1555).
        h3_cuda_sol_options o = h3_cuda_sol_current();
        if (!h3_cuda_sol_options_valid(o, g->error, sizeof(g->error))) return 0;
        s->sol.options = o;
    }
    s->mode = mode; s->configured = true;
    return 1;
}

extern "C" int h3_gpu_dit_attention_noise(h3_gpu *g, int step, float video, float audio) {
    if (!g) return 0;
    auto *s = g->attention;
    if (s->mode != MODE_SUBBLOCK && s->mode != MODE_SOL) return 1;
    if (step < 0 || !finite_f32(video) || !finite_f32(audio) || video < 0 || video > 1 || audio < 0 || audio > 1)
        return h3_set_error(g, "invalid HIP attention absolute step/noise");
    s->step = step;
    s->sigma_video = video;
    s->sigma_audio = audio;
    return 1;
}

extern "C" int h3_hip_dit_block_mask(h3_gpu *g, const uint8_t *mask, uint32_t qb, uint32_t kb, uint32_t block) {
    if (!g) return 0;
    auto *s = g->attention;
    if (g->active && !h3_hip_check(g, hipStreamSynchronize(g->compute), "mask rebind fence")) return 0;
    if (s->kv_list) { hipFree(s->kv_list); s->kv_list = nullptr; }
    if (s->kv_count) { hipFree(s->kv_count); s->kv_count = nullptr; }
    s->masked = false; s->kept_tiles = s->total_tiles = 0;
    if (!mask) return 1;
    if (block != 128) return h3_set_error(g, "block mask: block must be 128");
    if (!qb || !kb || qb > (1u << 20) || kb > (1u << 20)) return h3_set_error(g, "block mask: invalid shape");
    // The kernel walks 128-query blocks over 64-key tiles: each kept 128-key
    // block contributes its two 64-key tiles.
    const uint32_t q_rows = qb, tiles = kb * 2;
    std::vector<uint32_t> count(q_rows, 0), list((size_t)q_rows * tiles, 0);
    for (uint32_t r = 0; r < q_rows; r++) {
        uint32_t c = 0;
        for (uint32_t t = 0; t < tiles; t++)
            if (mask[(size_t)r * kb + t / 2]) list[(size_t)r * tiles + c++] = t;
        count[r] = c;
        s->kept_tiles += c;
    }
    s->total_tiles = (uint64_t)q_rows * tiles;
    if (!h3_hip_check(g, hipMalloc(&s->kv_list, list.size() * 4), "mask list") ||
        !h3_hip_check(g, hipMalloc(&s->kv_count, count.size() * 4), "mask counts") ||
        !h3_hip_check(g, hipMemcpy(s->kv_list, list.data(), list.size() * 4, hipMemcpyHostToDevice), "mask list upload") ||
        !h3_hip_check(g, hipMemcpy(s->kv_count, count.data(), count.size() * 4, hipMemcpyHostToDevice), "mask count upload"))
        return 0;
    s->mask_q_blocks = q_rows; s->mask_k_blocks = kb; s->mask_block = block; s->list_stride = tiles;
    s->masked = true;
    return 1;
}

static float round_scale_bf16(float scale) {
    uint32_t bits; memcpy(&bits, &scale, 4);
    bits = (bits + 0x7fffu + ((bits >> 16) & 1u)) & 0xffff0000u;
    memcpy(&scale, &bits, 4);
    return scale;
}

static int dispatch(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *q, const h3_gpu_tensor *k,
                    const h3_gpu_tensor *v, uint32_t seq, uint32_t heads, float scale, bool head_major,
                    int mode, bool masked) {
    auto *s = g->attention;
    hipEvent_t t0 = nullptr, t1 = nullptr;
    if (g->profiling) {
        hipEventCreate(&t0); hipEventCreate(&t1);
        hipEventRecord(t0, g->compute);
    }
    const uint32_t *list = masked ? s->kv_list : nullptr;
    const uint32_t *cnt = masked ? s->kv_count : nullptr;
    const uint32_t stride = s->list_stride;
    int ok;
    if (mode == MODE_SAGE2) {
        ok = h3_sage_attention(g, &s->sage, (uint16_t *)out->data, (const uint16_t *)q->data, (const uint16_t *)k->data,
                               (const uint16_t *)v->data, seq, heads, scale, head_major, list, cnt, stride);
        if (ok) g->stats.sage2_attention_dispatches++;
    } else {
        ok = h3_buffer_reserve(g, &s->bf16_ws, h3_attention_bf16_workspace(seq, heads), "attention workspace") &&
             h3_launch_attention_bf16(g, s->bf16_ws.ptr, (uint16_t *)out->data, (const uint16_t *)q->data, (const uint16_t *)k->data,
                                      (const uint16_t *)v->data, seq, heads, scale, head_major, list, cnt, stride);
    }
    g->stats.attention_workspace_bytes = s->sage.bytes + s->bf16_ws.bytes;
    if (g->profiling) {
        hipEventRecord(t1, g->compute);
        s->pending.emplace_back(t0, t1);
    }
    if (ok) {
        g->stats.attention_dispatches++;
        if (masked) { g->stats.subblock_calls++; g->stats.subblock_selected += s->kept_tiles; g->stats.subblock_possible += s->total_tiles; }
        else if (mode == MODE_DEFAULT) g->stats.main_dense_calls++;
    }
    return ok;
}

// SubBlock routed attention (reference gpu_cuda.cu:1620-1639) under the fixed
// workspace budget: heads in groups and 64-query blocks in slabs, as planned
// by h3_subblock_plan; each chunk routes its slab (pooling its head group's
// cells and transposing its V on the group's first slab) and runs the listed
// kernel over it. Every (head, query block) is computed as in one whole call,
// so the output does not depend on the split.
static int routed(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *q, const h3_gpu_tensor *k,
                  const h3_gpu_tensor *v, uint32_t seq, uint32_t heads, float scale, bool head_major, unsigned keep) {
    auto *s = g->attention;
    auto *r = &s->router;
    h3_subblock_chunking plan;
    if (!h3_subblock_plan(g, r, seq, heads, &plan)) return 0;
    if (!h3_buffer_reserve(g, &s->bf16_ws, plan.vt_bytes, "attention workspace")) return 0;
    hipEvent_t t0 = nullptr, t1 = nullptr;
    if (g->profiling) {
        hipEventCreate(&t0); hipEventCreate(&t1);
        hipEventRecord(t0, g->compute);
    }
    const uint32_t blocks = r->blocks;
    const auto *qd = (const uint16_t *)q->data, *kd = (const uint16_t *)k->data, *vd = (const uint16_t *)v->data;
    r->plan = plan;
    r->chunked = plan.group < heads || plan.slab < blocks;
    int ok = 1;
    for (uint32_t h0 = 0; ok && h0 < heads; h0 += plan.group) {
        const uint32_t gh = std::min(plan.group, heads - h0);
        for (uint32_t qb0 = 0; ok && qb0 < blocks; qb0 += plan.slab) {
            const uint32_t qs = std::min(plan.slab, blocks - qb0);
            ok = h3_subblock_route(g, r, qd, kd, seq, heads, h0, gh, qb0, qs, scale, keep, false, qb0 == 0) &&
                 h3_launch_attention_routed(g, s->bf16_ws.ptr, (uint16_t *)out->data, qd, kd, vd, seq, heads, scale,
                                            head_major, h3_subblock_lists(r), h3_subblock_counts(r), blocks, h0, gh,
                                            qb0, qs, qb0 == 0);
        }
    }
    g->stats.attention_workspace_bytes = s->sage.bytes + s->bf16_ws.bytes + r->ws.bytes;
    if (g->profiling) {
        hipEventRecord(t1, g->compute);
        s->pending.emplace_back(t0, t1);
    }
    if (ok) {
        g->stats.subblock_router_calls++;
        g->stats.attention_dispatches++;
        g->stats.subblock_calls++;
        g->stats.subblock_protected_calls += r->protected_ranges;
    }
    return ok;
}

static int validate(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *q, const h3_gpu_tensor *k,
                    const h3_gpu_tensor *v, uint32_t seq, uint32_t heads, uint32_t dim, float scale) {
    size_t n = (size_t)seq * heads * dim;
    if (!h3_launch_ready(g)) return 0;
    if (!seq || seq > INT32_MAX / 128 || !heads || heads > 65535 || dim != 128 || !finite_f32(scale) || scale <= 0 ||
        !out || !q || !k || !v || out == q || out == k || out == v)
        return h3_set_error(g, "DiT attention requires disjoint BF16 output, S>0, H>0, D=128 and a positive FP32 scale");
    return h3_require(g, q, H3_GPU_BF16, n, "DiT attention Q") && h3_require(g, k, H3_GPU_BF16, n, "DiT attention K") &&
           h3_require(g, v, H3_GPU_BF16, n, "DiT attention V") && h3_require(g, out, H3_GPU_BF16, n, "DiT attention output");
}

extern "C" int h3_gpu_dit_sdpa_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *q, const h3_gpu_tensor *k,
                                    const h3_gpu_tensor *v, uint32_t seq, uint32_t heads, uint32_t dim, float scale,
                                    int head_major, unsigned block, int step) {
    (void)block;
    if (!g) return 0;
    if (!validate(g, out, q, k, v, seq, heads, dim, scale)) return 0;
    if ((head_major != 0 && head_major != 1) || step < 0)
        return h3_set_error(g, "DiT attention: head_major must be 0/1 and step >= 0");
    auto *s = g->attention;
    bool masked = s->masked;
    if (s->mode == MODE_SOL) {
        // reference gpu_cuda.cu:1643-1662: the bypass rules run dense; routed
        // calls use the BF16-rounded scale.
        if (step != s->step) return h3_set_error(g, "SOL absolute step was not bound");
        if (h3_cuda_sol_dense_reason(s->sol.options, block, step, s->sigma_video, s->sigma_audio)) {
            s->sol.bypass++;
            return dispatch(g, out, q, k, v, seq, heads, round_scale_bf16(scale), head_major != 0, MODE_DEFAULT, false);
        }
        const float rounded = round_scale_bf16(scale);
        // Centroids of all heads, then routes, lists and attention per head
        // group under the fixed workspace budget.
        uint32_t group = 0;
        size_t bytes = 0;
        if (!h3_sol_plan(g, &s->sol, seq, heads, &group, &bytes) ||
            !h3_buffer_reserve(g, &s->bf16_ws, h3_attention_bf16_workspace(seq, group), "attention workspace") ||
            !h3_sol_prepare(g, &s->sol, (const uint16_t *)q->data, (const uint16_t *)k->data,
                            (const uint16_t *)v->data, seq, heads, group))
            return 0;
        for (uint32_t h0 = 0; h0 < heads; h0 += group) {
            const uint32_t gh = std::min(group, heads - h0);
            if (!h3_sol_route(g, &s->sol, seq, heads, h0, gh, rounded)) return 0;
            const h3_sol_lists lists = h3_sol_lists_of(&s->sol);
            if (!h3_launch_attention_sol(g, s->bf16_ws.ptr, (uint16_t *)out->data, (const uint16_t *)q->data,
                                         (const uint16_t *)k->data, (const uint16_t *)v->data, seq, heads, rounded,
                                         head_major != 0, (uint32_t)s->sol.options.q_block, &lists, h0, gh))
                return 0;
        }
        s->sol.plan_bytes = bytes;
        g->stats.attention_dispatches++;
        return 1;
    }
    if (s->mode == MODE_SUBBLOCK) {
        if (step != s->step) return h3_set_error(g, "SubBlock absolute step was not bound");
        const char *reason = h3_subblock_dense_reason(seq, block, step, s->subblock_sparsity, s->subblock_warmup);
        if (reason) {
            g->stats.subblock_bypass++;
            masked = false;
        } else if (!s->masked) {
            // Router path (reference gpu_cuda.cu:1620-1639): the scale is used
            // as given; protected query blocks route every key block, which
            // is the dense result the reference computes for them separately.
            const unsigned blocks = (seq + 63) / 64;
            const unsigned keep = h3_subblock_budget(blocks, s->subblock_sparsity);
            return routed(g, out, q, k, v, seq, heads, scale, head_major != 0, keep);
        }
    }
    // A kept last 128-key block may list a 64-key tile wholly past the sequence
    // end; the kernels load zeros there and mask keys >= seq to -inf.
    if (masked && (s->mask_q_blocks != (seq + 127) / 128 || s->mask_k_blocks != (seq + 127) / 128))
        return h3_set_error(g, "bound block mask does not match sequence %u", seq);
    return dispatch(g, out, q, k, v, seq, heads, round_scale_bf16(scale), head_major != 0,
                    s->mode == MODE_SAGE2 ? MODE_SAGE2 : MODE_DEFAULT, masked);
}

extern "C" int h3_gpu_sdpa_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *q, const h3_gpu_tensor *k,
                                const h3_gpu_tensor *v, uint32_t seq, uint32_t heads, uint32_t dim, float scale) {
    if (!g || !validate(g, out, q, k, v, seq, heads, dim, scale)) return 0;
    return dispatch(g, out, q, k, v, seq, heads, round_scale_bf16(scale), false, MODE_DEFAULT, false);
}

extern "C" int h3_gpu_sdpa_bf16_head_major_output(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *q,
                                                  const h3_gpu_tensor *k, const h3_gpu_tensor *v, uint32_t seq,
                                                  uint32_t heads, uint32_t dim, float scale) {
    if (!g || !validate(g, out, q, k, v, seq, heads, dim, scale)) return 0;
    return dispatch(g, out, q, k, v, seq, heads, round_scale_bf16(scale), true, MODE_DEFAULT, false);
}

// Dense BF16 SDPA (the kernels of h3_gpu_sdpa_bf16 / _head_major_output)
// with its workspace in the fixed scratch array: no device allocation and no
// allocating library call. Every call on one device shares that device's
// array, so calls that overlap on one GPU (two contexts, or two streams) race.
// Nothing in the array needs clearing: the V transpose writes every byte the
// kernel reads, and every wave of the main launch writes its retry byte.
extern "C" int h3_hip_sdpa_bf16_noalloc(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *q,
                                        const h3_gpu_tensor *k, const h3_gpu_tensor *v, uint32_t seq,
                                        uint32_t heads, uint32_t dim, float scale, int head_major) {
    if (!g || !validate(g, out, q, k, v, seq, heads, dim, scale)) return 0;
    if (head_major != 0 && head_major != 1) return h3_set_error(g, "no-allocation attention: head_major must be 0/1");
    const size_t need = h3_attention_bf16_workspace(seq, heads);
    if (need > NOALLOC_SCRATCH_BYTES)
        return h3_set_error(g, "no-allocation attention: S=%u H=%u needs %zu workspace bytes, above the fixed %zu",
                            seq, heads, need, NOALLOC_SCRATCH_BYTES);
    void *ws = nullptr;
    {
        std::lock_guard<std::mutex> lock(scratch_mutex);
        if (g->device >= 0 && g->device < MAX_DEVICES && scratch_resolved[g->device]) ws = scratch_address[g->device];
    }
    if (!ws) return h3_set_error(g, "no-allocation attention: the scratch array of device %d is not available", g->device);
    const int ok = h3_launch_attention_bf16(g, ws, (uint16_t *)out->data, (const uint16_t *)q->data,
                                            (const uint16_t *)k->data, (const uint16_t *)v->data, seq, heads,
                                            round_scale_bf16(scale), head_major != 0, nullptr, nullptr, 0);
    if (ok) g->stats.attention_dispatches++;
    return ok;
}

extern "C" int h3_hip_dit_subblock_policy(h3_gpu *g, float sparsity, int warmup) {
    if (!g) return 0;
    if (!(sparsity >= 0.f) || sparsity >= 1.f) return h3_set_error(g, "SubBlock sparsity must be in [0, 1)");
    g->attention->subblock_sparsity = sparsity;
    g->attention->subblock_warmup = warmup;
    return 1;
}

// SOL counters (the reference's per-synchronize "SOL counters" report,
// gpu_cuda.cu:452-460): out[0] routed calls, out[1] dense bypasses, out[2..8]
// pair counts exact, approximate, protected, local, floor, recovery, tail.
// Counts of calls not yet synchronized are collected first.
extern "C" int h3_hip_sol_counters(h3_gpu *g, uint64_t *out, size_t count) {
    if (!g || !g->attention) return 0;
    if (!out || count != 9) return h3_set_error(g, "SOL counters: expected 9 values");
    auto &r = g->attention->sol;
    if (r.pending) {
        if (!h3_hip_check(g, hipStreamSynchronize(g->compute), "SOL counters")) return 0;
        h3_sol_collect(g, &r);
    }
    out[0] = r.calls; out[1] = r.bypass;
    for (int j = 0; j < 7; j++) out[2 + j] = r.pairs[j];
    return 1;
}

extern "C" int h3_hip_dit_sol_force_exact(h3_gpu *g, int on) {
    if (!g) return 0;
    g->attention->sol.force_exact = on != 0;
    return 1;
}

// Workspace budget of SubBlock routed calls on this context (0 restores the
// fixed 512 MiB) and the split of the last routed call.
extern "C" int h3_hip_subblock_workspace_cap(h3_gpu *g, size_t bytes) {
    if (!g || !g->attention) return 0;
    g->attention->router.cap = bytes ? bytes : H3_SUBBLOCK_WORKSPACE_CAP;
    return 1;
}

extern "C" int h3_hip_subblock_plan_info(h3_gpu *g, uint32_t *group, uint32_t *slab, size_t *bytes) {
    if (!g || !g->attention) return 0;
    const auto &p = g->attention->router.plan;
    if (!p.group) return h3_set_error(g, "SubBlock plan: no routed call yet");
    if (group) *group = p.group;
    if (slab) *slab = p.slab;
    if (bytes) *bytes = p.bytes;
    return 1;
}

// Workspace budget of SOL routed calls on this context (0 restores 512 MiB)
// and the head group and bytes of the last routed call.
extern "C" int h3_hip_sol_workspace_cap(h3_gpu *g, size_t bytes) {
    if (!g || !g->attention) return 0;
    g->attention->sol.cap = bytes ? bytes : (size_t)512 << 20;
    return 1;
}

extern "C" int h3_hip_sol_plan_info(h3_gpu *g, uint32_t *group, size_t *bytes) {
    if (!g || !g->attention) return 0;
    const auto &r = g->attention->sol;
    if (!r.group) return h3_set_error(g, "SOL plan: no routed call yet");
    if (group) *group = r.group;
    if (bytes) *bytes = r.plan_bytes;
    return 1;
}
