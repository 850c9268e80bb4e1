// Context, tensors, events, command lifecycle and weight streaming of the gfx950
// backend. Mirrors the execution model of the reference operator surface
// (src/gpu.h:260-268; src/cuda/gpu_cuda.cu:429-489): one ordered compute stream,
// one copy stream for streamed weights, deferred device faults reported at submit.
#include "common.h"
#include "internal.h"
#include <algorithm>
#include <cerrno>
#include <cmath>
#include <fcntl.h>
#include <new>
#include <unistd.h>
#include <chrono>
#include <condition_variable>
#include <memory>
#include <mutex>
#include <thread>

#ifndef H3HIP_VERSION
#define H3HIP_VERSION "0.1"
#endif

static double now_seconds() {
    using namespace std::chrono;
    return duration<double>(steady_clock::now().time_since_epoch()).count();
}

extern "C" const char *h3_hip_version(void) { return "h3hip gfx950 " H3HIP_VERSION; }

int h3_set_error(h3_gpu *g, const char *fmt, ...) {
    if (!g) return 0;
    va_list ap; va_start(ap, fmt);
    vsnprintf(g->error, sizeof(g->error), fmt, ap);
    va_end(ap);
    return 0;
}

int h3_hip_check(h3_gpu *g, hipError_t e, const char *what) {
    if (e == hipSuccess) return 1;
    return h3_set_error(g, "%s: %s", what, hipGetErrorString(e));
}

int h3_launch_ready(h3_gpu *g) {
    if (!g) return 0;
    if (!g->active) return h3_set_error(g, "no active HIP command (call h3_gpu_begin)");
    return 1;
}

int h3_launch_status(h3_gpu *g, const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) { g->deferred_error = true; return h3_set_error(g, "%s launch: %s", what, hipGetErrorString(e)); }
    return 1;
}

static size_t item_size(h3_gpu_dtype d) {
    switch (d) {
    case H3_GPU_F32: case H3_GPU_U32: return 4;
    case H3_GPU_BF16: case H3_GPU_F16: return 2;
    case H3_GPU_I8: return 1;
    }
    return 0;
}

int h3_require(h3_gpu *g, const h3_gpu_tensor *t, h3_gpu_dtype dtype, size_t elements, const char *name) {
    if (!t) return h3_set_error(g, "%s: missing tensor", name);
    if (t->owner != g) return h3_set_error(g, "%s: tensor belongs to another context", name);
    if (t->q8) return h3_set_error(g, "%s: packed q8 weight is not a plain tensor", name);
    if (t->dtype != dtype) return h3_set_error(g, "%s: dtype %d, expected %d", name, (int)t->dtype, (int)dtype);
    if (t->elements < elements) return h3_set_error(g, "%s: %zu elements, need %zu", name, t->elements, elements);
    return 1;
}

void h3_stats_track_alloc(h3_gpu *g, size_t bytes, int sign) {
    if (sign > 0) {
        g->stats.allocated_bytes += bytes; g->stats.live_bytes += bytes; g->stats.tensor_allocations++;
        g->stats.device_bytes += bytes;
        g->stats.peak_live_bytes = std::max(g->stats.peak_live_bytes, g->stats.live_bytes);
    } else {
        g->stats.live_bytes -= std::min<uint64_t>(g->stats.live_bytes, bytes);
        g->stats.device_bytes -= std::min<uint64_t>(g->stats.device_bytes, bytes);
    }
}

// ------------------------------------------------------------------ context
extern "C" h3_gpu *h3_gpu_create(const char *shader_source_path, char *error, size_t error_size) {
    (void)shader_source_path;
    auto fail = [&](const char *what, hipError_t e) -> h3_gpu * {
        if (error && error_size) snprintf(error, error_size, "%s: %s", what, hipGetErrorString(e));
        return nullptr;
    };
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return fail("no HIP device", e);
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess) return fail("device properties", e);
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        if (error && error_size) snprintf(error, error_size, "h3hip is built for gfx950, device is %s", prop.gcnArchName);
        return nullptr;
    }
    h3_gpu *g = new (std::nothrow) h3_gpu();
    if (!g) { if (error && error_size) snprintf(error, error_size, "out of host memory"); return nullptr; }
    g->device = device;
    g->created = now_seconds();
    g->profiling = getenv("H3_PROFILE") != nullptr;
    if (const char *v = getenv("H3_HIP_ATTENTION_VARIANT")) g->attention_variant = atoi(v);
    if (const char *v = getenv("H3_HIP_GEMM_VARIANT")) g->gemm_variant = atoi(v);
    // Both streams keep the default priority.
    if ((e = hipStreamCreateWithFlags(&g->compute, hipStreamNonBlocking)) != hipSuccess ||
        (e = hipStreamCreateWithFlags(&g->copy, hipStreamNonBlocking)) != hipSuccess) {
        h3_gpu_free(g); return fail("create streams", e);
    }
    if ((e = hipMalloc(&g->fault, 4 * sizeof(unsigned))) != hipSuccess) { g->fault = nullptr; h3_gpu_free(g); return fail("fault flags", e); }
    if ((e = hipMemset(g->fault, 0, 4 * sizeof(unsigned))) != hipSuccess) { h3_gpu_free(g); return fail("fault flags", e); }
    if (!h3_attention_init(g)) {
        if (error && error_size) snprintf(error, error_size, "%s", g->error);
        h3_gpu_free(g); return nullptr;
    }
    return g;
}

static void kernel_events_clear(h3_gpu *g);

extern "C" void h3_gpu_free(h3_gpu *g) {
    if (!g) return;
    if (g->compute) hipStreamSynchronize(g->compute);
    if (g->copy) hipStreamSynchronize(g->copy);
    h3_attention_destroy(g);
    h3_streaming_destroy(g);
    h3_quant_destroy(g);
    kernel_events_clear(g);
    delete g->kernel_events;
    if (g->fault) hipFree(g->fault);
    if (g->gemm_weights) hipFree(g->gemm_weights);
    if (g->compute) hipStreamDestroy(g->compute);
    if (g->copy) hipStreamDestroy(g->copy);
    delete g;
}

extern "C" const char *h3_gpu_backend_name(const h3_gpu *g) { (void)g; return "hip"; }

extern "C" int h3_gpu_begin(h3_gpu *g) {
    if (!g) return 0;
    if (g->active) return h3_set_error(g, "HIP command stream already active");
    g->error[0] = 0; g->deferred_error = false;
    g->active = true;
    return 1;
}

extern "C" int h3_gpu_continue(h3_gpu *g) {
    if (!h3_launch_ready(g)) return 0;
    return h3_hip_check(g, hipPeekAtLastError(), "continue");
}

extern "C" int h3_gpu_synchronize(h3_gpu *g) {
    if (!g) return 0;
    double t = now_seconds();
    int ok = h3_hip_check(g, hipStreamSynchronize(g->compute), "compute synchronization");
    if (ok) {
        unsigned flags[4] = {0, 0, 0, 0};
        ok = h3_hip_check(g, hipMemcpy(flags, g->fault, sizeof(flags), hipMemcpyDeviceToHost), "fault flags");
        if (ok && flags[0]) ok = h3_set_error(g, "nonfinite attention input or output");
        else if (ok && flags[1]) ok = h3_set_error(g, "nonfinite input encountered in Sage quantization");
        else if (ok && flags[2]) ok = h3_set_error(g, "nonfinite input encountered in quantized DiT projection");
        if (flags[0] || flags[1] || flags[2]) {
            // Sticky until cancel, like the reference's deferred faults.
            g->deferred_error = true;
        }
    }
    g->stats.command_wait_seconds += now_seconds() - t;
    if (ok) h3_attention_collect_timing(g);
    return ok && !g->deferred_error;
}

extern "C" int h3_gpu_submit(h3_gpu *g) {
    if (!h3_launch_ready(g)) return 0;
    int ok = h3_gpu_synchronize(g);
    g->active = false; g->stats.submissions++;
    return ok;
}

extern "C" void h3_gpu_cancel(h3_gpu *g) {
    if (!g) return;
    hipStreamSynchronize(g->compute);
    hipStreamSynchronize(g->copy);
    if (g->fault) { hipMemsetAsync(g->fault, 0, 4 * sizeof(unsigned), g->compute); hipStreamSynchronize(g->compute); }
    hipGetLastError();
    g->deferred_error = false; g->active = false; g->error[0] = 0;
}

extern "C" const char *h3_gpu_error(const h3_gpu *g) { return g ? g->error : "missing HIP context"; }

extern "C" int h3_gpu_get_stats(const h3_gpu *g, h3_gpu_stats *s) {
    if (!g || !s) return 0;
    *s = g->stats;
    return 1;
}

// ------------------------------------------------------------------ tensors
extern "C" h3_gpu_tensor *h3_gpu_tensor_alloc(h3_gpu *g, size_t elements, h3_gpu_dtype dtype, h3_gpu_storage storage) {
    if (!g) return nullptr;
    size_t size = item_size(dtype);
    if (!size || !elements || elements > SIZE_MAX / size) { h3_set_error(g, "tensor: invalid size/dtype"); return nullptr; }
    auto *t = new (std::nothrow) h3_gpu_tensor();
    if (!t) { h3_set_error(g, "tensor: out of host memory"); return nullptr; }
    t->owner = g; t->elements = elements; t->dtype = dtype; t->storage = storage;
    t->bytes = elements * size;
    // 256-byte slack keeps vectorized tail loads inside the allocation.
    size_t alloc = (t->bytes + 511) & ~(size_t)255;
    hipError_t e = storage == H3_GPU_DEVICE_ONLY ? hipMalloc(&t->data, alloc)
                                                 : hipHostMalloc(&t->data, alloc, hipHostMallocDefault);
    if (e != hipSuccess) {
        size_t free_b = 0, total_b = 0; hipMemGetInfo(&free_b, &total_b);
        h3_set_error(g, "tensor allocation of %zu bytes failed: %s (free %.2f GiB)", alloc, hipGetErrorString(e), free_b / 1073741824.0);
        if (e == hipErrorOutOfMemory) g->allocation_failed = true;
        delete t; hipGetLastError(); return nullptr;
    }
    if (storage != H3_GPU_DEVICE_ONLY) { g->stats.pinned_bytes += alloc; g->stats.peak_pinned_bytes = std::max(g->stats.peak_pinned_bytes, g->stats.pinned_bytes); }
    else h3_stats_track_alloc(g, alloc, +1);
    t->bytes_alloc = alloc;
    return t;
}

extern "C" void *h3_hip_tensor_device_pointer(h3_gpu_tensor *t) {
    return t && t->storage == H3_GPU_DEVICE_ONLY ? t->data : nullptr;
}

extern "C" void *h3_hip_compute_stream(h3_gpu *g) { return g ? (void *)g->compute : nullptr; }

extern "C" void *h3_gpu_tensor_contents(h3_gpu_tensor *t) {
    if (!t || t->storage == H3_GPU_DEVICE_ONLY) return nullptr;
    hipStreamSynchronize(t->owner->compute);
    return t->data;
}

extern "C" h3_gpu_tensor *h3_gpu_tensor_new_f32(h3_gpu *g, size_t n) { return h3_gpu_tensor_alloc(g, n, H3_GPU_F32, H3_GPU_DEVICE_ONLY); }
extern "C" h3_gpu_tensor *h3_gpu_tensor_new_bf16(h3_gpu *g, size_t n) { return h3_gpu_tensor_alloc(g, n, H3_GPU_BF16, H3_GPU_DEVICE_ONLY); }
extern "C" h3_gpu_tensor *h3_gpu_tensor_new_i8(h3_gpu *g, size_t n) { return h3_gpu_tensor_alloc(g, n, H3_GPU_I8, H3_GPU_DEVICE_ONLY); }

static int write_bytes(h3_gpu_tensor *t, size_t offset, const void *src, size_t bytes) {
    h3_gpu *g = t->owner;
    if (offset > t->bytes || bytes > t->bytes - offset) return h3_set_error(g, "tensor write out of range");
    if (!bytes) return 1;
    return h3_hip_check(g, hipMemcpyAsync((char *)t->data + offset, src, bytes, hipMemcpyHostToDevice, g->compute), "tensor write") &&
           h3_hip_check(g, hipStreamSynchronize(g->compute), "tensor write sync") &&
           (g->stats.h2d_bytes += bytes, 1);
}
static int read_bytes(const h3_gpu_tensor *t, size_t offset, void *dst, size_t bytes) {
    h3_gpu *g = t->owner;
    if (offset > t->bytes || bytes > t->bytes - offset) return h3_set_error(g, "tensor read out of range");
    if (!bytes) return 1;
    return h3_hip_check(g, hipStreamSynchronize(g->compute), "tensor read sync") &&
           h3_hip_check(g, hipMemcpy(dst, (const char *)t->data + offset, bytes, hipMemcpyDeviceToHost), "tensor read") &&
           (g->stats.d2h_bytes += bytes, 1);
}

static h3_gpu_tensor *from_values(h3_gpu *g, const void *v, size_t n, h3_gpu_dtype d) {
    if (!g || !v) return nullptr;
    h3_gpu_tensor *t = h3_gpu_tensor_alloc(g, n, d, H3_GPU_DEVICE_ONLY);
    if (t && !write_bytes(t, 0, v, t->bytes)) { h3_gpu_tensor_free(t); return nullptr; }
    return t;
}
extern "C" h3_gpu_tensor *h3_gpu_tensor_from_f32(h3_gpu *g, const float *v, size_t n) { return from_values(g, v, n, H3_GPU_F32); }
extern "C" h3_gpu_tensor *h3_gpu_tensor_from_bf16(h3_gpu *g, const uint16_t *v, size_t n) { return from_values(g, v, n, H3_GPU_BF16); }
extern "C" h3_gpu_tensor *h3_gpu_tensor_from_u32(h3_gpu *g, const uint32_t *v, size_t n) { return from_values(g, v, n, H3_GPU_U32); }

extern "C" void h3_gpu_tensor_free(h3_gpu_tensor *t) {
    if (!t) return;
    h3_gpu *g = t->owner;
    // A queued kernel may still read the buffer.
    hipStreamSynchronize(g->compute);
    hipStreamSynchronize(g->copy);
    if (t->ready) hipEventDestroy(t->ready);
    if (t->released) hipEventDestroy(t->released);
    if (t->storage == H3_GPU_DEVICE_ONLY) { hipFree(t->data); h3_stats_track_alloc(g, t->bytes_alloc, -1); }
    else { hipHostFree(t->data); g->stats.pinned_bytes -= std::min<uint64_t>(g->stats.pinned_bytes, t->bytes_alloc); }
    if (t->q8_scales) hipFree(t->q8_scales);
    if (t->quant_dequant) { hipFree(t->quant_dequant); t->quant_dequant = nullptr; }
    delete t;
}

extern "C" size_t h3_gpu_tensor_elements(const h3_gpu_tensor *t) { return t ? t->elements : 0; }
extern "C" h3_gpu_dtype h3_gpu_tensor_dtype(const h3_gpu_tensor *t) { return t ? t->dtype : H3_GPU_F32; }

#define TYPED_IO(T, D, NAME)                                                                  \
    extern "C" int h3_gpu_tensor_read_##NAME(const h3_gpu_tensor *t, T *v, size_t n) {       \
        if (!t || !v || t->dtype != D || t->q8) return 0;                                     \
        return read_bytes(t, 0, v, n * sizeof(T));                                            \
    }
TYPED_IO(float, H3_GPU_F32, f32)
TYPED_IO(uint16_t, H3_GPU_BF16, bf16)
TYPED_IO(uint32_t, H3_GPU_U32, u32)
#undef TYPED_IO

extern "C" int h3_gpu_tensor_read_f32_range(const h3_gpu_tensor *t, size_t off, float *v, size_t n) {
    if (!t || !v || t->dtype != H3_GPU_F32 || off > SIZE_MAX / 4) return 0;
    return read_bytes(t, off * 4, v, n * 4);
}
extern "C" int h3_gpu_tensor_write_f32(h3_gpu_tensor *t, const float *v, size_t n) {
    if (!t || !v || t->dtype != H3_GPU_F32) return 0;
    return write_bytes(t, 0, v, n * 4);
}
extern "C" int h3_gpu_tensor_write_f32_range(h3_gpu_tensor *t, size_t off, const float *v, size_t n) {
    if (!t || !v || t->dtype != H3_GPU_F32 || off > SIZE_MAX / 4) return 0;
    return write_bytes(t, off * 4, v, n * 4);
}
extern "C" int h3_gpu_tensor_write_bf16(h3_gpu_tensor *t, const uint16_t *v, size_t n) {
    if (!t || !v || t->dtype != H3_GPU_BF16) return 0;
    return write_bytes(t, 0, v, n * 2);
}
extern "C" int h3_gpu_tensor_write_bf16_range(h3_gpu_tensor *t, size_t off, const uint16_t *v, size_t n) {
    if (!t || !v || t->dtype != H3_GPU_BF16 || off > SIZE_MAX / 2) return 0;
    return write_bytes(t, off * 2, v, n * 2);
}

// ------------------------------------------------------------------ events
extern "C" h3_gpu_event *h3_gpu_event_new(h3_gpu *g) {
    if (!g) return nullptr;
    auto *e = new (std::nothrow) h3_gpu_event();
    if (!e) return nullptr;
    if (!h3_hip_check(g, hipEventCreateWithFlags(&e->event, hipEventDisableTiming), "create event")) { delete e; return nullptr; }
    return e;
}
extern "C" h3_gpu_event *h3_hip_timing_event_new(h3_gpu *g) {
    if (!g) return nullptr;
    auto *e = new (std::nothrow) h3_gpu_event();
    if (!e) return nullptr;
    if (!h3_hip_check(g, hipEventCreate(&e->event), "create timing event")) { delete e; return nullptr; }
    return e;
}
extern "C" int h3_gpu_event_record(h3_gpu *g, h3_gpu_event *e) {
    return g && e && h3_hip_check(g, hipEventRecord(e->event, g->compute), "record event");
}
extern "C" int h3_gpu_event_wait(h3_gpu *g, h3_gpu_event *e) {
    return g && e && h3_hip_check(g, hipStreamWaitEvent(g->compute, e->event, 0), "wait event");
}
extern "C" void h3_gpu_event_free(h3_gpu_event *e) {
    if (!e) return;
    hipEventDestroy(e->event);
    delete e;
}
extern "C" int h3_hip_event_elapsed_ms(h3_gpu *g, h3_gpu_event *a, h3_gpu_event *b, float *ms) {
    if (!g || !a || !b || !ms) return 0;
    return h3_hip_check(g, hipEventElapsedTime(ms, a->event, b->event), "event elapsed time");
}

// ------------------------------------------------------------------ weight streaming
// File → device fills (the reference's h3_gpu_tensor_read/stream_file_bf16,
// src/gpu.h:225-236; behaviour of src/cuda/gpu_cuda.cu:761-840) go through a
// ring of pinned staging slots. A reader thread pulls the file into the slots
// while the calling thread queues each filled slot's H2D copy on the copy
// stream and records that slot's "drained" event behind it; the reader waits on
// that event before it reuses the slot. Each destination tensor also carries a
// "ready" event (recorded on the copy stream after its last chunk; kernels that
// read the tensor wait on it) and a "released" event (recorded on the compute
// stream after the last kernel that read it; the next fill waits on it).
namespace {
constexpr unsigned kStagingSlots = 4;
constexpr size_t kStagingSlotBytes = 8u << 20;

struct StagingSlot {
    void *host = nullptr;
    hipEvent_t drained = nullptr;
    bool armed = false;  // drained has been recorded at least once
};
}  // namespace

struct h3_stream_state {
    StagingSlot slots[kStagingSlots];
};

void h3_streaming_destroy(h3_gpu *g) {
    h3_stream_state *ring = g->streaming;
    if (!ring) return;
    for (StagingSlot &s : ring->slots) {
        if (s.armed) hipEventSynchronize(s.drained);
        if (s.drained) hipEventDestroy(s.drained);
        if (s.host) hipHostFree(s.host);
    }
    delete ring;
    g->streaming = nullptr;
}

static h3_stream_state *staging_ring(h3_gpu *g) {
    if (g->streaming) return g->streaming;
    std::unique_ptr<h3_stream_state> ring(new (std::nothrow) h3_stream_state());
    if (!ring) { h3_set_error(g, "streaming: out of host memory"); return nullptr; }
    for (StagingSlot &s : ring->slots) {
        bool ok = h3_hip_check(g, hipHostMalloc(&s.host, kStagingSlotBytes, hipHostMallocDefault), "pinned staging slot") &&
                  h3_hip_check(g, hipEventCreateWithFlags(&s.drained, hipEventDisableTiming), "staging slot event");
        if (!ok) {
            g->streaming = ring.release();
            h3_streaming_destroy(g);
            return nullptr;
        }
    }
    g->stats.pinned_bytes += kStagingSlots * kStagingSlotBytes;
    g->stats.peak_pinned_bytes = std::max(g->stats.peak_pinned_bytes, g->stats.pinned_bytes);
    g->streaming = ring.release();
    return g->streaming;
}

int h3_tensor_events(h3_gpu *g, h3_gpu_tensor *t) {
    if (!t->ready && !h3_hip_check(g, hipEventCreateWithFlags(&t->ready, hipEventDisableTiming), "tensor ready event")) return 0;
    if (!t->released && !h3_hip_check(g, hipEventCreateWithFlags(&t->released, hipEventDisableTiming), "tensor release event")) return 0;
    return 1;
}

// Compute-side use of a possibly streamed tensor: wait for its fill, and
// remember that the fill after this one must wait for this use.
int h3_tensor_acquire(h3_gpu *g, const h3_gpu_tensor *ct) {
    auto *t = const_cast<h3_gpu_tensor *>(ct);
    if (t && t->ready_pending) {
        if (!h3_hip_check(g, hipStreamWaitEvent(g->compute, t->ready, 0), "wait streamed weight")) return 0;
        t->ready_pending = false;
    }
    return 1;
}
int h3_tensor_release(h3_gpu *g, const h3_gpu_tensor *ct) {
    auto *t = const_cast<h3_gpu_tensor *>(ct);
    if (t && t->released) {
        if (!h3_hip_check(g, hipEventRecord(t->released, g->compute), "record weight release")) return 0;
        t->release_recorded = true;
    }
    return 1;
}

static int fill_begin(h3_gpu *g, h3_gpu_tensor *t) {
    if (!h3_tensor_events(g, t)) return 0;
    if (t->release_recorded && !h3_hip_check(g, hipStreamWaitEvent(g->copy, t->released, 0), "stream slot release")) return 0;
    return 1;
}
static int fill_end(h3_gpu *g, h3_gpu_tensor *t) {
    if (!h3_hip_check(g, hipEventRecord(t->ready, g->copy), "weight ready event")) return 0;
    t->ready_pending = true;
    return 1;
}

namespace {
// One file range → device tensor transfer. Chunk c of the range lands in slot
// c % kStagingSlots. The reader thread owns the file and the slots' contents;
// the calling thread owns every HIP call that queues work. They meet on two
// counters under one mutex: `staged` (chunks read) and `queued` (chunks whose
// copy and drained event are on the copy stream).
class FileFill {
public:
    FileFill(h3_gpu *g, h3_stream_state *ring, int fd, uint64_t offset, size_t bytes)
        : g_(g), ring_(ring), fd_(fd), offset_(offset), bytes_(bytes),
          chunks_((bytes + kStagingSlotBytes - 1) / kStagingSlotBytes) {}

    // Runs the transfer into dst; returns 1, or 0 with g->error set.
    int run(char *dst, const char *path) {
        if (!chunks_) return 1;
        std::thread reader([this] { read_all(); });
        int ok = 1;
        for (size_t c = 0; c < chunks_ && ok; c++) {
            std::unique_lock<std::mutex> lock(mutex_);
            changed_.wait(lock, [&] { return staged_ > c || read_failed_; });
            if (staged_ <= c) {  // the reader stopped at chunk c
                ok = read_failed_hip_
                         ? h3_set_error(g_, "%s", hip_error_)
                         : h3_set_error(g_, "read weight %s at %llu: %s", path, (unsigned long long)failed_at_,
                                        read_errno_ ? strerror(read_errno_) : "unexpected EOF");
                break;
            }
            lock.unlock();
            StagingSlot &s = ring_->slots[c % kStagingSlots];
            const size_t at = c * kStagingSlotBytes, n = std::min(kStagingSlotBytes, bytes_ - at);
            ok = h3_hip_check(g_, hipMemcpyAsync(dst + at, s.host, n, hipMemcpyHostToDevice, g_->copy), "weight H2D") &&
                 h3_hip_check(g_, hipEventRecord(s.drained, g_->copy), "staging slot release");
            lock.lock();
            if (ok) { s.armed = true; queued_ = c + 1; }
            else stop_ = true;
            changed_.notify_all();
        }
        {
            std::lock_guard<std::mutex> lock(mutex_);
            stop_ = true;
            changed_.notify_all();
        }
        reader.join();
        return ok;
    }

private:
    void read_all() {
        for (size_t c = 0; c < chunks_; c++) {
            StagingSlot &s = ring_->slots[c % kStagingSlots];
            {
                // The slot's previous chunk of this transfer must be queued
                // before its drained event says anything about it.
                std::unique_lock<std::mutex> lock(mutex_);
                changed_.wait(lock, [&] { return stop_ || c < kStagingSlots || queued_ + kStagingSlots > c; });
                if (stop_) return;
            }
            if (s.armed) {
                if (hipEventQuery(s.drained) == hipErrorNotReady) stalls_++;
                hipError_t e = hipEventSynchronize(s.drained);
                if (e != hipSuccess) { fail(0, e, 0); return; }
            }
            const size_t at = c * kStagingSlotBytes, n = std::min(kStagingSlotBytes, bytes_ - at);
            size_t got = 0;
            while (got < n) {
                const ssize_t r = pread(fd_, (char *)s.host + got, n - got, (off_t)(offset_ + at + got));
                if (r > 0) { got += (size_t)r; continue; }
                if (r < 0 && errno == EINTR) continue;
                fail(r < 0 ? errno : 0, hipSuccess, offset_ + at + got);
                return;
            }
            std::lock_guard<std::mutex> lock(mutex_);
            staged_ = c + 1;
            changed_.notify_all();
        }
    }

    void fail(int err, hipError_t e, uint64_t where) {
        std::lock_guard<std::mutex> lock(mutex_);
        read_failed_ = true;
        read_errno_ = err;
        failed_at_ = where;
        if (e != hipSuccess) {
            read_failed_hip_ = true;
            snprintf(hip_error_, sizeof(hip_error_), "staging slot reuse: %s", hipGetErrorString(e));
        }
        changed_.notify_all();
    }

public:
    uint64_t stalls_ = 0;

private:
    h3_gpu *g_;
    h3_stream_state *ring_;
    int fd_;
    uint64_t offset_;
    size_t bytes_, chunks_;
    std::mutex mutex_;
    std::condition_variable changed_;
    size_t staged_ = 0, queued_ = 0;
    bool stop_ = false, read_failed_ = false, read_failed_hip_ = false;
    int read_errno_ = 0;
    uint64_t failed_at_ = 0;
    char hip_error_[160] = {};
};
}  // namespace

// Fills the first n elements of t from path at offset. On failure the message
// is left in g->error and copied to error[error_size] when that is another buffer.
static int file_into(h3_gpu_tensor *t, const char *path, uint64_t offset, size_t n, h3_gpu_dtype dtype,
                     bool streaming, char *error, size_t error_size) {
    if (!t || !path || t->dtype != dtype || t->q8 || n > t->elements) return 0;
    h3_gpu *g = t->owner;
    const size_t bytes = n * item_size(dtype);
    if (offset > (uint64_t)INT64_MAX - bytes) return h3_set_error(g, "read weight %s: range overflows", path);
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        if (error && error_size) snprintf(error, error_size, "%s: %s", path, strerror(errno));
        return 0;
    }
    const double started = now_seconds();
    int ok;
    {
        std::lock_guard<std::mutex> lock(g->copy_mutex);
        h3_stream_state *ring = staging_ring(g);
        ok = ring && fill_begin(g, t);
        if (ok) {
            FileFill fill(g, ring, fd, offset, bytes);
            ok = fill.run((char *)t->data, path);
            g->stats.stream_stalls += fill.stalls_;
        }
        if (ok) ok = fill_end(g, t);
        g->stats.h2d_bytes += bytes;
        if (streaming) g->stats.streamed_bytes += bytes;
        g->stats.transfer_seconds += now_seconds() - started;
    }
    close(fd);
    if (!ok && error && error_size && error != g->error) snprintf(error, error_size, "%s", g->error);
    return ok;
}

extern "C" int h3_gpu_tensor_read_file_bf16(h3_gpu_tensor *t, const char *p, uint64_t off, size_t n, char *e, size_t s) {
    return file_into(t, p, off, n, H3_GPU_BF16, false, e, s);
}
extern "C" int h3_gpu_tensor_stream_file_bf16(h3_gpu_tensor *t, const char *p, uint64_t off, size_t n, char *e, size_t s) {
    return file_into(t, p, off, n, H3_GPU_BF16, true, e, s);
}

// gpu.h:220-224 (src/cuda/gpu_cuda.cu:843-846): a new device tensor filled from a file.
static h3_gpu_tensor *load_file(h3_gpu *g, const char *path, uint64_t offset, size_t n, h3_gpu_dtype dtype) {
    h3_gpu_tensor *t = h3_gpu_tensor_alloc(g, n, dtype, H3_GPU_DEVICE_ONLY);
    if (t && !file_into(t, path, offset, n, dtype, false, g->error, sizeof(g->error))) {
        h3_gpu_tensor_free(t);
        t = nullptr;
    }
    return t;
}
extern "C" h3_gpu_tensor *h3_gpu_tensor_load_bf16(h3_gpu *g, const char *p, uint64_t off, size_t n) {
    return load_file(g, p, off, n, H3_GPU_BF16);
}
extern "C" h3_gpu_tensor *h3_gpu_tensor_load_f32(h3_gpu *g, const char *p, uint64_t off, size_t n) {
    return load_file(g, p, off, n, H3_GPU_F32);
}
// Tensors here are always device (or pinned) allocations, never file mappings.
extern "C" int h3_gpu_tensor_is_file_mapped(const h3_gpu_tensor *t) { (void)t; return 0; }

// gpu.h:333-338 (src/cuda/gpu_cuda.cu:847-856): ordered device-to-device copy on the compute stream.
static int copy_tensor(h3_gpu *g, h3_gpu_tensor *d, size_t dst, const h3_gpu_tensor *s, size_t src, size_t n,
                       h3_gpu_dtype dtype) {
    if (!h3_launch_ready(g)) return 0;
    if (!d || !s || d->dtype != dtype || s->dtype != dtype || d->q8 || s->q8 || dst > d->elements ||
        n > d->elements - dst || src > s->elements || n > s->elements - src)
        return h3_set_error(g, "tensor copy: dtype or range mismatch");
    if (!n) return 1;
    size_t z = item_size(dtype);
    g->stats.d2d_bytes += n * z;
    // Either side may be a streamed slot: wait for its fill, and make the
    // next fill of it wait for this copy.
    return h3_tensor_acquire(g, s) && h3_tensor_acquire(g, d) &&
           h3_hip_check(g, hipMemcpyAsync((char *)d->data + dst * z, (const char *)s->data + src * z, n * z,
                                          hipMemcpyDeviceToDevice, g->compute), "tensor D2D") &&
           h3_launch_status(g, "tensor D2D") && h3_tensor_release(g, s) && h3_tensor_release(g, d);
}
extern "C" int h3_gpu_copy_bf16(h3_gpu *g, h3_gpu_tensor *d, size_t dst, const h3_gpu_tensor *s, size_t src, size_t n) {
    return copy_tensor(g, d, dst, s, src, n, H3_GPU_BF16);
}
extern "C" int h3_gpu_copy_f32(h3_gpu *g, h3_gpu_tensor *d, size_t dst, const h3_gpu_tensor *s, size_t src, size_t n) {
    return copy_tensor(g, d, dst, s, src, n, H3_GPU_F32);
}

extern "C" void *h3_hip_host_alloc(h3_gpu *g, size_t bytes) {
    if (!g || !bytes) return nullptr;
    void *p = nullptr;
    if (!h3_hip_check(g, hipHostMalloc(&p, bytes, hipHostMallocDefault), "pinned host allocation")) return nullptr;
    g->stats.pinned_bytes += bytes;
    g->stats.peak_pinned_bytes = std::max(g->stats.peak_pinned_bytes, g->stats.pinned_bytes);
    return p;
}
extern "C" void h3_hip_host_free(h3_gpu *g, void *p, size_t bytes) {
    if (!p) return;
    if (g) { hipStreamSynchronize(g->copy); g->stats.pinned_bytes -= std::min<uint64_t>(g->stats.pinned_bytes, bytes); }
    hipHostFree(p);
}

// Asynchronous fill of a device tensor (plain or q8) from pinned host memory on
// the copy stream. For a q8 weight, src holds codes followed by fp32 scales in
// the h3_hip_q8_from_packed layout.
extern "C" int h3_hip_tensor_stream_host(h3_gpu_tensor *t, const void *src, size_t bytes) {
    if (!t || !src) return 0;
    h3_gpu *g = t->owner;
    std::lock_guard<std::mutex> lock(g->copy_mutex);
    size_t code_bytes = t->bytes, scale_bytes = 0;
    if (t->q8) scale_bytes = (size_t)t->q8_rows * ((t->q8_cols + t->q8_group - 1) / t->q8_group) * 4;
    if (bytes != code_bytes + scale_bytes) return h3_set_error(g, "stream host: %zu bytes, tensor holds %zu", bytes, code_bytes + scale_bytes);
    double started = now_seconds();
    int ok = fill_begin(g, t) &&
             h3_hip_check(g, hipMemcpyAsync(t->data, src, code_bytes, hipMemcpyHostToDevice, g->copy), "stream H2D") &&
             (!scale_bytes || h3_hip_check(g, hipMemcpyAsync(t->q8_scales, (const char *)src + code_bytes, scale_bytes, hipMemcpyHostToDevice, g->copy), "stream scales H2D")) &&
             fill_end(g, t);
    g->stats.h2d_bytes += bytes; g->stats.streamed_bytes += bytes;
    g->stats.transfer_seconds += now_seconds() - started;
    return ok;
}

// Raw device contents of any tensor (parity tests read int8 / fp8 codes).
extern "C" int h3_hip_tensor_read_bytes(const h3_gpu_tensor *t, void *dst, size_t bytes) {
    if (!t || !dst) return 0;
    return read_bytes(t, 0, dst, bytes);
}

int h3_buffer_reserve(h3_gpu *g, h3_device_buffer *b, size_t bytes, const char *what) {
    if (b->bytes >= bytes) return 1;
    if (b->ptr && !h3_hip_check(g, hipStreamSynchronize(g->compute), what)) return 0;
    h3_buffer_free(b);
    if (!h3_hip_check(g, hipMalloc(&b->ptr, bytes), what)) { b->ptr = nullptr; return 0; }
    b->bytes = bytes;
    return 1;
}

void h3_buffer_free(h3_device_buffer *b) {
    if (b->ptr) hipFree(b->ptr);
    b->ptr = nullptr; b->bytes = 0;
}

// ------------------------------------------------------------ kernel timing
hipEvent_t h3_kernel_timing_begin(h3_gpu *g) {
    if (!g->kernel_timing) return nullptr;
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    hipEventRecord(e, g->compute);
    return e;
}

void h3_kernel_timing_end(h3_gpu *g, hipEvent_t start) {
    if (!start) return;
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) { hipEventDestroy(start); return; }
    hipEventRecord(e, g->compute);
    if (!g->kernel_events) g->kernel_events = new std::vector<std::pair<hipEvent_t, hipEvent_t>>();
    g->kernel_events->emplace_back(start, e);
}

static void kernel_events_clear(h3_gpu *g) {
    if (!g->kernel_events) return;
    for (auto &p : *g->kernel_events) { hipEventDestroy(p.first); hipEventDestroy(p.second); }
    g->kernel_events->clear();
}

extern "C" int h3_hip_kernel_timing(h3_gpu *g, int enable) {
    if (!g) return 0;
    if (g->active) return h3_set_error(g, "kernel timing: cannot change inside begin/submit");
    kernel_events_clear(g);
    g->kernel_timing = enable != 0;
    return 1;
}

extern "C" int h3_hip_kernel_timing_read(h3_gpu *g, double *ms_total, uint64_t *launches) {
    if (!g || !ms_total || !launches) return 0;
    if (g->active) return h3_set_error(g, "kernel timing: read after submit");
    double total = 0;
    uint64_t n = 0;
    if (g->kernel_events) {
        for (auto &p : *g->kernel_events) {
            float ms = 0;
            if (!h3_hip_check(g, hipEventSynchronize(p.second), "kernel timing") ||
                !h3_hip_check(g, hipEventElapsedTime(&ms, p.first, p.second), "kernel timing"))
                return 0;
            total += ms;
            n++;
        }
        kernel_events_clear(g);
    }
    *ms_total = total;
    *launches = n;
    return 1;
}
