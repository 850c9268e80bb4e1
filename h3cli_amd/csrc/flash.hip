// FlashAttention-2-style forward with log-sum-exp, on the stream-level
// interface of the reference's SGLang-parity path
// (src/cuda/cuda_sglang_flash.h:8-16, src/cuda/cuda_sglang_flash.cu:14-74):
// raw device pointers, a stream, 1 on success, 0 for arguments or shapes the
// backend does not take, -1 with a message when a launch fails.
//
// Both entries run the dense BF16 kernel of h3_gpu_sdpa_bf16 (sequence-major
// Q/K/V [seq, heads, 128], non-causal) and also write lse [batch, heads,
// query rows] = log sum_j exp(scale q.k_j) in FP32, FlashAttention's layout.
// The kernel needs a workspace (V transposed, retry bytes). Each device keeps
// one, grown only when a call needs more (the only allocation, after the last
// use of the old buffer has finished), and reused by every later call: a call
// first makes its stream wait for the previous call's last use of the buffer
// and records its own after its launches, so calls on different streams take
// the workspace in turn instead of racing on it.
//
// Taken: BF16, head dimension 128, heads == kv_heads, non-causal. The
// reference's other cases (causal text attention, the head-dimension-72
// vision and 64 VAE attention, grouped K/V heads) belong to components this
// backend does not provide and return 0 with a message.
#include "common.h"
#include "internal.h"
#include <cmath>
#include <cstdio>
#include <mutex>

namespace {

int refuse(char *error, size_t size, const char *what) {
    if (error && size) snprintf(error, size, "%s", what);
    return 0;
}

constexpr int MAX_DEVICES = 16;

// A device's reusable workspace and the event recorded after its last use.
struct DeviceWorkspace {
    std::mutex lock;
    void *ptr = nullptr;
    size_t bytes = 0;
    hipEvent_t last_use = nullptr;
};
DeviceWorkspace workspaces[MAX_DEVICES];

int fail(char *error, size_t size, const char *what, hipError_t e) {
    if (error && size) snprintf(error, size, "%s: %s", what, hipGetErrorString(e));
    return -1;
}

// One call on the device's workspace, under its lock: wait for the last use,
// grow if needed, launch, record this use.
int run(void *out, const void *q, const void *k, const void *v, float *lse, unsigned seq, unsigned qrows,
        unsigned heads, float scale, bool head_major, hipStream_t stream, char *error, size_t size) {
    h3_gpu g{};
    hipError_t e = hipGetDevice(&g.device);
    if (e != hipSuccess) return fail(error, size, "FlashAttention device", e);
    if (g.device < 0 || g.device >= MAX_DEVICES) return refuse(error, size, "FlashAttention: device ordinal out of range");
    g.compute = stream;
    DeviceWorkspace &w = workspaces[g.device];
    std::lock_guard<std::mutex> guard(w.lock);
    if (!w.last_use && (e = hipEventCreateWithFlags(&w.last_use, hipEventDisableTiming)) != hipSuccess) {
        w.last_use = nullptr;
        return fail(error, size, "FlashAttention workspace event", e);
    }
    // The kernels' non-finite flag goes to the 256 bytes after the workspace:
    // this interface reports no deferred faults, as the reference's does not.
    const size_t bytes = h3_attention_bf16_workspace(seq, heads) + 256;
    if (w.bytes < bytes) {
        if (w.ptr) {
            if ((e = hipEventSynchronize(w.last_use)) != hipSuccess) return fail(error, size, "FlashAttention workspace", e);
            (void)hipFree(w.ptr);
            w.ptr = nullptr;
            w.bytes = 0;
        }
        if ((e = hipMalloc(&w.ptr, bytes)) != hipSuccess) {
            w.ptr = nullptr;
            return fail(error, size, "FlashAttention workspace", e);
        }
        w.bytes = bytes;
    }
    if ((e = hipStreamWaitEvent(stream, w.last_use, 0)) != hipSuccess) return fail(error, size, "FlashAttention workspace", e);
    g.fault = reinterpret_cast<unsigned *>(static_cast<uint8_t *>(w.ptr) + bytes - 256);
    const int ok = h3_launch_attention_flash(&g, w.ptr, static_cast<uint16_t *>(out), static_cast<const uint16_t *>(q),
                                             static_cast<const uint16_t *>(k), static_cast<const uint16_t *>(v), lse,
                                             seq, qrows, heads, scale, head_major);
    if ((e = hipEventRecord(w.last_use, stream)) != hipSuccess) return fail(error, size, "FlashAttention workspace", e);
    if (!ok) {
        if (error && size) snprintf(error, size, "FlashAttention launch: %s", g.error);
        return -1;
    }
    return 1;
}

bool valid_scale(float scale) { return std::isfinite(scale) && scale > 0.f; }

}  // namespace

extern "C" int h3_sglang_flash(void *out, const void *q, const void *k, const void *v, float *lse, unsigned batch,
                               unsigned sequence, unsigned heads, unsigned kv_heads, unsigned dim, float scale,
                               int causal, int head_major_output, void *stream, char *error, size_t size) {
    if (!out || !q || !k || !v || !lse || !batch || !sequence || sequence > 1000000 || !heads || !kv_heads ||
        heads % kv_heads || !valid_scale(scale) || (head_major_output != 0 && head_major_output != 1))
        return 0;
    if (dim != 128 || causal || kv_heads != heads)
        return refuse(error, size, "FlashAttention: only non-causal BF16 D=128 with heads == kv_heads on the HIP backend");
    const size_t elems = (size_t)sequence * heads * 128;
    for (unsigned b = 0; b < batch; b++) {
        const int r = run(static_cast<uint16_t *>(out) + b * elems, static_cast<const uint16_t *>(q) + b * elems,
                          static_cast<const uint16_t *>(k) + b * elems, static_cast<const uint16_t *>(v) + b * elems,
                          lse + (size_t)b * heads * sequence, sequence, sequence, heads, scale, head_major_output != 0,
                          static_cast<hipStream_t>(stream), error, size);
        if (r != 1) return r;
    }
    return 1;
}

extern "C" int h3_sglang_flash_query_range(void *out, const void *q, const void *k, const void *v, float *lse,
                                           unsigned sequence, unsigned heads, unsigned first, unsigned count,
                                           float scale, int head_major_output, void *stream, char *error,
                                           size_t size) {
    if (!out || !q || !k || !v || !lse || !sequence || sequence > 1000000 || !heads || !count || first >= sequence ||
        count > sequence - first || !valid_scale(scale) || (head_major_output != 0 && head_major_output != 1))
        return 0;
    // Q rows and output rows start at `first`; the head-major output keeps the
    // full sequence as its head stride.
    const size_t q_off = (size_t)first * heads * 128;
    const size_t o_off = (size_t)first * (head_major_output ? 128 : (size_t)heads * 128);
    return run(static_cast<uint16_t *>(out) + o_off, static_cast<const uint16_t *>(q) + q_off, k, v, lse, sequence,
               count, heads, scale, head_major_output != 0, static_cast<hipStream_t>(stream), error, size);
}
