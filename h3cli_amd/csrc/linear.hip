// Projection entry points of the operator surface: BF16 / W8A16 linear, the
// fused QKV projection + norm/RoPE, the SwiGLU MLP, and q8 weight tensors.
#include "common.h"
#include "internal.h"
#include <cerrno>
#include <cmath>
#include <fcntl.h>
#include <new>
#include <unistd.h>
#include <vector>

int h3_gemm(h3_gpu *g, uint16_t *y, const uint16_t *x, const h3_gpu_tensor *w, const uint16_t *bias, uint32_t m,
            uint32_t k, uint32_t n, int gelu);

static int linear(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in, const h3_gpu_tensor *w,
                  const h3_gpu_tensor *bias, uint32_t rows, uint32_t k, uint32_t n, int gelu) {
    if (!h3_launch_ready(g)) return 0;
    if (!rows || !k || !n || !w || w->owner != g)
        return h3_set_error(g, "linear %ux%ux%u: invalid shape or weight", rows, n, k);
    if (!h3_require(g, in, H3_GPU_BF16, (size_t)rows * k, "linear input") ||
        !h3_require(g, out, H3_GPU_BF16, (size_t)rows * n, "linear output") ||
        (bias && !h3_require(g, bias, H3_GPU_BF16, n, "linear bias")))
        return 0;
    if (w->quant_mode) {
        // Reference gpu_cuda.cu:928-930: packed FP8 weights take no bias or epilogue.
        if (bias || gelu) return h3_set_error(g, "unsupported quantized projection offset/bias/type");
        if (out == in) return h3_set_error(g, "linear: output aliases input");
        return h3_quant_gemm(g, out, in, w, rows, k, n);
    }
    if (w->q8) {
        if (w->q8_rows != n || w->q8_cols != k)
            return h3_set_error(g, "linear: q8 weight is %ux%u, need %ux%u", w->q8_rows, w->q8_cols, n, k);
    } else if (w->dtype != H3_GPU_BF16 || w->elements < (size_t)n * k) {
        return h3_set_error(g, "linear %ux%ux%u: weight must be BF16 with %zu elements", rows, n, k, (size_t)n * k);
    }
    if (out == in) return h3_set_error(g, "linear: output aliases input");
    return h3_gemm(g, (uint16_t *)out->data, (const uint16_t *)in->data, w,
                   bias ? (const uint16_t *)bias->data : nullptr, rows, k, n, gelu);
}

extern "C" int h3_gpu_linear_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in, const h3_gpu_tensor *w,
                                  const h3_gpu_tensor *bias, uint32_t rows, uint32_t k, uint32_t n) {
    return g && linear(g, out, in, w, bias, rows, k, n, 0);
}

extern "C" int h3_hip_linear_gelu_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in, const h3_gpu_tensor *w,
                                       const h3_gpu_tensor *bias, uint32_t rows, uint32_t k, uint32_t n) {
    return g && linear(g, out, in, w, bias, rows, k, n, 1);
}

extern "C" int h3_gpu_grouped_qkv_linear_rope_bf16(h3_gpu *g, h3_gpu_tensor *q, h3_gpu_tensor *k, h3_gpu_tensor *v,
                                                   h3_gpu_tensor *qkv, const h3_gpu_tensor *in, const h3_gpu_tensor *w,
                                                   const h3_gpu_tensor *qw, const h3_gpu_tensor *kw,
                                                   const h3_gpu_tensor *c, const h3_gpu_tensor *s, uint32_t rows,
                                                   uint32_t width, uint32_t heads, uint32_t dim, uint32_t half, float eps) {
    return g && h3_gpu_linear_bf16(g, qkv, in, w, nullptr, rows, width, heads * dim * 3) &&
           h3_gpu_grouped_qkv_rope_bf16(g, q, k, v, qkv, qw, kw, c, s, rows, heads, dim, half, eps);
}

// fc1 (2*hidden, gate rows then up rows) -> SwiGLU -> fc2, as src/cuda/gpu_cuda.cu:1108-1112.
extern "C" int h3_gpu_mlp_bf16(h3_gpu *g, h3_gpu_tensor *out, const h3_gpu_tensor *in, const h3_gpu_tensor *w1,
                               const h3_gpu_tensor *w2, uint32_t rows, uint32_t width, uint32_t hidden, uint32_t output_dim) {
    if (!g) return 0;
    h3_gpu_tensor *fused = h3_gpu_tensor_new_bf16(g, (size_t)rows * hidden * 2);
    h3_gpu_tensor *act = h3_gpu_tensor_new_bf16(g, (size_t)rows * hidden);
    int ok = fused && act && h3_gpu_linear_bf16(g, fused, in, w1, nullptr, rows, width, hidden * 2) &&
             h3_gpu_swiglu_bf16(g, act, fused, rows, hidden) &&
             h3_gpu_linear_bf16(g, out, act, w2, nullptr, rows, hidden, output_dim);
    h3_gpu_tensor_free(fused);
    h3_gpu_tensor_free(act);
    return ok;
}

// ------------------------------------------------------------------ q8 weights
static h3_gpu_tensor *q8_tensor(h3_gpu *g, uint32_t rows, uint32_t cols, uint32_t group) {
    if (!rows || !cols || !group || group > cols) { h3_set_error(g, "q8: invalid %ux%u group %u", rows, cols, group); return nullptr; }
    h3_gpu_tensor *t = h3_gpu_tensor_alloc(g, (size_t)rows * cols, H3_GPU_I8, H3_GPU_DEVICE_ONLY);
    if (!t) return nullptr;
    size_t groups = (cols + group - 1) / group, sbytes = (size_t)rows * groups * 4;
    if (!h3_hip_check(g, hipMalloc(&t->q8_scales, sbytes), "q8 scales")) { t->q8_scales = nullptr; h3_gpu_tensor_free(t); return nullptr; }
    t->q8 = 1; t->q8_rows = rows; t->q8_cols = cols; t->q8_group = group;
    g->stats.q8_weights++;
    g->stats.q8_storage_bytes += t->bytes + sbytes;
    return t;
}

extern "C" h3_gpu_tensor *h3_hip_q8_new(h3_gpu *g, uint32_t rows, uint32_t cols, uint32_t group) {
    return g ? q8_tensor(g, rows, cols, group) : nullptr;
}

extern "C" h3_gpu_tensor *h3_hip_q8_from_packed(h3_gpu *g, const int8_t *codes, const float *scales, uint32_t rows,
                                                uint32_t cols, uint32_t group) {
    if (!g || !codes || !scales) return nullptr;
    h3_gpu_tensor *t = q8_tensor(g, rows, cols, group);
    if (!t) return nullptr;
    size_t groups = (cols + group - 1) / group;
    if (!h3_hip_check(g, hipMemcpy(t->data, codes, (size_t)rows * cols, hipMemcpyHostToDevice), "q8 codes upload") ||
        !h3_hip_check(g, hipMemcpy(t->q8_scales, scales, (size_t)rows * groups * 4, hipMemcpyHostToDevice), "q8 scales upload")) {
        h3_gpu_tensor_free(t);
        return nullptr;
    }
    return t;
}

// Reference q8 packing (src/weights/q8.c:26-56), restated on the device: one
// thread per (row, 64-wide group): scale = max|w| / 127 (IEEE division; 1 for an
// all-zero group, floored at FLT_MIN), code = round-half-to-even(w / scale)
// clamped to +-127. Bit-identical to h3_q8_pack_rows. A non-finite weight sets
// bad[0] (the whole tensor is then rejected, as the reference does).
__global__ __launch_bounds__(256) void q8_pack_kernel(const uint16_t *src, int8_t *codes, float *scales, uint32_t rows,
                                                      uint32_t cols, uint32_t groups, unsigned *bad) {
    const size_t id = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= (size_t)rows * groups) return;
    const uint32_t r = (uint32_t)(id / groups), gi = (uint32_t)(id % groups);
    const uint32_t begin = gi * 64, end = min(begin + 64, cols);
    const uint16_t *row = src + (size_t)r * cols;
    float amax = 0.f;
    bool finite = true;
    for (uint32_t c = begin; c < end; c++) {
        const float w = bf16_to_f32(row[c]);
        finite &= finite_f32(w);
        amax = fmaxf(amax, fabsf(w));
    }
    if (!finite) { bad[0] = 1u; return; }
    const float scale = amax == 0.f ? 1.f : fmaxf(__fdiv_rn(amax, 127.f), 1.17549435e-38f);
    scales[id] = scale;
    int8_t *out = codes + (size_t)r * cols;
    for (uint32_t c = begin; c < end; c++) {
        const float q = rintf(__fdiv_rn(bf16_to_f32(row[c]), scale));
        out[c] = (int8_t)fminf(fmaxf(q, -127.f), 127.f);
    }
}

extern "C" int h3_q8_layout(uint32_t rows, uint32_t columns, size_t *offset, size_t *bytes);

// Reads rows x columns BF16 at `offset` of `path` and packs it on the device.
extern "C" h3_gpu_tensor *h3_gpu_q8_load(h3_gpu *g, const char *path, uint64_t offset, uint32_t rows, uint32_t columns) {
    if (!g || !path || !rows || !columns) return nullptr;
    size_t layout_offset, layout_bytes;
    if (!h3_q8_layout(rows, columns, &layout_offset, &layout_bytes)) {
        h3_set_error(g, "q8 load %s: invalid shape %ux%u", path, rows, columns);
        return nullptr;
    }
    const size_t n = (size_t)rows * columns, groups = (columns + 63) / 64;
    std::vector<uint16_t> src(n);
    int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) { h3_set_error(g, "q8 load %s: %s", path, strerror(errno)); return nullptr; }
    size_t got = 0;
    while (got < n * 2) {
        ssize_t r = pread(fd, (char *)src.data() + got, n * 2 - got, (off_t)(offset + got));
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) { close(fd); h3_set_error(g, "q8 load %s: short read", path); return nullptr; }
        got += (size_t)r;
    }
    close(fd);
    h3_gpu_tensor *t = q8_tensor(g, rows, columns, 64);
    if (!t) return nullptr;
    void *staging = nullptr;
    const size_t flag_at = (n * 2 + 255) & ~(size_t)255;
    unsigned bad = 0;
    bool ok = h3_hip_check(g, hipMalloc(&staging, flag_at + 4), "q8 load staging") &&
              h3_hip_check(g, hipMemcpy(staging, src.data(), n * 2, hipMemcpyHostToDevice), "q8 load upload") &&
              h3_hip_check(g, hipMemset((char *)staging + flag_at, 0, 4), "q8 load flag");
    if (ok) {
        const size_t threads = (size_t)rows * groups;
        hipLaunchKernelGGL(q8_pack_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, nullptr,
                           (const uint16_t *)staging, (int8_t *)t->data, (float *)t->q8_scales, rows, columns,
                           (uint32_t)groups, (unsigned *)((char *)staging + flag_at));
        ok = h3_hip_check(g, hipGetLastError(), "q8 pack") &&
             h3_hip_check(g, hipMemcpy(&bad, (char *)staging + flag_at, 4, hipMemcpyDeviceToHost), "q8 pack flag");
    }
    if (staging) hipFree(staging);
    if (ok && bad) { h3_set_error(g, "q8 load %s: non-finite weight or invalid shape", path); ok = false; }
    if (!ok) { h3_gpu_tensor_free(t); return nullptr; }
    g->stats.q8_source_bytes += n * 2;
    return t;
}
