"""Shared helpers of the parity tests: metrics, tolerances and C-ABI drivers."""
import math

import numpy as np

from h3cli_amd import synth

# BASELINE tolerances (north star): attention vs an fp32-accumulate reference.
ATTN_MAX_ABS = 2e-2
ATTN_COSINE = 0.999
GEMM_REL_L2 = 1e-2


def metrics(actual, expected):
    a = np.asarray(actual, np.float64).reshape(-1)
    e = np.asarray(expected, np.float64).reshape(-1)
    d = a - e
    norm = float(np.dot(e, e))
    return dict(
        max_abs=float(np.max(np.abs(d))) if d.size else 0.0,
        rel_l2=math.sqrt(float(np.dot(d, d)) / max(norm, 1e-30)),
        cosine=float(np.dot(a, e)) / math.sqrt(max(float(np.dot(a, a)) * norm, 1e-300)),
    )


def bf16(x):
    return synth.bf16_to_f32(x)


def scale_bf16(scale):
    """The boundary rounds the softmax scale to BF16 (reference gpu_cuda.cu:1652-1654)."""
    return float(bf16(synth.f32_to_bf16(np.float32(scale))))


def sdpa(gpu, q, k, v, seq, heads, scale=None, head_major=False, dit=True, step=0, block=1):
    """Run the DiT attention entry point on bf16 arrays; returns bf16 bits
    shaped [seq, heads, 128] (head-major outputs are transposed back)."""
    lib = gpu.lib
    scale = 1.0 / math.sqrt(128.0) if scale is None else scale
    n = seq * heads * 128
    tq, tk, tv = gpu.from_bf16(q), gpu.from_bf16(k), gpu.from_bf16(v)
    out = gpu.empty(n)
    gpu.begin()
    if dit:
        ok = lib.h3_gpu_dit_sdpa_bf16(gpu.handle, out.handle, tq.handle, tk.handle, tv.handle, seq, heads, 128,
                                      scale, int(head_major), block, step)
    elif head_major:
        ok = lib.h3_gpu_sdpa_bf16_head_major_output(gpu.handle, out.handle, tq.handle, tk.handle, tv.handle,
                                                    seq, heads, 128, scale)
    else:
        ok = lib.h3_gpu_sdpa_bf16(gpu.handle, out.handle, tq.handle, tk.handle, tv.handle, seq, heads, 128, scale)
    if not ok:
        err = gpu.error()
        gpu.cancel()
        raise RuntimeError(err)
    gpu.submit()
    res = out.read()
    for t in (tq, tk, tv, out):
        gpu.free(t)
    res = res.reshape((heads, seq, 128) if head_major else (seq, heads, 128))
    return res.transpose(1, 0, 2).copy() if head_major else res
