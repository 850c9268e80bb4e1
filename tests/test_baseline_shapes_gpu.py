"""Parity at BASELINE's own shapes (configs 2-4), through the C ABI.

The GPU runs each workload at its full size; the oracle checks sampled query
rows (all keys, all 40 heads) or sampled GEMM rows, including the ragged tail
of the sequence (rows 32256-32399: the last 128-query workgroup holds 80 rows,
the last 64-key tile 16 keys).
- config 2: BF16 attention S=32400 H=40, 0.5 N(0,1) with the 3D RoPE, against
  the FP32 online-softmax oracle and a direct FP64 softmax;
- config 3: the Sage quantizers bit-exact over the whole tensor, and Sage
  attention on sampled rows against both the BF16 oracle and attention over
  the same quantized operands;
- config 4: the four W8A16 GEMMs at M=32400, K=5120/13824, per-output-channel
  scales, GELU-tanh on the up projection, against FP64 on 256 rows."""
import math

import numpy as np
import pytest

from h3cli_amd import synth
from h3cli_amd.runtime import Gpu, Tensor
from oracle import oracle
from tests.helpers import ATTN_COSINE, ATTN_MAX_ABS, GEMM_REL_L2, bf16, metrics, scale_bf16
from tests.test_block_gpu import ulp_diff

pytestmark = pytest.mark.gpu

SEQ, HEADS, DIM = 32400, 40, 128
N = SEQ * HEADS * DIM
ROPE_SHAPE = (27, 30, 40)
# Sampled query rows: the start, three interior slices, the start of the last
# workgroup and the ragged tail up to the last row.
ROW_RANGES = [(0, 16), (8000, 16 + 8000), (16190, 16206), (24001, 24017), (32256, 32272), (32384, 32400)]


def device_inputs(gpu, seed, scale, rope=False, k_bias=False):
    """Q, K, V filled on the device with the documented generator (seed*16+i),
    then prepared on the host: RoPE on Q and K (config 2) or +4.0 on 1% of K's
    channels per head (config 3). Returns device tensors and host BF16 bits."""
    lib = gpu.lib
    ts = [gpu.empty(N) for _ in range(3)]
    gpu.begin()
    for i, t in enumerate(ts):
        gpu.check(lib.h3_hip_fill_normal_bf16(gpu.handle, t.handle, seed * 16 + i, scale, N), "fill")
    gpu.submit()
    host = [t.read() for t in ts]
    if rope or k_bias:
        q = bf16(host[0]).reshape(SEQ, HEADS, DIM)
        k = bf16(host[1]).reshape(SEQ, HEADS, DIM)
        if rope:
            cos, sin = synth.rope_tables(*ROPE_SHAPE)
            q, k = synth.apply_rope(q, cos, sin), synth.apply_rope(k, cos, sin)
        if k_bias:
            rng = np.random.default_rng(seed)
            for h in range(HEADS):
                k[:, h, rng.choice(DIM, size=max(1, round(0.01 * DIM)), replace=False)] += 4.0
        for i, a in ((0, q), (1, k)):
            host[i] = synth.f32_to_bf16(a.reshape(-1))
            gpu.check(lib.h3_gpu_tensor_write_bf16(ts[i].handle, host[i].ctypes.data, N), "upload")
    return ts, host


def run_attention(gpu, ts):
    out = gpu.empty(N)
    gpu.begin()
    gpu.check(gpu.lib.h3_gpu_dit_sdpa_bf16(gpu.handle, out.handle, ts[0].handle, ts[1].handle, ts[2].handle, SEQ,
                                           HEADS, DIM, 1 / math.sqrt(DIM), 0, 0, 0), "sdpa")
    gpu.submit()
    return bf16(out.read()).reshape(SEQ, HEADS, DIM)


def test_config2_bf16_attention_full_shape():
    print(f"[config 2] S={SEQ} H={HEADS}: BF16 attention, sampled rows {ROW_RANGES}", flush=True)
    with Gpu() as gpu:
        ts, host = device_inputs(gpu, seed=2, scale=0.5, rope=True)
        got = run_attention(gpu, ts)
    assert np.all(np.isfinite(got))
    q, k, v = (bf16(a) for a in host)
    scale = scale_bf16(1 / math.sqrt(DIM))
    for r0, r1 in ROW_RANGES:
        ref = oracle.attention(q, k, v, SEQ, HEADS, scale, tile=64, rows=(r0, r1))
        m = metrics(got[r0:r1], ref)
        assert m["max_abs"] <= ATTN_MAX_ABS and m["cosine"] >= ATTN_COSINE, (r0, m)
        ref64 = oracle.attention_f64(q, k, v, SEQ, HEADS, scale, rows=(r0, r1))
        m64 = metrics(got[r0:r1], ref64)
        assert m64["max_abs"] <= ATTN_MAX_ABS and m64["cosine"] >= ATTN_COSINE, (r0, m64)
        # Every head of the slice on its own, too.
        for h in range(HEADS):
            mh = metrics(got[r0:r1, h], ref64[:, h])
            assert mh["cosine"] >= ATTN_COSINE, (r0, h, mh)


def test_config3_sage_full_shape():
    print(f"[config 3] S={SEQ} H={HEADS}: Sage pack (all heads) and sampled rows", flush=True)
    from tests.test_sage_gpu import gpu_pack
    with Gpu() as gpu:
        gpu.check(gpu.lib.h3_gpu_dit_attention_configure(gpu.handle, 1), "configure sage2++")
        ts, host = device_inputs(gpu, seed=3, scale=1.0, k_bias=True)
        got = run_attention(gpu, ts)
        for t in ts:
            gpu.free(t)
        pack = gpu_pack(gpu, *host, SEQ, HEADS)
    ref_pack = oracle.sage_pack(*host, SEQ, HEADS)
    for name in ("k_mean", "q_scale", "k_scale", "v_scale"):
        a, b = pack[name], ref_pack[name]
        view = np.uint32 if a.dtype == np.float32 else np.uint16
        assert np.array_equal(a.view(view), b.view(view)), name
    for name in ("q8", "k8", "v8"):
        diff = np.flatnonzero(pack[name] != ref_pack[name])
        assert diff.size == 0, (name, diff[:8])
    assert np.all(np.isfinite(got))
    q, k, v = (bf16(a) for a in host)
    scale = scale_bf16(1 / math.sqrt(DIM))
    for r0, r1 in ROW_RANGES:
        ref = oracle.attention(q, k, v, SEQ, HEADS, scale, tile=64, rows=(r0, r1))
        m = metrics(got[r0:r1], ref)
        assert m["max_abs"] <= ATTN_MAX_ABS and m["cosine"] >= ATTN_COSINE, (r0, m)
        mq = metrics(got[r0:r1], oracle.sage_attention(ref_pack, SEQ, HEADS, scale, rows=(r0, r1)))
        assert mq["max_abs"] <= ATTN_MAX_ABS and mq["cosine"] >= 0.9995, (r0, mq)


GEMM_SHAPES = [("qkv", 5120, 15360, False), ("out", 5120, 5120, False), ("up_gelu", 5120, 13824, True),
               ("down", 13824, 5120, False)]
GEMM_ROWS = [(0, 64), (10000, 10064), (20031, 20095), (32336, 32400)]


@pytest.mark.parametrize("name,k,n,gelu", GEMM_SHAPES)
def test_config4_w8a16_full_shape(name, k, n, gelu):
    m_rows = 32400
    print(f"[config 4] {name}: M={m_rows} K={k} N={n} gelu={gelu}", flush=True)
    rng = np.random.default_rng(40 + k + n)
    codes = rng.integers(-127, 128, size=n * k, dtype=np.int8)
    scales = rng.uniform(1e-3, 1e-2, size=n).astype(np.float32)
    with Gpu() as gpu:
        lib = gpu.lib
        x = gpu.empty(m_rows * k)
        gpu.begin()
        gpu.check(lib.h3_hip_fill_normal_bf16(gpu.handle, x.handle, 4 * 16 + k, 1.0, m_rows * k), "fill")
        gpu.submit()
        h = lib.h3_hip_q8_from_packed(gpu.handle, codes.ctypes.data, scales.ctypes.data, n, k, k)
        gpu.check(h, "q8 weight")
        w = Tensor(gpu, h, n * k, 2)
        gpu.tensors.append(w)
        y = gpu.empty(m_rows * n)
        fn = lib.h3_hip_linear_gelu_bf16 if gelu else lib.h3_gpu_linear_bf16
        gpu.begin()
        gpu.check(fn(gpu.handle, y.handle, x.handle, w.handle, None, m_rows, k, n), "linear")
        gpu.submit()
        xs = x.read().reshape(m_rows, k)
        ys = y.read().reshape(m_rows, n)
    assert np.all(np.isfinite(bf16(ys)))
    for r0, r1 in GEMM_ROWS:
        xr = np.ascontiguousarray(xs[r0:r1])
        ref, ref64 = oracle.linear_q8(xr, codes, scales, r1 - r0, k, n, k, gelu=gelu)
        met = metrics(bf16(ys[r0:r1]), ref64)
        # BASELINE gate rel-L2 <= 1e-2; the reference's own q8 gate is 0.006
        # (tests/metal_q8.c:156).
        assert met["rel_l2"] < 0.006 and met["rel_l2"] <= GEMM_REL_L2, (r0, met)
        # Each output rounds to BF16 once: within one BF16 step of the FP64
        # value's rounding almost everywhere.
        same = np.mean(ulp_diff(ys[r0:r1].reshape(-1), ref) <= 1)
        assert same > 0.99, (r0, same)
