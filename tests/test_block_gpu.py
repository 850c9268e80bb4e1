"""DiT block operators on the GPU vs the CPU oracle: BF16 and W8A16 projections,
fused GELU, AdaLN, gates, Q/K norm + RoPE, activations and Euler."""
import ctypes as C
import math
import os
import tempfile

import numpy as np
import pytest

from h3cli_amd import synth
from h3cli_amd.runtime import Gpu
from oracle import oracle
from tests.helpers import GEMM_REL_L2, bf16, metrics

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    g = Gpu()
    yield g
    g.close()


def ulp_diff(a, b, floor=2.0 ** -17):
    """|a - b| in units of the BF16 ulp at the larger magnitude of the pair, with
    the ulp floored at `floor`: outputs that cancel to near zero (fma(x, 1+scale,
    shift) with x*(1+scale) ~ -shift) inherit the absolute error of the O(1) terms,
    not the tiny ulp of the result."""
    fa, fb = bf16(a).astype(np.float64), bf16(b).astype(np.float64)
    mag = np.maximum(np.maximum(np.abs(fa), np.abs(fb)), 2.0 ** -126)
    ulp = np.maximum(2.0 ** (np.floor(np.log2(mag)) - 7), floor)
    return np.abs(fa - fb) / ulp


def run(gpu, fn, *args):
    gpu.begin()
    ok = fn(gpu.handle, *args)
    if not ok:
        err = gpu.error()
        gpu.cancel()
        raise RuntimeError(err)
    gpu.submit()


def q8_weight(gpu, codes, scales, n, k, group):
    c = np.ascontiguousarray(codes, np.int8)
    s = np.ascontiguousarray(scales, np.float32)
    h = gpu.lib.h3_hip_q8_from_packed(gpu.handle, c.ctypes.data, s.ctypes.data, n, k, group)
    assert h, gpu.error()
    from h3cli_amd.runtime import Tensor
    t = Tensor(gpu, h, n * k, 2)
    gpu.tensors.append(t)
    return t


def synthetic_q8(seed, n, k, group):
    """BASELINE config 4 weights: int8 uniform in [-127, 127], per-output-channel
    (group = k) or per-group fp32 scales uniform in [1e-3, 1e-2]."""
    rng = np.random.default_rng(seed)
    codes = rng.integers(-127, 128, size=n * k, dtype=np.int8)
    scales = rng.uniform(1e-3, 1e-2, size=n * ((k + group - 1) // group)).astype(np.float32)
    return codes, scales


@pytest.mark.parametrize("m,k,n,group,bias,gelu", [
    (300, 512, 256, 512, False, False),     # per-channel, ragged M
    (513, 1024, 512, 64, True, False),      # reference q8 recipe (group 64) + bias
    (256, 768, 768, 768, False, True),      # fused GELU-tanh epilogue
    (33, 256, 256, 256, False, False),      # M smaller than a tile
    (300, 1024, 512, 1024, True, False),    # hand-scheduled GEMM, bias epilogue
    (300, 1024, 512, 1024, True, True),     # hand-scheduled GEMM, bias + GELU-tanh epilogue
    (50, 100, 30, 100, True, False),        # unaligned shape: small-GEMM path
])
def test_w8a16_linear(gpu, m, k, n, group, bias, gelu):
    print(f"[w8a16] m={m} k={k} n={n} group={group} bias={bias} gelu={gelu}", flush=True)
    codes, scales = synthetic_q8(m + n, n, k, group)
    x = synth.normal_bf16(m * 3 + 1, m * k)
    b = synth.normal_bf16(7, n, scale=0.1) if bias else None
    w = q8_weight(gpu, codes, scales, n, k, group)
    tx, ty = gpu.from_bf16(x), gpu.empty(m * n)
    tb = gpu.from_bf16(b) if bias else None
    fn = gpu.lib.h3_hip_linear_gelu_bf16 if gelu else gpu.lib.h3_gpu_linear_bf16
    run(gpu, fn, ty.handle, tx.handle, w.handle, tb.handle if tb else None, m, k, n)
    got = ty.read()
    ref, ref64 = oracle.linear_q8(x, codes, scales, m, k, n, group, bias=b, gelu=gelu)
    met = metrics(bf16(got), ref64)
    assert met["rel_l2"] <= GEMM_REL_L2, met
    # Reference gate for its q8 kernel (tests/metal_q8.c:156).
    assert met["rel_l2"] < 0.006, met
    # Nearly every element equals the FP64 reference rounded to BF16.
    assert np.mean(ulp_diff(got, ref) <= 1) > 0.99


def test_bf16_linear_exact_pattern(gpu):
    """tests/quant_native.c:31-50 power-of-two pattern: the BF16 GEMM output must
    equal bf16(exact sum) bit for bit, for several row counts."""
    n, k = 256, 256
    j = np.arange(n)[:, None]
    c = np.arange(k)[None, :]
    w = synth.f32_to_bf16(np.ldexp(1.0, (j % 3) - 1 + (c // 16) % 3).astype(np.float32))
    for rows in (1, 17, 129, 300):
        r = np.arange(rows)[:, None]
        x = synth.f32_to_bf16((np.where(r % 2, -1.0, 1.0) * np.ldexp(1.0, (r % 3) - 1 + (c // 16) % 2)).astype(np.float32))
        tw, tx, ty = gpu.from_bf16(w), gpu.from_bf16(x), gpu.empty(rows * n)
        run(gpu, gpu.lib.h3_gpu_linear_bf16, ty.handle, tx.handle, tw.handle, None, rows, k, n)
        exact = synth.bf16_to_f32(x).astype(np.float64) @ synth.bf16_to_f32(w).astype(np.float64).T
        assert np.array_equal(ty.read(), synth.f32_to_bf16(exact.astype(np.float32)).reshape(-1)), rows


def test_bf16_linear_random(gpu):
    m, k, n = 700, 1024, 512
    x = synth.normal_bf16(1, m * k)
    w = synth.normal_bf16(2, n * k, scale=0.03)
    tw, tx, ty = gpu.from_bf16(w), gpu.from_bf16(x), gpu.empty(m * n)
    run(gpu, gpu.lib.h3_gpu_linear_bf16, ty.handle, tx.handle, tw.handle, None, m, k, n)
    _, ref64 = oracle.linear_bf16(x, w, m, k, n)
    assert metrics(bf16(ty.read()), ref64)["rel_l2"] < 5e-3


def test_q8_load_from_file(gpu):
    """h3_gpu_q8_load packs BF16 weights from a file with the reference recipe."""
    n, k, m = 256, 320, 40
    w = synth.normal_bf16(3, n * k, scale=0.125)
    with tempfile.NamedTemporaryFile(delete=False) as f:
        f.write(b"\0" * 6 + w.tobytes())
        path = f.name
    try:
        h = gpu.lib.h3_gpu_q8_load(gpu.handle, path.encode(), 6, n, k)
        assert h, gpu.error()
        from h3cli_amd.runtime import Tensor
        t = Tensor(gpu, h, n * k, 2)
        gpu.tensors.append(t)
        x = synth.normal_bf16(4, m * k)
        tx, ty = gpu.from_bf16(x), gpu.empty(m * n)
        run(gpu, gpu.lib.h3_gpu_linear_bf16, ty.handle, tx.handle, t.handle, None, m, k, n)
        codes, scales = oracle.q8_pack(w, n, k, 64)
        _, ref64 = oracle.linear_q8(x, codes, scales, m, k, n, 64)
        assert metrics(bf16(ty.read()), ref64)["rel_l2"] < 0.006
    finally:
        os.unlink(path)


def test_q8_load_device_pack_bit_exact(gpu):
    """The device packer of h3_gpu_q8_load gives the codes and scales of the
    reference recipe bit for bit (vs the oracle and the host h3_q8_pack_rows):
    exact half ties, an all-zero group, a ragged last group (200 columns =
    64+64+64+8), large and tiny magnitudes. A NaN weight is rejected."""
    import ctypes as C
    n, k = 67, 200
    rng = np.random.default_rng(8)
    w = rng.standard_normal((n, k)).astype(np.float32)
    w[0, :64] = 0.0                                    # all-zero group -> scale 1
    w[1, :64] = np.arange(64) - 31.5                   # ties after scaling by 127/amax
    w[2] *= 1e30
    w[3] *= 1e-30
    w[4, 192:] = [127, -127, 63.5, -63.5, 0.5, -0.5, 1.5, 2.5]
    wb = synth.f32_to_bf16(w).reshape(-1)
    with tempfile.NamedTemporaryFile(delete=False) as f:
        f.write(b"\0" * 10 + wb.tobytes())
        path = f.name
    try:
        h = gpu.lib.h3_gpu_q8_load(gpu.handle, path.encode(), 10, n, k)
        assert h, gpu.error()
        from h3cli_amd.runtime import Tensor
        t = Tensor(gpu, h, n * k, 2)
        gpu.tensors.append(t)
        groups = (k + 63) // 64
        raw = np.zeros(n * k + n * groups * 4, np.uint8)
        assert gpu.lib.h3_hip_tensor_copy_to_host(h, raw.ctypes.data, raw.size), gpu.error()
        codes, scales = raw[:n * k].view(np.int8), raw[n * k:].view(np.float32)
        ref_codes, ref_scales = oracle.q8_pack(wb, n, k, 64)
        assert np.array_equal(codes, ref_codes) and np.array_equal(scales.view(np.uint32), ref_scales.view(np.uint32))
        host_codes, host_scales = np.zeros(n * k, np.int8), np.zeros(n * groups, np.float32)
        gpu.lib.h3_q8_pack_rows.restype = C.c_int
        assert gpu.lib.h3_q8_pack_rows(C.c_void_p(wb.ctypes.data), C.c_void_p(host_codes.ctypes.data),
                                       C.c_void_p(host_scales.ctypes.data), C.c_uint32(n), C.c_uint32(k))
        assert np.array_equal(codes, host_codes) and np.array_equal(scales, host_scales)
        bad = wb.copy()
        bad[5 * k + 7] = 0x7FC0
        with open(path, "r+b") as f:
            f.seek(10)
            f.write(bad.tobytes())
        assert not gpu.lib.h3_gpu_q8_load(gpu.handle, path.encode(), 10, n, k)
        assert "non-finite" in gpu.error()
    finally:
        os.unlink(path)


def test_linear_contract_errors(gpu):
    w = gpu.from_bf16(np.zeros(256 * 256, np.uint16))
    x = gpu.from_bf16(np.zeros(4 * 256, np.uint16))
    y = gpu.empty(4 * 256)
    gpu.begin()
    assert not gpu.lib.h3_gpu_linear_bf16(gpu.handle, y.handle, x.handle, w.handle, None, 4, 256, 257)
    assert not gpu.lib.h3_gpu_linear_bf16(gpu.handle, x.handle, x.handle, w.handle, None, 4, 256, 256)
    gpu.submit()


def modulation(seed, rows_map, slots, width):
    return synth.normal_bf16(seed, rows_map * slots * width, scale=0.3)


@pytest.mark.parametrize("rows,width", [(37, 512), (300, 5120), (5, 8192)])
def test_adaln(gpu, rows, width):
    x = synth.normal_bf16(rows, rows * width, scale=2.0)
    w = synth.normal_bf16(9, width, scale=0.5)
    mod = modulation(11, 3, 6, width)
    rmap = (np.arange(rows) % 3).astype(np.uint32)
    tx, tw, tm, tr, ty = gpu.from_bf16(x), gpu.from_bf16(w), gpu.from_bf16(mod), gpu.from_u32(rmap), gpu.empty(rows * width)
    run(gpu, gpu.lib.h3_gpu_adaln_bf16, ty.handle, tx.handle, tw.handle, tm.handle, tr.handle, rows, width, 6, 0, 1,
        C.c_float(1e-6))
    ref = oracle.adaln(x, w, mod, rmap, rows, width, 6, 0, 1, 1e-6)
    d = ulp_diff(ty.read(), ref)
    assert d.max() <= 1 and d.mean() < 0.02


def test_gate_and_gate_adaln(gpu):
    rows, width = 129, 5120
    res = synth.normal_bf16(1, rows * width)
    br = synth.normal_bf16(2, rows * width)
    w = synth.normal_bf16(3, width, scale=0.5)
    mod = modulation(4, 2, 6, width)
    rmap = (np.arange(rows) >= 100).astype(np.uint32)
    t = {n: gpu.from_bf16(a) for n, a in (("res", res), ("br", br), ("w", w), ("mod", mod))}
    tr = gpu.from_u32(rmap)
    out, gated, norm = gpu.empty(rows * width), gpu.empty(rows * width), gpu.empty(rows * width)
    run(gpu, gpu.lib.h3_gpu_gate_bf16, out.handle, t["res"].handle, t["br"].handle, t["mod"].handle, tr.handle,
        rows, width, 6, 2)
    ref_gate = oracle.gate(res, br, mod, rmap, rows, width, 6, 2)
    assert np.array_equal(out.read(), ref_gate)
    run(gpu, gpu.lib.h3_gpu_gate_adaln_bf16, gated.handle, norm.handle, t["res"].handle, t["br"].handle,
        t["w"].handle, t["mod"].handle, t["mod"].handle, tr.handle, rows, width, 6, 2, 3, 4, C.c_float(1e-6))
    assert np.array_equal(gated.read(), ref_gate)
    ref_norm = oracle.adaln(ref_gate, w, mod, rmap, rows, width, 6, 3, 4, 1e-6)
    assert ulp_diff(norm.read(), ref_norm).max() <= 1


@pytest.mark.parametrize("grouped,norm,half,dim", [(0, False, 64, 128), (1, True, 48, 128), (0, True, 64, 128),
                                                   (1, False, 36, 72)])
def test_qkv_rope(gpu, grouped, norm, half, dim):
    seq, heads = 97, 5
    qkv = synth.normal_bf16(5, seq * heads * dim * 3)
    cos, sin = synth.rope_tables(27, 30, 40)
    cos = synth.f32_to_bf16(cos[:seq, :half].copy()).reshape(-1)
    sin = synth.f32_to_bf16(sin[:seq, :half].copy()).reshape(-1)
    qw = synth.normal_bf16(6, dim, scale=0.5) if norm else None
    kw = synth.normal_bf16(7, dim, scale=0.5) if norm else None
    tq, tk, tv = gpu.empty(seq * heads * dim), gpu.empty(seq * heads * dim), gpu.empty(seq * heads * dim)
    tin, tc, ts = gpu.from_bf16(qkv), gpu.from_bf16(cos), gpu.from_bf16(sin)
    tqw = gpu.from_bf16(qw) if norm else None
    tkw = gpu.from_bf16(kw) if norm else None
    fn = gpu.lib.h3_gpu_grouped_qkv_rope_bf16 if grouped else gpu.lib.h3_gpu_qkv_rope_bf16
    run(gpu, fn, tq.handle, tk.handle, tv.handle, tin.handle, tqw.handle if tqw else None,
        tkw.handle if tkw else None, tc.handle, ts.handle, seq, heads, dim, half, C.c_float(1e-6))
    rq, rk, rv = oracle.qkv_rope(qkv, qw, kw, cos, sin, seq, heads, dim, half, 1e-6, grouped)
    assert np.array_equal(tv.read(), rv)
    assert ulp_diff(tq.read(), rq).max() <= 1 and ulp_diff(tk.read(), rk).max() <= 1


def test_activations_and_euler(gpu):
    n = 100003
    x = synth.normal_bf16(1, n, scale=3.0)
    tx, ty = gpu.from_bf16(x), gpu.empty(n)
    for approx in (1, 0):
        run(gpu, gpu.lib.h3_gpu_gelu_bf16, ty.handle, tx.handle, n, approx)
        assert ulp_diff(ty.read(), oracle.gelu(x, bool(approx))).max() <= 1
    rows, width = 77, 640
    fused = synth.normal_bf16(2, rows * width * 2, scale=2.0)
    tf, to = gpu.from_bf16(fused), gpu.empty(rows * width)
    run(gpu, gpu.lib.h3_gpu_swiglu_bf16, to.handle, tf.handle, rows, width)
    assert ulp_diff(to.read(), oracle.swiglu(fused, rows, width)).max() <= 1
    sample = synth.normal(3, n + 10).astype(np.float32)
    last, prev = synth.normal_bf16(4, n), synth.normal_bf16(5, n)
    ts, tl, tp = gpu.from_f32(sample), gpu.from_bf16(last), gpu.from_bf16(prev)
    run(gpu, gpu.lib.h3_gpu_euler_bf16, ts.handle, C.c_size_t(7), tl.handle, tp.handle, n, C.c_float(-0.05),
        C.c_float(0.25))
    want = sample.copy()
    want[7:7 + n] = oracle.euler(sample[7:7 + n], last, prev, -0.05, 0.25)
    assert np.array_equal(ts.read(), want)


def test_adaln_offset_and_rms_norms(gpu):
    rows, width, off = 45, 1024, 3 * 1024 + 8
    x = synth.normal_bf16(21, off + rows * width, scale=2.0)
    w = synth.normal_bf16(22, width, scale=0.5)
    mod = modulation(23, 2, 6, width)
    rmap = (np.arange(rows) % 2).astype(np.uint32)
    tx, tw, tm, tr, ty = gpu.from_bf16(x), gpu.from_bf16(w), gpu.from_bf16(mod), gpu.from_u32(rmap), gpu.empty(rows * width)
    run(gpu, gpu.lib.h3_gpu_adaln_bf16_offset, ty.handle, tx.handle, off, tw.handle, tm.handle, tr.handle, rows, width,
        6, 3, 4, C.c_float(1e-6))
    ref = oracle.adaln(x[off:], w, mod, rmap, rows, width, 6, 3, 4, 1e-6)
    assert ulp_diff(ty.read(), ref).max() <= 1
    with pytest.raises(RuntimeError):  # offset not a multiple of 8
        run(gpu, gpu.lib.h3_gpu_adaln_bf16_offset, ty.handle, tx.handle, 3, tw.handle, tm.handle, tr.handle, rows,
            width, 6, 3, 4, C.c_float(1e-6))
    run(gpu, gpu.lib.h3_gpu_rms_norm_bf16, ty.handle, tx.handle, tw.handle, rows, width, C.c_float(1e-5))
    assert ulp_diff(ty.read(), oracle.rms_norm(x[:rows * width], w, rows, width, 1e-5)).max() <= 1
    seq, heads, dim = 131, 6, 128
    t = synth.normal_bf16(24, seq * heads * dim, scale=3.0)
    hw = synth.normal_bf16(25, dim, scale=0.5)
    tt, thw = gpu.from_bf16(t), gpu.from_bf16(hw)
    run(gpu, gpu.lib.h3_gpu_head_rms_norm_bf16, tt.handle, thw.handle, seq, heads, dim, C.c_float(1e-6))
    assert ulp_diff(tt.read(), oracle.head_rms_norm(t, hw, seq, heads, dim, 1e-6)).max() <= 1


def test_sub_silu_mul_copy(gpu):
    n = 70001
    a, b = synth.normal_bf16(31, n, scale=3.0), synth.normal_bf16(32, n, scale=3.0)
    ta, tb, to = gpu.from_bf16(a), gpu.from_bf16(b), gpu.empty(n)
    run(gpu, gpu.lib.h3_gpu_sub_bf16, to.handle, ta.handle, tb.handle, n)
    want = synth.f32_to_bf16(bf16(a) - bf16(b))  # one rounding of an exact FP32 difference
    assert np.array_equal(to.read(), want)
    run(gpu, gpu.lib.h3_gpu_silu_mul_bf16, to.handle, ta.handle, tb.handle, n)
    fa = bf16(a).astype(np.float64)
    ref = synth.f32_to_bf16((fa / (1 + np.exp(-fa)) * bf16(b)).astype(np.float32))
    assert ulp_diff(to.read(), ref).max() <= 1
    dst = gpu.empty(n + 100)
    run(gpu, gpu.lib.h3_gpu_copy_bf16, dst.handle, 100, ta.handle, 5, n - 5)
    assert np.array_equal(dst.read()[100:100 + n - 5], a[5:])
    with pytest.raises(RuntimeError):
        run(gpu, gpu.lib.h3_gpu_copy_bf16, dst.handle, 101, ta.handle, 0, n)  # destination range overflows


@pytest.mark.parametrize("m,k,n,mapped", [(33, 128, 320, False), (200, 48, 5120, False), (70, 100, 130, True)])
def test_patch_linear_bit_exact(gpu, m, k, n, mapped):
    """FP32 patch projection: bit-exact against the ordered-fma restatement."""
    rng = np.random.default_rng(m + k + n)
    x = rng.standard_normal(m * k).astype(np.float32)
    w = (rng.standard_normal(n * k) * 0.1).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    tx, tw, tb = gpu.from_f32(x), gpu.from_f32(w), gpu.from_f32(bias)
    if mapped:
        out_rows = m + 9
        rmap = rng.permutation(out_rows)[:m].astype(np.uint32)
        rmap[3] = out_rows + 4  # out-of-range entries are skipped
        tr = gpu.from_u32(rmap)
        zero = gpu.from_bf16(np.zeros(out_rows * n, np.uint16))
        run(gpu, gpu.lib.h3_gpu_patch_linear_bf16_map, zero.handle, tx.handle, tw.handle, tb.handle, tr.handle,
            out_rows, m, k, n)
        got = zero.read()
        want = oracle.patch_linear(x, w, bias, m, k, n, row_map=rmap, out_rows=out_rows)
    else:
        ty = gpu.empty(m * n)
        run(gpu, gpu.lib.h3_gpu_patch_linear_bf16, ty.handle, tx.handle, tw.handle, tb.handle, m, k, n)
        got = ty.read()
        want = oracle.patch_linear(x, w, bias, m, k, n)
    assert np.array_equal(got, want)


def test_tensor_load_files(gpu):
    vals = synth.normal(41, 1000).astype(np.float32)
    with tempfile.NamedTemporaryFile(delete=False) as f:
        f.write(b"\0" * 12 + vals.tobytes())
        path = f.name
    try:
        h = gpu.lib.h3_gpu_tensor_load_f32(gpu.handle, path.encode(), 12, 1000)
        assert h, gpu.error()
        from h3cli_amd.runtime import Tensor
        t = Tensor(gpu, h, 1000, 0)
        gpu.tensors.append(t)
        assert np.array_equal(t.read(), vals)
        assert not gpu.lib.h3_gpu_tensor_load_f32(gpu.handle, path.encode(), 12, 2000)  # short file
    finally:
        os.unlink(path)
