"""Pins of the CPU oracle against checks independent of its own formulas:
FP64 brute force, invariants, torch's float8 cast, closed forms, brute-force
enumeration and the reference's own known-answer cases."""
import math

import numpy as np
import pytest

from h3cli_amd import synth
from oracle import oracle
from tests.helpers import bf16, metrics

torch = pytest.importorskip("torch")


def test_attention_matches_f64_bruteforce():
    seq, heads = 300, 3
    q, k, v = (bf16(a) for a in synth.attention_inputs(seq, heads, seed=1, scale=1.0))
    scale = 1 / math.sqrt(128)
    got = oracle.attention(q, k, v, seq, heads, scale, tile=64)
    ref = oracle.attention_f64(q, k, v, seq, heads, scale)
    m = metrics(got, ref)
    assert m["max_abs"] < 1e-5 and m["rel_l2"] < 1e-5, m


def test_attention_matches_torch_sdpa():
    """Against the textbook routine (torch's math SDPA in float64)."""
    seq, heads = 257, 2
    q, k, v = (bf16(a).reshape(seq, heads, 128) for a in synth.attention_inputs(seq, heads, seed=2))
    scale = 0.0883
    got = oracle.attention(q, k, v, seq, heads, scale, tile=16)
    t = lambda a: torch.from_numpy(a.astype(np.float64)).permute(1, 0, 2)
    ref = torch.softmax(t(q) @ t(k).transpose(1, 2) * scale, -1) @ t(v)
    m = metrics(got, ref.permute(1, 0, 2).numpy())
    assert m["max_abs"] < 1e-5, m


def test_attention_tile_size_and_invariants():
    seq, heads = 130, 2
    q, k, v = (bf16(a) for a in synth.attention_inputs(seq, heads, seed=3))
    scale = 0.1
    a = oracle.attention(q, k, v, seq, heads, scale, tile=16)
    b = oracle.attention(q, k, v, seq, heads, scale, tile=64)
    assert metrics(a, b)["max_abs"] < 1e-5
    c = np.full_like(v, 0.75)
    assert np.allclose(oracle.attention(q, k, c, seq, heads, scale), 0.75, atol=1e-6)
    z = np.zeros_like(q)
    assert np.all(oracle.attention(z, z, z, seq, heads, scale) == 0)
    # Permuting heads permutes outputs.
    perm = [1, 0]
    qp, kp, vp = (x.reshape(seq, heads, 128)[:, perm].copy() for x in (q, k, v))
    assert np.array_equal(oracle.attention(qp, kp, vp, seq, heads, scale, tile=16), a.reshape(seq, heads, 128)[:, perm])


def test_masked_attention_equals_dense_on_full_mask_and_bruteforce():
    seq, heads = 300, 2
    q, k, v = (bf16(a) for a in synth.attention_inputs(seq, heads, seed=4))
    blocks = (seq + 127) // 128
    full = np.ones((blocks, blocks), np.uint8)
    a = oracle.attention(q, k, v, seq, heads, 0.1, tile=128)
    b = oracle.attention(q, k, v, seq, heads, 0.1, mask=full, block=128)
    assert metrics(a, b)["max_abs"] < 1e-6
    # Brute force: masked keys get -inf in an FP64 softmax.
    mask = np.array([[1, 0, 1], [0, 1, 0], [1, 1, 0]], np.uint8)
    got = oracle.attention(q, k, v, seq, heads, 0.1, mask=mask, block=128)
    qq, kk, vv = (x.reshape(seq, heads, 128).astype(np.float64) for x in (q, k, v))
    s = np.einsum("qhd,khd->hqk", qq, kk) * 0.1
    allow = mask[np.arange(seq)[:, None] // 128, np.arange(seq)[None, :] // 128].astype(bool)
    s[:, ~allow] = -np.inf
    p = np.exp(s - s.max(-1, keepdims=True))
    ref = np.einsum("hqk,khd->qhd", p / p.sum(-1, keepdims=True), vv)
    assert metrics(got, ref)["max_abs"] < 1e-5


def test_e4m3_encoder_matches_torch_cast():
    """The brute-force e4m3 encoder equals torch's float8_e4m3fn cast (RNE) for
    every in-range value class: all codes, midpoints, subnormals, random values."""
    codes = np.arange(0x7F, dtype=np.uint8)
    vals = oracle.e4m3_decode(codes)
    mids = (vals[:-1] + vals[1:]) / 2
    rng = np.random.default_rng(0)
    rand = rng.uniform(-448, 448, 2000).astype(np.float32)
    tiny = rng.uniform(-0.02, 0.02, 500).astype(np.float32)
    xs = np.concatenate([vals, -vals, mids, -mids, rand, tiny, np.float32([448.0, -448.0, 1e-9, 0.0])])
    ref = torch.from_numpy(xs).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = oracle.e4m3_encode(xs)
    bad = np.flatnonzero(got != ref)
    assert bad.size == 0, (xs[bad[:5]], got[bad[:5]], ref[bad[:5]])
    # Decoding agrees with torch as well.
    back = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(vals, back)


def test_e4m3_saturates_above_448():
    assert oracle.e4m3_encode([500.0, 463.9, 1e6])[0] == 0x7E
    assert oracle.e4m3_encode([463.9])[0] == 0x7E


def test_sage_pack_closed_forms():
    """Scale = fmaf(amax, 1/127, 1e-7); codes within one step of x/scale; a
    block's extreme value codes to +/-127; zero blocks code to 0 with scale 1e-7;
    K mean within one BF16 ulp of the FP64 mean; V codes are the nearest e4m3."""
    seq, heads = 200, 2
    n = seq * heads * 128
    q = synth.normal_bf16(1, n)
    k = synth.normal_bf16(2, n, scale=2.0)
    v = synth.normal_bf16(3, n)
    q[: heads * 128 * 64] = 0  # first 64-row block of Q is all zeros
    p = oracle.sage_pack(q, k, v, seq, heads)
    padded, blocks = 256, 4
    q3 = bf16(q).reshape(seq, heads, 128)
    assert np.all(p["q_scale"].reshape(heads, blocks)[:, 0] == np.float32(1e-7))
    for h in range(heads):
        for b in range(1, blocks):
            x = q3[b * 64:min(seq, b * 64 + 64), h]
            amax = np.float32(np.abs(x).max())
            # fmaf(amax, 1/127, 1e-7): the FP64 evaluation of the two FP32 terms is
            # exact here (48-bit product plus a term inside its 53-bit span), so one
            # rounding to FP32 gives the fused result.
            fused = np.float32(np.float64(amax) * np.float64(np.float32(1 / 127)) + np.float64(np.float32(1e-7)))
            assert p["q_scale"][h * blocks + b] == fused
            s = p["q_scale"][h * blocks + b]
            codes = p["q8"].reshape(heads, padded, 128)[h, b * 64:b * 64 + x.shape[0]]
            assert np.all(np.abs(codes - x / s) <= 0.5 + 1e-6)
            assert np.abs(codes).max() == 127
    m64 = oracle.k_mean_f64(k, seq, heads)
    mean = bf16(p["k_mean"]).astype(np.float64)
    assert np.all(np.abs(mean - m64) <= np.abs(m64) * 2.0 ** -7 + 1e-12)
    # V: decode(code) * v_scale approximates v; code is the nearest e4m3 of v * 448 / vmax.
    v3 = bf16(v).reshape(seq, heads, 128)
    vmax = np.abs(v3).max(0)
    assert np.array_equal(p["v_scale"].reshape(heads, 128), (vmax / np.float32(448)).astype(np.float32))
    pos = np.array([oracle.sage_v_position(j) for j in range(64)])
    assert sorted(pos) == list(range(64))
    v8 = p["v8"].reshape(heads, 128, padded)
    for h in range(heads):
        for j in (0, 17, 63, 64, 199):
            codes = v8[h, :, (j // 64) * 64 + pos[j % 64]]
            want = torch.from_numpy((v3[j, h] * (np.float32(448) / vmax[h])).astype(np.float32)).to(
                torch.float8_e4m3fn).view(torch.uint8).numpy()
            assert np.array_equal(codes, want)


def test_sage_attention_oracle_close_to_fp_reference():
    # Quantization error averages over keys: the BASELINE gate is met from a
    # few thousand keys on (max-abs falls roughly as 1/sqrt(seq)).
    seq, heads = 2048, 2
    q, k, v = synth.attention_inputs(seq, heads, seed=8, scale=1.0)
    p = oracle.sage_pack(q, k, v, seq, heads)
    a = oracle.sage_attention(p, seq, heads, 0.0884, rows=(0, 128))
    b = oracle.attention_f64(bf16(q), bf16(k), bf16(v), seq, heads, 0.0884, rows=(0, 128))
    m = metrics(a, b)
    assert m["cosine"] > 0.999 and m["max_abs"] < 2e-2, m


def test_reference_input_generator_known_values():
    """tests/cuda_attention.c:14-18 from seed 123: first values by hand."""
    st = np.array([123], np.uint32)
    out = oracle.xorshift_bf16(3, st)
    s = 123
    vals = []
    for _ in range(3):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        vals.append(((s % 4097) - 2048) / 1024.0)
    assert np.array_equal(out, synth.f32_to_bf16(np.float32(vals)))
    assert st[0] == s


def test_rms_norm_oracle_closed_form():
    rows, width = 9, 640
    x = synth.normal_bf16(1, rows * width, scale=2.0)
    w = synth.normal_bf16(2, width, scale=0.5)
    xf = synth.bf16_to_f32(x).astype(np.float64).reshape(rows, width)
    inv = 1 / np.sqrt((xf * xf).mean(axis=1, keepdims=True) + 1e-5)
    want = xf * inv * synth.bf16_to_f32(w).astype(np.float64)
    got = synth.bf16_to_f32(oracle.rms_norm(x, w, rows, width, 1e-5)).reshape(rows, width)
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -7 + 1e-30)
    # head RMSNorm is the same per (row, head) slice
    h = oracle.head_rms_norm(x, w[:128], rows * 5, 1, 128, 1e-5)
    assert np.array_equal(h, oracle.rms_norm(x, w[:128], rows * 5, 128, 1e-5))


def test_patch_linear_oracle_exact_and_mapped():
    m, k, n = 13, 40, 24
    rng = np.random.default_rng(0)
    # Small integers times powers of two: every partial sum is exact in FP32, so
    # the result is bf16 of the exact dot product in any order.
    x = (rng.integers(-8, 9, m * k) * 0.25).astype(np.float32)
    w = (rng.integers(-8, 9, n * k) * 0.5).astype(np.float32)
    b = (rng.integers(-8, 9, n) * 1.0).astype(np.float32)
    exact = x.reshape(m, k).astype(np.float64) @ w.reshape(n, k).T.astype(np.float64) + b
    assert np.array_equal(oracle.patch_linear(x, w, b, m, k, n), synth.f32_to_bf16(exact.astype(np.float32)).reshape(-1))
    rmap = np.array([5, 0, 99] + list(range(6, 16)), np.uint32)
    got = oracle.patch_linear(x, w, b, m, k, n, row_map=rmap, out_rows=16).reshape(16, n)
    full = synth.f32_to_bf16(exact.astype(np.float32))
    assert np.array_equal(got[5], full[0]) and np.array_equal(got[0], full[1])
    assert not got[1:5].any()  # row 2 maps out of range and is skipped; rows 1-4 untouched
    xr = rng.standard_normal(m * k).astype(np.float32)
    wr = rng.standard_normal(n * k).astype(np.float32)
    ref = xr.reshape(m, k).astype(np.float64) @ wr.reshape(n, k).T.astype(np.float64)
    got = synth.bf16_to_f32(oracle.patch_linear(xr, wr, None, m, k, n)).reshape(m, n)
    assert np.max(np.abs(got - ref)) <= 2.0 ** -7 * np.abs(ref).max()


def _ulps(got_bits, want):
    g = synth.bf16_to_f32(got_bits).astype(np.float64)
    w = np.asarray(want, np.float64)
    mag = np.maximum(np.maximum(np.abs(g), np.abs(w)), 2.0 ** -126)
    return np.abs(g - w) / np.maximum(2.0 ** (np.floor(np.log2(mag)) - 7), 2.0 ** -17)


def test_elementwise_oracles_closed_forms():
    """AdaLN, gate, GELU, SwiGLU and Euler against FP64 numpy closed forms."""
    rows, width, slots = 7, 256, 6
    x = synth.normal_bf16(1, rows * width, scale=2.0)
    w = synth.normal_bf16(2, width, scale=0.5)
    mod = synth.normal_bf16(3, 2 * slots * width, scale=0.3)
    rmap = (np.arange(rows) % 2).astype(np.uint32)
    xf = bf16(x).astype(np.float64).reshape(rows, width)
    mf = bf16(mod).astype(np.float64).reshape(2, slots, width)[rmap]
    inv = 1 / np.sqrt((xf * xf).mean(1, keepdims=True) + 1e-6)
    want = xf * inv * bf16(w) * (1 + mf[:, 4]) + mf[:, 3]
    assert _ulps(oracle.adaln(x, w, mod, rmap, rows, width, slots, 3, 4, 1e-6), want.reshape(-1)).max() <= 1
    br = synth.normal_bf16(4, rows * width)
    want = xf + bf16(br).astype(np.float64).reshape(rows, width) * mf[:, 2]
    assert _ulps(oracle.gate(x, br, mod, rmap, rows, width, slots, 2), want.reshape(-1)).max() <= 0.5 + 1e-9
    g = np.linspace(-12, 12, 4001)
    gb = synth.f32_to_bf16(g.astype(np.float32))
    gf = bf16(gb).astype(np.float64)
    tanh_form = 0.5 * gf * (1 + np.tanh(0.7978845608028654 * (gf + 0.044715 * gf ** 3)))
    erf_form = 0.5 * gf * (1 + np.array([math.erf(t / math.sqrt(2)) for t in gf]))
    assert _ulps(oracle.gelu(gb, True), tanh_form).max() <= 1
    assert _ulps(oracle.gelu(gb, False), erf_form).max() <= 1
    fused = synth.normal_bf16(5, 2 * rows * width, scale=2.0)
    ff = bf16(fused).astype(np.float64).reshape(rows, 2, width)
    want = ff[:, 0] / (1 + np.exp(-ff[:, 0])) * ff[:, 1]
    assert _ulps(oracle.swiglu(fused, rows, width), want.reshape(-1)).max() <= 1
    sample = synth.normal(6, 1000).astype(np.float32)
    last, prev = synth.normal_bf16(7, 1000), synth.normal_bf16(8, 1000)
    lf, pf = bf16(last).astype(np.float64), bf16(prev).astype(np.float64)
    want = sample + (-0.05) * (lf + 0.25 * (lf - pf))
    assert np.max(np.abs(oracle.euler(sample, last, prev, -0.05, 0.25) - want)) <= 4e-7 * np.abs(want).max()


def test_qkv_rope_oracle_identities():
    """RoPE restatement: zero angle is the identity on Q/K, a rotation preserves
    each pair's norm and matches the FP64 rotate-half formula, V is copied, and
    the optional per-head RMSNorm matches its closed form."""
    seq, heads, dim, half = 5, 3, 128, 64
    qkv = synth.normal_bf16(9, seq * heads * dim * 3)
    ones = synth.f32_to_bf16(np.ones(seq * half, np.float32))
    zeros = np.zeros(seq * half, np.uint16)
    q, k, v = oracle.qkv_rope(qkv, None, None, ones, zeros, seq, heads, dim, half, 1e-6, 0)
    src = qkv.reshape(seq, 3, heads, dim)
    assert np.array_equal(q, src[:, 0].reshape(-1)) and np.array_equal(k, src[:, 1].reshape(-1))
    assert np.array_equal(v, src[:, 2].reshape(-1))
    ang = np.random.default_rng(1).uniform(-3, 3, (seq, half))
    cb, sb = synth.f32_to_bf16(np.cos(ang).astype(np.float32)), synth.f32_to_bf16(np.sin(ang).astype(np.float32))
    c, s = bf16(cb).astype(np.float64), bf16(sb).astype(np.float64)
    q, _, _ = oracle.qkv_rope(qkv, None, None, cb.reshape(-1), sb.reshape(-1), seq, heads, dim, half, 1e-6, 0)
    x = bf16(src[:, 0]).astype(np.float64)  # [seq, heads, dim]
    lo, hi = x[..., :half], x[..., half:]
    want = np.concatenate([lo * c[:, None] - hi * s[:, None], hi * c[:, None] + lo * s[:, None]], -1)
    assert _ulps(q, want.reshape(-1)).max() <= 1
    qw = synth.normal_bf16(10, dim, scale=0.5)
    q, _, _ = oracle.qkv_rope(qkv, qw, qw, ones, zeros, seq, heads, dim, half, 1e-6, 0)
    normed = x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6) * bf16(qw)
    assert _ulps(q, normed.reshape(-1)).max() <= 1
