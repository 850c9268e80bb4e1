"""BF16 DiT attention on the GPU vs the CPU oracle (reference
src/cuda/cuda_attention.cuh:7-51 restated in oracle/attention.c), through the C ABI."""
import math

import numpy as np
import pytest

from h3cli_amd import synth
from h3cli_amd.runtime import Gpu
from oracle import oracle
from tests.helpers import ATTN_COSINE, ATTN_MAX_ABS, bf16, metrics, scale_bf16, sdpa

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    g = Gpu()
    yield g
    g.close()


def _check(gpu, q, k, v, seq, heads, head_major=False, dit=True, rows=None):
    print(f"[attention] seq={seq} heads={heads} head_major={head_major} dit={dit}", flush=True)
    out = sdpa(gpu, q, k, v, seq, heads, head_major=head_major, dit=dit)
    scale = scale_bf16(1 / math.sqrt(128))
    r0, r1 = rows if rows else (0, seq)
    ref = oracle.attention(bf16(q), bf16(k), bf16(v), seq, heads, scale, tile=64, rows=(r0, r1))
    got = bf16(out)[r0:r1]
    m = metrics(got, ref)
    assert np.all(np.isfinite(got))
    assert m["max_abs"] <= ATTN_MAX_ABS and m["cosine"] >= ATTN_COSINE, m
    return m


@pytest.mark.parametrize("seq,heads,head_major", [(19, 4, False), (513, 3, False), (1025, 4, True),
                                                  (2048, 8, False), (1, 2, False), (64, 1, False),
                                                  (65, 1, True), (300, 40, False)])
def test_reference_patterns(gpu, seq, heads, head_major):
    """Shapes and the xorshift input pattern of the reference's
    tests/cuda_attention.c:14-18,52 (D fixed at 128 on this path)."""
    st = np.array([123], np.uint32)
    n = seq * heads * 128
    q, k, v = (oracle.xorshift_bf16(n, st) for _ in range(3))
    m = _check(gpu, q, k, v, seq, heads, head_major)
    # The reference's own gate for its tiled kernel (tests/cuda_attention.c:43).
    assert m["max_abs"] < 0.016, m


@pytest.mark.parametrize("seq,heads", [(1000, 2), (4096, 4)])
def test_gaussian_rope_inputs(gpu, seq, heads):
    """BASELINE config 2 input distribution (0.5 N(0,1), 3D RoPE) at small S."""
    q, k, v = synth.attention_inputs(seq, heads, seed=2, scale=0.5, rope_shape=(27, 30, 40))
    _check(gpu, q, k, v, seq, heads)


def test_plain_entry_points(gpu):
    seq, heads = 700, 3
    q, k, v = synth.attention_inputs(seq, heads, seed=5)
    _check(gpu, q, k, v, seq, heads, dit=False)
    _check(gpu, q, k, v, seq, heads, head_major=True, dit=False)


def _growth_inputs(seq, heads, pattern):
    """Scores that rise across the keys (the running max is raised many times),
    fall (the first tile holds the max), or jump at one late key by more than
    128 in log2 units (its P overflows FP32 until the max is raised)."""
    rng = np.random.default_rng(21)
    n = seq * heads * 128
    one = np.float32(1.0)
    q = np.full((seq, heads, 128), one, np.float32)
    if pattern == "rise":
        k = np.repeat(np.linspace(0, 20, seq, dtype=np.float32)[:, None, None], heads, 1).repeat(128, 2)
    elif pattern == "fall":
        k = np.repeat(np.linspace(20, 0, seq, dtype=np.float32)[:, None, None], heads, 1).repeat(128, 2)
    else:
        k = rng.normal(0, 0.25, (seq, heads, 128)).astype(np.float32)
        k[seq - 100] = 8.0
    v = rng.normal(0, 1, (seq, heads, 128)).astype(np.float32)
    return tuple(synth.f32_to_bf16(x.reshape(n)) for x in (q, k, v))


@pytest.mark.parametrize("pattern", ["rise", "fall", "spike"])
def test_score_growth(gpu, pattern):
    """Large, moving score ranges: the lazily raised running max must keep every
    P finite and the result equal to the oracle's and to a direct FP64 softmax."""
    seq, heads = 1500, 2
    q, k, v = _growth_inputs(seq, heads, pattern)
    _check(gpu, q, k, v, seq, heads)
    out = bf16(sdpa(gpu, q, k, v, seq, heads))
    scale = scale_bf16(1 / math.sqrt(128))
    for r0 in (0, 700, seq - 10):
        ref = oracle.attention_f64(bf16(q), bf16(k), bf16(v), seq, heads, scale, rows=(r0, r0 + 10))
        m = metrics(out[r0:r0 + 10], ref)
        assert m["max_abs"] <= ATTN_MAX_ABS and m["cosine"] >= ATTN_COSINE, m


def test_recomputation_launch_matches_tile_max_kernel(gpu, monkeypatch):
    """A 130-log2-unit spike overflows P in every workgroup of the default
    kernel, so the recomputation launch redoes all rows with the per-tile-max
    kernel (attention variant 3): the two outputs agree bit for bit. A rising
    ramp, which only raises the max by exponent shifts, stays within tolerance
    of variant 3."""
    seq, heads = 1500, 2
    q, k, v = _growth_inputs(seq, heads, "spike")
    fast = sdpa(gpu, q, k, v, seq, heads)
    monkeypatch.setenv("H3_HIP_ATTENTION_VARIANT", "3")
    g3 = Gpu()
    try:
        assert np.array_equal(sdpa(g3, q, k, v, seq, heads), fast)
        q, k, v = _growth_inputs(seq, heads, "rise")
        m = metrics(bf16(sdpa(gpu, q, k, v, seq, heads)), bf16(sdpa(g3, q, k, v, seq, heads)))
        assert m["max_abs"] <= ATTN_MAX_ABS and m["cosine"] >= ATTN_COSINE, m
    finally:
        g3.close()


@pytest.mark.parametrize("seq,heads", [(4200, 2), (65, 3), (1, 1)])
def test_global_load_path_matches_buffer_path(gpu, monkeypatch, seq, heads):
    """K and V^T below 4 GiB load their tiles with buffer loads (keys past the
    sequence read as zeros); larger tensors take the global-load path (rows
    clamped to the last key), forced here with attention variant 13. Both
    mask the same keys, so the outputs agree bit for bit, ragged tails
    included."""
    q, k, v = synth.attention_inputs(seq, heads, seed=31, scale=0.5)
    buffered = sdpa(gpu, q, k, v, seq, heads)
    monkeypatch.setenv("H3_HIP_ATTENTION_VARIANT", "13")
    g13 = Gpu()
    try:
        assert np.array_equal(sdpa(g13, q, k, v, seq, heads), buffered)
    finally:
        g13.close()


@pytest.mark.parametrize("case", ["257x3", "300x40", "4200x2", "8191x2", "rise", "fall", "spike"])
def test_scheduled_kernel_matches_wide_kernel(gpu, monkeypatch, case):
    """Sequences above 256 keys run the hand-scheduled kernel (four waves of
    64 queries); attention variant 14 forces the compiler-scheduled wide
    kernel (eight waves of 32). Both compute the same products, sums and
    lazily raised maxima in the same order, so they agree bit for bit: on
    ragged tails, on many raises of the max, and when the recomputation
    launch redoes every row."""
    if case[0].isdigit():
        seq, heads = map(int, case.split("x"))
        q, k, v = synth.attention_inputs(seq, heads, seed=47, scale=0.5)
    else:
        seq, heads = 1500, 2
        q, k, v = _growth_inputs(seq, heads, case)
    print(f"[attention] scheduled vs wide {case}", flush=True)
    pipe = sdpa(gpu, q, k, v, seq, heads)
    monkeypatch.setenv("H3_HIP_ATTENTION_VARIANT", "14")
    g14 = Gpu()
    try:
        assert np.array_equal(sdpa(g14, q, k, v, seq, heads), pipe)
    finally:
        g14.close()


def test_large_values_after_score_jump(gpu):
    """A 41-log2-unit score jump with |V| near 1e26: P that large must not
    reach O unscaled (it would overflow FP32). The rows go to the
    recomputation launch, and with constant V the output is V."""
    seq, heads = 1500, 2
    rng = np.random.default_rng(5)
    q = np.ones((seq, heads, 128), np.float32)
    k = rng.normal(0, 0.25, (seq, heads, 128)).astype(np.float32)
    k[seq - 300] = 2.5
    big = synth.bf16_to_f32(synth.f32_to_bf16(np.float32(1e26)))
    v = np.full((seq, heads, 128), big, np.float32)
    q, k, v = (synth.f32_to_bf16(x.reshape(-1)) for x in (q, k, v))
    out = bf16(sdpa(gpu, q, k, v, seq, heads))
    assert np.all(np.isfinite(out))
    assert np.max(np.abs(out / big - 1)) < 2e-2


def test_large_values_after_small_score_jump(gpu):
    """A score jump of about 30 log2 units (below the 32-unit retry bound on
    partial sums) with |V| = 1e30: P near 2^30 times V overflows FP32 in the
    fast kernel's O before the max is raised. The non-finite output sends
    those rows to the per-tile-max launch, whose P <= 256 keeps O finite; with
    constant V the output is V, and the call does not fail."""
    seq, heads = 1500, 2
    rng = np.random.default_rng(8)
    q = np.ones((seq, heads, 128), np.float32)
    k = rng.normal(0, 0.25, (seq, heads, 128)).astype(np.float32)
    k[seq - 300] = 1.90625
    big = synth.bf16_to_f32(synth.f32_to_bf16(np.float32(1e30)))
    v = np.full((seq, heads, 128), big, np.float32)
    qb, kb, vb = (synth.f32_to_bf16(x.reshape(-1)) for x in (q, k, v))
    # The jump stays below 32 log2 units over every row's running max.
    scale = scale_bf16(1 / math.sqrt(128))
    s = bf16(kb).reshape(seq, heads, 128).sum(-1) * scale * math.log2(math.e)
    jump = s[seq - 300] - s[:128].max(0)
    assert np.all((jump > 28) & (jump < 32)), jump
    out = bf16(sdpa(gpu, qb, kb, vb, seq, heads))
    assert np.all(np.isfinite(out))
    assert np.max(np.abs(out / big - 1)) < 2e-2
    ref = oracle.attention(bf16(qb), bf16(kb), bf16(vb), seq, heads, scale, rows=(seq - 310, seq - 290))
    m = metrics(out[seq - 310:seq - 290] / big, ref / big)
    assert m["max_abs"] <= ATTN_MAX_ABS and m["cosine"] >= ATTN_COSINE, m


def test_f64_bruteforce_rows(gpu):
    """Sampled rows against a direct FP64 softmax (tests/metal_attention.c:55-67)."""
    seq, heads = 3000, 2
    q, k, v = synth.attention_inputs(seq, heads, seed=9, scale=1.0)
    out = bf16(sdpa(gpu, q, k, v, seq, heads))
    scale = scale_bf16(1 / math.sqrt(128))
    for r0 in (0, 1234, 2990):
        ref = oracle.attention_f64(bf16(q), bf16(k), bf16(v), seq, heads, scale, rows=(r0, r0 + 10))
        m = metrics(out[r0:r0 + 10], ref)
        assert m["max_abs"] <= ATTN_MAX_ABS and m["cosine"] >= ATTN_COSINE, m


def test_invariants(gpu):
    """Zero input -> zero output; constant V -> V (tests/attention_native.c:79-80)."""
    seq, heads = 777, 2
    n = seq * heads * 128
    z = np.zeros(n, np.uint16)
    assert np.all((sdpa(gpu, z, z, z, seq, heads) & 0x7FFF) == 0)
    q, k, _ = synth.attention_inputs(seq, heads, seed=11)
    c = np.full(n, synth.f32_to_bf16(np.float32(0.5)), np.uint16)
    out = bf16(sdpa(gpu, q, k, c, seq, heads))
    assert np.max(np.abs(out - 0.5)) < 0.02


def test_nonfinite_rejected(gpu):
    """NaN input must fail the submit with an error naming 'nonfinite'
    (tests/attention_native.c:71)."""
    seq, heads = 200, 2
    q, k, v = synth.attention_inputs(seq, heads, seed=3)
    q = q.copy()
    q[0] = 0x7FC0
    with pytest.raises(Exception) as e:
        sdpa(gpu, q, k, v, seq, heads)
    assert "nonfinite" in str(e.value)
    gpu.cancel()
    # The context recovers after cancel.
    q, k, v = synth.attention_inputs(seq, heads, seed=4)
    _check(gpu, q, k, v, seq, heads)


def test_inputs_unchanged_and_guards(gpu):
    """Inputs are not modified and nothing is written past the output
    (tests/attention_native.c:57-66,74-77 guard words)."""
    lib = gpu.lib
    seq, heads = 333, 3
    n = seq * heads * 128
    q, k, v = synth.attention_inputs(seq, heads, seed=6)
    guard = np.full(256, 0x7F7F, np.uint16)
    q, k, v = (a.reshape(-1) for a in (q, k, v))
    tq, tk, tv = (gpu.from_bf16(np.concatenate([a, guard])) for a in (q, k, v))
    out = gpu.from_bf16(np.concatenate([np.full(n, 0xFFFF, np.uint16), guard]))
    gpu.begin()
    gpu.check(lib.h3_gpu_dit_sdpa_bf16(gpu.handle, out.handle, tq.handle, tk.handle, tv.handle, seq, heads, 128,
                                       1 / math.sqrt(128), 0, 0, 0), "sdpa")
    gpu.submit()
    for t, a in ((tq, q), (tk, k), (tv, v)):
        assert np.array_equal(t.read()[:n], a)
    o = out.read()
    assert np.all(o[n:] == 0x7F7F)
    assert np.all((o[:n] & 0x7F80) != 0x7F80)


def test_contract_errors(gpu):
    lib = gpu.lib
    seq, heads = 64, 1
    n = seq * heads * 128
    t = gpu.from_bf16(np.zeros(n, np.uint16))
    o = gpu.empty(n)
    # Not inside begin/submit.
    assert not lib.h3_gpu_dit_sdpa_bf16(gpu.handle, o.handle, t.handle, t.handle, t.handle, seq, heads, 128, 0.1, 0, 0, 0)
    gpu.begin()
    # Output aliases an input; D != 128; non-positive scale; short tensor.
    assert not lib.h3_gpu_dit_sdpa_bf16(gpu.handle, t.handle, t.handle, t.handle, t.handle, seq, heads, 128, 0.1, 0, 0, 0)
    assert not lib.h3_gpu_dit_sdpa_bf16(gpu.handle, o.handle, t.handle, t.handle, t.handle, seq, heads * 2, 64, 0.1, 0, 0, 0)
    assert not lib.h3_gpu_dit_sdpa_bf16(gpu.handle, o.handle, t.handle, t.handle, t.handle, seq, heads, 128, -1.0, 0, 0, 0)
    assert not lib.h3_gpu_dit_sdpa_bf16(gpu.handle, o.handle, t.handle, t.handle, t.handle, seq + 1, heads, 128, 0.1, 0, 0, 0)
    gpu.submit()
