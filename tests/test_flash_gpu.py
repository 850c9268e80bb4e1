"""FlashAttention-2-style forward with log-sum-exp (h3_sglang_flash,
h3_sglang_flash_query_range; the reference's src/cuda/cuda_sglang_flash.h
interface) on the GPU: outputs against the CPU oracle, lse against a float64
log-sum-exp, a query range equal to the same rows of the full call, and the
argument rules (invalid -> 0, unsupported shapes -> 0 with a message)."""
import ctypes as C
import math

import numpy as np
import pytest

from h3cli_amd import synth
from h3cli_amd.runtime import Gpu
from oracle import oracle
from tests.helpers import ATTN_COSINE, ATTN_MAX_ABS, bf16, metrics

pytestmark = pytest.mark.gpu

SCALE = 1 / math.sqrt(128)


def ptr(g, t):
    p = g.lib.h3_hip_tensor_device_pointer(t.handle)
    assert p
    return p


def lse64(q, k, rows, heads):
    """float64 log sum_j exp(scale q_i . k_j) for query rows `rows`, [heads, len(rows)]."""
    qf, kf = bf16(q).astype(np.float64), bf16(k).astype(np.float64)
    out = np.zeros((heads, len(rows)))
    for h in range(heads):
        s = qf[rows, h] @ kf[:, h].T * SCALE
        mx = s.max(axis=1)
        out[h] = mx + np.log(np.exp(s - mx[:, None]).sum(axis=1))
    return out


def flash(g, out, q, k, v, lse, batch, seq, heads, head_major=0, dim=128, causal=0, kv_heads=None):
    err = C.create_string_buffer(256)
    g.begin()
    r = g.lib.h3_sglang_flash(ptr(g, out), ptr(g, q), ptr(g, k), ptr(g, v), ptr(g, lse), batch, seq, heads,
                              heads if kv_heads is None else kv_heads, dim, C.c_float(SCALE), causal, head_major,
                              g.lib.h3_hip_compute_stream(g.handle), err, 256)
    g.submit()
    return r, err.value.decode()


@pytest.mark.parametrize("head_major", [0, 1])
def test_flash_outputs_and_lse(head_major):
    batch, seq, heads = 2, 1000, 4
    print(f"[flash] batch={batch} seq={seq} heads={heads} head_major={head_major}", flush=True)
    n = seq * heads * 128
    xs = [synth.attention_inputs(seq, heads, seed=40 + b, scale=0.5, rope_shape=(27, 30, 40)) for b in range(batch)]
    with Gpu() as g:
        tq, tk, tv = (g.from_bf16(np.concatenate([x[i].reshape(-1) for x in xs])) for i in range(3))
        out = g.empty(batch * n)
        lse = g.from_f32(np.zeros(batch * heads * seq, np.float32))
        r, msg = flash(g, out, tq, tk, tv, lse, batch, seq, heads, head_major)
        assert r == 1, msg
        got = bf16(out.read()).reshape(batch, -1)
        got_lse = lse.read().reshape(batch, heads, seq)
    rows = np.arange(seq)
    for b, (q, k, v) in enumerate(xs):
        o = got[b].reshape((heads, seq, 128) if head_major else (seq, heads, 128))
        if head_major:
            o = o.transpose(1, 0, 2)
        ref = oracle.attention(bf16(q), bf16(k), bf16(v), seq, heads, SCALE)
        m = metrics(o, ref)
        assert m["max_abs"] <= ATTN_MAX_ABS and m["cosine"] >= ATTN_COSINE, m
        want = lse64(q.reshape(seq, heads, 128), k.reshape(seq, heads, 128), rows, heads)
        assert np.max(np.abs(got_lse[b] - want)) < 1e-4 * max(1.0, float(np.abs(want).max()))


@pytest.mark.parametrize("first,count,head_major", [(300, 200, 0), (0, 1, 1), (1000, 25, 0), (513, 512, 1)])
def test_query_range_equals_full_rows(first, count, head_major):
    seq, heads = 1025, 3
    print(f"[flash range] seq={seq} first={first} count={count} head_major={head_major}", flush=True)
    q, k, v = synth.attention_inputs(seq, heads, seed=7, scale=0.5)
    n = seq * heads * 128
    with Gpu() as g:
        tq, tk, tv = g.from_bf16(q), g.from_bf16(k), g.from_bf16(v)
        full, lse_full = g.empty(n), g.from_f32(np.zeros(heads * seq, np.float32))
        assert flash(g, full, tq, tk, tv, lse_full, 1, seq, heads, head_major)[0] == 1
        sentinel = np.full(n, 0x7F7F, np.uint16)
        part = g.from_bf16(sentinel)
        lse_part = g.from_f32(np.zeros(heads * count, np.float32))
        err = C.create_string_buffer(256)
        g.begin()
        r = g.lib.h3_sglang_flash_query_range(ptr(g, part), ptr(g, tq), ptr(g, tk), ptr(g, tv), ptr(g, lse_part), seq,
                                              heads, first, count, C.c_float(SCALE), head_major,
                                              g.lib.h3_hip_compute_stream(g.handle), err, 256)
        g.submit()
        assert r == 1, err.value
        a = full.read().reshape((heads, seq, 128) if head_major else (seq, heads, 128))
        b = part.read().reshape(a.shape)
        la, lb = lse_full.read().reshape(heads, seq), lse_part.read().reshape(heads, count)
    sl = (slice(None), slice(first, first + count)) if head_major else (slice(first, first + count),)
    assert np.array_equal(b[sl], a[sl])
    outside = np.ones(a.shape, bool)
    outside[sl] = False
    assert np.all(b[outside] == 0x7F7F)
    assert np.array_equal(lb, la[:, first:first + count])


def test_argument_rules():
    seq, heads = 128, 2
    n = seq * heads * 128
    with Gpu() as g:
        t = [g.from_bf16(np.zeros(n, np.uint16)) for _ in range(4)]
        lse = g.from_f32(np.zeros(heads * seq, np.float32))
        # Unsupported shapes: a message and 0.
        for kw in (dict(causal=1), dict(dim=64), dict(kv_heads=1)):
            r, msg = flash(g, t[3], t[0], t[1], t[2], lse, 1, seq, heads, **kw)
            assert r == 0 and "HIP backend" in msg, kw
        # Invalid arguments: 0.
        err = C.create_string_buffer(256)
        s = g.lib.h3_hip_compute_stream(g.handle)
        P = [ptr(g, x) for x in t]
        assert g.lib.h3_sglang_flash(P[3], P[0], P[1], P[2], ptr(g, lse), 0, seq, heads, heads, 128,
                                     C.c_float(SCALE), 0, 0, s, err, 256) == 0
        assert g.lib.h3_sglang_flash(P[3], P[0], P[1], P[2], ptr(g, lse), 1, seq, heads, heads, 128,
                                     C.c_float(-1.0), 0, 0, s, err, 256) == 0
        rng = g.lib.h3_sglang_flash_query_range
        assert rng(P[3], P[0], P[1], P[2], ptr(g, lse), seq, heads, seq, 1, C.c_float(SCALE), 0, s, err, 256) == 0
        assert rng(P[3], P[0], P[1], P[2], ptr(g, lse), seq, heads, 100, 29, C.c_float(SCALE), 0, s, err, 256) == 0
        assert rng(P[3], P[0], P[1], P[2], None, seq, heads, 0, 1, C.c_float(SCALE), 0, s, err, 256) == 0
