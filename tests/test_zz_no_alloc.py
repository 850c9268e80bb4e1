"""The no-allocation dense attention entry point (h3_hip_sdpa_bf16_noalloc)
against the allocating one (h3_gpu_sdpa_bf16 / _head_major_output), through
the C ABI: bit-identical outputs on two calls in a row, the second smaller,
no device allocation by the library during either, and a clear error for a
workspace above the fixed scratch size."""
import ctypes as C
import math

import numpy as np
import pytest

from h3cli_amd import synth
from h3cli_amd._lib import GpuStats
from h3cli_amd.runtime import Gpu

pytestmark = pytest.mark.gpu

SCALE = 1 / math.sqrt(128)


def stats(g):
    s = GpuStats()
    assert g.lib.h3_gpu_get_stats(g.handle, C.byref(s))
    return s


def run(g, fn, out, ts, seq, heads, *extra):
    g.begin()
    g.check(fn(g.handle, out.handle, ts[0].handle, ts[1].handle, ts[2].handle, seq, heads, 128, C.c_float(SCALE),
               *extra), "attention")
    g.submit()
    return out.read()


def test_noalloc_matches_allocating_entry():
    with Gpu() as g:
        lib = g.lib
        # Two calls in a row on the no-allocation entry, the second smaller,
        # each compared with the allocating entry on the same inputs.
        cases = [(4133, 6, 0), (700, 3, 1)]
        inputs = []
        for seq, heads, hm in cases:
            q, k, v = synth.attention_inputs(seq, heads, seed=seq, scale=0.5, rope_shape=(27, 30, 40))
            inputs.append(([g.from_bf16(x) for x in (q, k, v)], g.empty(seq * heads * 128), g.empty(seq * heads * 128)))
        before = stats(g)
        got = []
        for (seq, heads, hm), (ts, out, _) in zip(cases, inputs):
            print(f"[noalloc] seq={seq} heads={heads} head_major={hm}", flush=True)
            got.append(run(g, lib.h3_hip_sdpa_bf16_noalloc, out, ts, seq, heads, hm))
        after = stats(g)
        assert after.allocated_bytes == before.allocated_bytes
        assert after.tensor_allocations == before.tensor_allocations
        assert after.attention_workspace_bytes == before.attention_workspace_bytes == 0
        for (seq, heads, hm), (ts, _, ref_out), out in zip(cases, inputs, got):
            fn = lib.h3_gpu_sdpa_bf16_head_major_output if hm else lib.h3_gpu_sdpa_bf16
            want = run(g, fn, ref_out, ts, seq, heads)
            assert np.array_equal(out, want), (seq, heads, hm)
            assert np.all(np.isfinite(synth.bf16_to_f32(out)))


def test_noalloc_refuses_oversized_workspace():
    """S = 65536, H = 56 needs 940 MB of workspace: refused before any launch,
    with the size in the message; the context stays usable."""
    with Gpu() as g:
        lib = g.lib
        seq, heads = 65536, 56
        n = seq * heads * 128
        ts = [g.empty(n) for _ in range(3)]
        out = g.empty(n)
        g.begin()
        ok = lib.h3_hip_sdpa_bf16_noalloc(g.handle, out.handle, ts[0].handle, ts[1].handle, ts[2].handle, seq, heads,
                                          128, C.c_float(SCALE), 0)
        assert not ok and "above the fixed" in g.error()
        g.cancel()
        seq, heads = 300, 2
        q, k, v = synth.attention_inputs(seq, heads, seed=1)
        small = [g.from_bf16(x) for x in (q, k, v)]
        a = run(g, lib.h3_hip_sdpa_bf16_noalloc, g.empty(seq * heads * 128), small, seq, heads, 0)
        b = run(g, lib.h3_gpu_sdpa_bf16, g.empty(seq * heads * 128), small, seq, heads)
        assert np.array_equal(a, b)
