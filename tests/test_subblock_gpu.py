"""SubBlock router (attention mode 4 with a bound layout) on the GPU.

Mirrors the reference's native test and oracle (tests/subblock_native.cu,
tests/subblock_oracle.py): pooled cells bit-exact vs oracle_sb_pool; scores
within the contract tolerance of the float64 scores of those cells (golden
vectors written by the reference's oracle); routes exactly the oracle's
selection of the returned scores (ties, protection) and, on rows where the
keep-th gap exceeds twice the tolerance, exactly the reference's selection;
attention output vs the routed oracle; layout-independent output (row vs head
major); the constant-value invariant; nonfinite rejection; route counters.
"""
import ctypes as C
import math

import numpy as np
import pytest

from h3cli_amd import synth
from h3cli_amd._lib import GpuStats
from h3cli_amd.runtime import Gpu
from oracle import oracle
from tests.helpers import ATTN_COSINE, ATTN_MAX_ABS, bf16, metrics, sdpa
from tests.router_inputs import Layout, native_inputs, protect_ends, subblock_case_inputs, vectors

pytestmark = pytest.mark.gpu

SCALE = 1 / math.sqrt(128)
SPARSITY = 0.75
STEP, BLOCK = 12, 1   # past the default warmup, not the probe block


def make_router(seq, q_protect=None, k_protect=None, sparsity=SPARSITY):
    g = Gpu()
    g.check(g.lib.h3_gpu_dit_attention_configure(g.handle, 4), "configure")
    g.check(g.lib.h3_hip_dit_subblock_policy(g.handle, sparsity, 0), "policy")
    g.layout = Layout(seq, q_protect=q_protect, k_protect=k_protect)
    g.check(g.lib.h3_gpu_dit_sol_layout(g.handle, g.layout.ptr), "layout")
    g.check(g.lib.h3_gpu_dit_attention_noise(g.handle, STEP, 0.5, 0.5), "noise")
    return g


def capture(g, seq, heads):
    blocks = (seq + 63) // 64
    nr = heads * blocks * blocks
    npool = heads * blocks * 4 * 128
    routes = np.zeros(nr, np.uint8)
    scores = np.zeros(nr, np.float32)
    qp = np.zeros(npool, np.uint16)
    kp = np.zeros(npool, np.uint16)
    g.check(g.lib.h3_hip_subblock_routes(g.handle, routes.ctypes.data, scores.ctypes.data, nr, qp.ctypes.data,
                                         kp.ctypes.data, npool), "routes")
    return (routes.reshape(heads, blocks, blocks), scores.reshape(heads, blocks, blocks), qp, kp)


def stats(g):
    s = GpuStats()
    assert g.lib.h3_gpu_get_stats(g.handle, C.byref(s))
    return s


def keep_of(g, blocks):
    return g.lib.h3_subblock_budget(blocks, C.c_float(SPARSITY))


def check_router(g, q, k, seq, heads, kind, q_protect=None, k_protect=None):
    """Pools, scores and routes of the last call vs the oracle and the golden
    vectors of case (seq, heads, kind); returns routes."""
    blocks = (seq + 63) // 64
    routes, scores, qp, kp = capture(g, seq, heads)
    qscale = np.float32(np.float32(SCALE) * np.float32(1.4426950408889634))
    assert np.array_equal(qp, oracle.sb_pool(q, seq, heads, qscale)), "Q pool"
    assert np.array_equal(kp, oracle.sb_pool(k, seq, heads, 1.0)), "K pool"
    tag = f"{seq}_{heads}_{kind}"
    expected = vectors()[f"sb_scores_{tag}"]
    err = np.abs(scores - expected)
    assert np.all(err <= 2e-4 + 2e-5 * np.abs(expected)), float(err.max())
    keep = keep_of(g, blocks)
    # Selection of the returned scores: exact (ties to the lower index).
    own = oracle.sb_select(scores, heads, blocks, keep, q_protect, k_protect).reshape(heads, blocks, blocks)
    assert np.array_equal(routes, own), "selection/tie/protection"
    # The reference's selection where its float64 ranking is separated.
    indep, separated = vectors()[f"sb_routes_{tag}"], vectors()[f"sb_separated_{tag}"]
    assert np.array_equal(routes[separated], indep[separated])
    print(f"  keep={keep}/{blocks} density={routes.mean():.3f} separated rows={int(separated.sum())}", flush=True)
    return routes


def sample_rows(seq, blocks_protected=()):
    rows = set(np.unique(np.linspace(0, seq - 1, 40).astype(int)).tolist())
    rows |= {0, 63, 64, 127, 128, seq - 1}
    for b in blocks_protected:
        rows |= {b * 64, min(seq - 1, b * 64 + 63)}
    return sorted(r for r in rows if r < seq)


@pytest.mark.parametrize("seq,heads,kind", [(4200, 2, 0), (4200, 2, 4), (5000, 3, 9)])
def test_router_and_output(seq, heads, kind):
    print(f"[subblock] seq={seq} heads={heads} kind={kind}", flush=True)
    q, k, v = subblock_case_inputs(seq, heads, kind)
    q_protect = protect_ends(seq) if kind == 4 else None
    g = make_router(seq, q_protect, q_protect)
    try:
        out = bf16(sdpa(g, q, k, v, seq, heads, scale=SCALE, step=STEP, block=BLOCK))
        routes = check_router(g, q, k, seq, heads, kind, q_protect, q_protect)
        blocks = (seq + 63) // 64
        assert routes.mean() < 0.5        # the router is actually sparse
        if q_protect is not None:
            assert np.all(routes[:, 0] == 1) and np.all(routes[:, -1] == 1) and np.all(routes[:, :, 0] == 1)
        rows = sample_rows(seq, (0, blocks - 1))
        ref = np.concatenate([oracle.attention_routed(bf16(q), bf16(k), bf16(v), seq, heads, SCALE, routes,
                                                      (r, r + 1)) for r in rows]).reshape(len(rows), heads, 128)
        m = metrics(out[rows], ref)
        assert m["max_abs"] <= ATTN_MAX_ABS and m["cosine"] >= ATTN_COSINE, m
        s = stats(g)
        assert s.subblock_calls == 1 and s.subblock_router_calls == 1
        assert s.subblock_selected == int(routes.sum()) and s.subblock_possible == heads * blocks * blocks
        assert s.subblock_protected_calls == (2 if kind == 4 else 0)
        # The same call with a head-major output is the same numbers.
        hm = bf16(sdpa(g, q, k, v, seq, heads, scale=SCALE, step=STEP, block=BLOCK, head_major=True))
        assert np.array_equal(hm, out)
    finally:
        g.close()


def plan_info(g):
    grp, slab, nbytes = C.c_uint32(), C.c_uint32(), C.c_size_t()
    g.check(g.lib.h3_hip_subblock_plan_info(g.handle, C.byref(grp), C.byref(slab), C.byref(nbytes)), "plan")
    return grp.value, slab.value, nbytes.value


def test_chunked_workspace_matches_whole_call():
    """Bounded workspace (plan order of the reference's h3_subblock_plan_make,
    src/denoise/subblock.c:18-42, under the 512 MiB cap of
    src/denoise/attention.h:12). Lowering this context's budget splits the call
    into head groups, then query slabs; every split gives the whole call's
    output bit for bit (row- and head-major) and the same route counters, the
    planned bytes stay within the budget, and a budget no chunk fits fails."""
    seq, heads = 5000, 3
    blocks = (seq + 63) // 64
    print(f"[subblock] chunked seq={seq} heads={heads}", flush=True)
    q, k, v = subblock_case_inputs(seq, heads, 4)
    prot = protect_ends(seq)
    g = make_router(seq, prot, prot)
    try:
        whole = sdpa(g, q, k, v, seq, heads, scale=SCALE, step=STEP, block=BLOCK)
        whole_hm = sdpa(g, q, k, v, seq, heads, scale=SCALE, step=STEP, block=BLOCK, head_major=True)
        assert np.array_equal(whole_hm, whole)
        grp, slab, nbytes = plan_info(g)
        assert (grp, slab) == (heads, blocks) and nbytes <= 512 << 20
        routes = capture(g, seq, heads)[0]
        per_call = int(routes.sum())
        selected = stats(g).subblock_selected
        assert selected == 2 * per_call
        seen_group = seen_slab = failed = False
        for _ in range(20):
            # A budget one byte below the last plan forces the next smaller one.
            cap = nbytes - 1
            g.check(g.lib.h3_hip_subblock_workspace_cap(g.handle, cap), "cap")
            try:
                out = sdpa(g, q, k, v, seq, heads, scale=SCALE, step=STEP, block=BLOCK)
            except RuntimeError as e:
                assert "fixed budget" in str(e), str(e)
                failed = True
                break
            grp, slab, nbytes = plan_info(g)
            print(f"  cap={cap} -> head group {grp}, slab {slab}, {nbytes} bytes", flush=True)
            assert nbytes <= cap and grp <= heads and slab <= blocks
            assert slab == blocks or slab % 32 == 0
            assert np.array_equal(out, whole), (grp, slab)
            s = stats(g).subblock_selected
            assert s - selected == per_call, (grp, slab)
            selected = s
            if slab < blocks:
                hm = sdpa(g, q, k, v, seq, heads, scale=SCALE, step=STEP, block=BLOCK, head_major=True)
                assert np.array_equal(hm, whole)
                selected = stats(g).subblock_selected
                # A chunked call keeps no whole-call routes.
                assert not g.lib.h3_hip_subblock_routes(g.handle, None, None, 0, None, None, 0)
            seen_group |= grp < heads
            seen_slab |= slab < blocks
        assert seen_group and seen_slab and failed
        # The default budget again: one chunk.
        g.check(g.lib.h3_hip_subblock_workspace_cap(g.handle, 0), "cap")
        assert np.array_equal(sdpa(g, q, k, v, seq, heads, scale=SCALE, step=STEP, block=BLOCK), whole)
        assert plan_info(g)[:2] == (heads, blocks)
    finally:
        g.close()


def test_constant_value_and_ties():
    """Zero Q and K: all scores tie, so each query block keeps the first
    `keep` key blocks; V = 0.5 gives exactly 0.5 (subblock_oracle.py:95)."""
    seq, heads = 4200, 2
    q, k, v = native_inputs(seq, heads, 1)
    g = make_router(seq)
    try:
        out = bf16(sdpa(g, q, k, v, seq, heads, scale=SCALE, step=STEP, block=BLOCK))
        assert np.all(out == 0.5)
        routes, scores, _, _ = capture(g, seq, heads)
        blocks = (seq + 63) // 64
        keep = keep_of(g, blocks)
        assert np.all(routes[:, :, :keep] == 1) and np.all(routes[:, :, keep:] == 0)
    finally:
        g.close()


def test_large_values_kind3():
    """Q = 100, K = +-100 by channel parity: every pooled dot is exactly 0, so
    the ranking is decided by index alone, and outputs are V means."""
    seq, heads = 4160, 1
    q, k, v = native_inputs(seq, heads, 3)
    g = make_router(seq)
    try:
        out = bf16(sdpa(g, q, k, v, seq, heads, scale=SCALE, step=STEP, block=BLOCK))
        routes = check_router(g, q, k, seq, heads, 3)
        blocks = (seq + 63) // 64
        assert np.all(routes[:, :, :keep_of(g, blocks)] == 1)
        rows = sample_rows(seq)
        ref = np.concatenate([oracle.attention_routed(bf16(q), bf16(k), bf16(v), seq, heads, SCALE, routes,
                                                      (r, r + 1)) for r in rows]).reshape(len(rows), heads, 128)
        m = metrics(out[rows], ref)
        assert m["max_abs"] <= ATTN_MAX_ABS, m
    finally:
        g.close()


def test_nonfinite_rejected_and_recovers():
    seq, heads = 4200, 1
    q, k, v = native_inputs(seq, heads, 2)
    g = make_router(seq)
    try:
        with pytest.raises(Exception) as e:
            sdpa(g, q, k, v, seq, heads, scale=SCALE, step=STEP, block=BLOCK)
        assert "nonfinite" in str(e.value)
        g.cancel()
        q = q.copy()
        q.reshape(-1)[-1] = 0
        out = bf16(sdpa(g, q, k, v, seq, heads, scale=SCALE, step=STEP, block=BLOCK))
        assert np.isfinite(out).all()
    finally:
        g.close()


def test_layout_rules():
    """Layout geometry is validated as in the reference's configure
    (cuda_subblock.cu:352-361); a second layout is rejected; a call whose
    sequence differs from the layout fails; no layout fails."""
    seq = 4200
    g = Gpu()
    try:
        g.check(g.lib.h3_gpu_dit_attention_configure(g.handle, 4), "configure")
        g.check(g.lib.h3_hip_dit_subblock_policy(g.handle, SPARSITY, 0), "policy")
        g.check(g.lib.h3_gpu_dit_attention_noise(g.handle, STEP, 0.5, 0.5), "noise")
        q, k, v = synth.attention_inputs(seq, 1, seed=2)
        with pytest.raises(RuntimeError):
            sdpa(g, q, k, v, seq, 1, step=STEP, block=BLOCK)          # no layout bound
        bad = Layout(seq)
        bad.arrays[0][0].rows = 0
        assert not g.lib.h3_gpu_dit_sol_layout(g.handle, bad.ptr)
        good = Layout(seq)
        g.check(g.lib.h3_gpu_dit_sol_layout(g.handle, good.ptr), "layout")
        assert not g.lib.h3_gpu_dit_sol_layout(g.handle, good.ptr)   # already configured
        q2, k2, v2 = synth.attention_inputs(seq + 64, 1, seed=2)
        with pytest.raises(RuntimeError):
            sdpa(g, q2, k2, v2, seq + 64, 1, step=STEP, block=BLOCK)
    finally:
        g.close()


def test_real_h3_shape_under_cap():
    """The real H3 video shape (S = 109078, H = 56): the whole call would need
    about 3 GB of router buffers and transposed V; under the default 512 MiB
    budget it runs in head groups and its output equals the whole call's (a
    budget large enough for one chunk) bit for bit. Inputs are 0.5 N(0,1) from
    the device generator; the first and last 64-row blocks are protected."""
    seq, heads = 109078, 56
    blocks = (seq + 63) // 64
    n = seq * heads * 128
    print(f"[subblock] real shape seq={seq} heads={heads}", flush=True)
    prot = protect_ends(seq)
    g = make_router(seq, prot, prot)
    try:
        lib = g.lib
        q, k, v, out = (g.empty(n) for _ in range(4))
        g.begin()
        for i, t in enumerate((q, k, v)):
            g.check(lib.h3_hip_fill_normal_bf16(g.handle, t.handle, 77 * 16 + i, 0.5, n), "fill")
        g.submit()

        def run():
            g.begin()
            g.check(lib.h3_gpu_dit_sdpa_bf16(g.handle, out.handle, q.handle, k.handle, v.handle, seq, heads, 128,
                                             C.c_float(SCALE), 0, BLOCK, STEP), "routed attention")
            g.submit()
            return out.read()

        chunked = run()
        grp, slab, nbytes = plan_info(g)
        print(f"  default budget: head group {grp}, slab {slab}, {nbytes} bytes", flush=True)
        assert nbytes <= 512 << 20 and grp < heads
        assert np.all(np.isfinite(bf16(chunked[:: 997])))
        g.check(lib.h3_hip_subblock_workspace_cap(g.handle, 8 << 30), "cap")
        whole = run()
        assert plan_info(g)[:2] == (heads, blocks)
        assert np.array_equal(chunked, whole)
    finally:
        g.close()
