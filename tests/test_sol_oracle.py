"""Pins of the SOL C restatement (oracle/sol.c) against vectors from the
reference's own NumPy oracle (tests/cuda_sol_oracle.py, run by
tests/golden/make_router_vectors.py), closed forms and the routing rules one
by one."""
import math

import numpy as np

from h3cli_amd import synth
from oracle import oracle
from tests.helpers import scale_bf16
from tests.router_inputs import SOL_ATTENTION_ROWS, SOL_ROUTE_OPTIONS, sol_inputs, sol_layout, vectors

SCALE = scale_bf16(1 / math.sqrt(128))


def _ulps(a, b):
    return np.abs(synth.f32_to_bf16(a).astype(np.int64) - synth.f32_to_bf16(b).astype(np.int64))


def test_summary_and_moments():
    seq, heads = 300, 2                       # ragged last blocks: 300 = 9*32 + 12 = 4*64 + 44
    q, k, _ = sol_inputs(seq, heads, seed=3)
    for name, x, b in (("q32", q, 32), ("q64", q, 64), ("k64", k, 64)):
        got = synth.bf16_to_f32(oracle.sol_summary(x, seq, heads, b)).reshape(heads, -1, 128)
        want = vectors()[f"sol_summary_300_{name}"].transpose(1, 0, 2)
        assert got.shape == want.shape and _ulps(got, want).max() <= 1 and (got == want).mean() > 0.99
    const = synth.f32_to_bf16(np.full((70, 1, 128), 0.375, np.float32))
    assert np.all(synth.bf16_to_f32(oracle.sol_summary(const, 70, 1, 64)) == 0.375)
    kc = oracle.sol_summary(k, seq, heads, 64)
    mom = oracle.sol_moments(kc, heads, 5).reshape(heads, 256)
    kf = synth.bf16_to_f32(kc).reshape(heads, 5, 128).astype(np.float64)
    assert np.allclose(mom[:, :128], kf.mean(axis=1), rtol=1e-6, atol=1e-7)
    assert np.allclose(mom[:, 128:], np.maximum((kf ** 2).mean(axis=1) - kf.mean(axis=1) ** 2, 0), rtol=1e-4,
                       atol=1e-6)


def test_routes_match_float64_rule():
    """Routes equal the reference's float64 rule on the same centroids on
    every pair that a 1e-5 relative change of tau does not flip (near ties
    are < 2% of pairs); protection, locality, floor and tail force exact."""
    seq, heads, qb = 1000, 3, 32
    q, k, _ = sol_inputs(seq, heads, seed=5)
    meta = sol_layout(seq, qb, protected=True)
    qc, kc = oracle.sol_summary(q, seq, heads, qb), oracle.sol_summary(k, seq, heads, 64)
    kb = (seq + 63) // 64
    mom = oracle.sol_moments(kc, heads, kb)
    for n, (minimum, tau, radius) in enumerate(SOL_ROUTE_OPTIONS):
        floor_count = int(np.ceil(float(np.float32(minimum)) * kb))
        got, counts = oracle.sol_route(qc, kc, mom, meta[0], meta[1], heads, radius, floor_count, SCALE, tau)
        assert counts[0] + counts[1] == heads * len(meta[0]) * kb
        assert counts[0] == got.sum()
        want, sep = vectors()[f"sol_routes_{n}"], vectors()[f"sol_separated_{n}"]
        assert np.array_equal(got[sep], want[sep]), (minimum, tau, radius)
        assert (~sep).mean() < 0.02
    # Everything exact with force_exact; tail block (40 rows) always exact.
    got, _ = oracle.sol_route(qc, kc, mom, meta[0], meta[1], heads, 0, 0, SCALE, 16.0, True)
    assert got.all()
    meta0 = sol_layout(seq, qb)
    got, _ = oracle.sol_route(qc, kc, mom, meta0[0], meta0[1], heads, 0, 0, SCALE, 16.0)
    assert got[:, :, -1].all() and not got[:, :, :-1].all()


def test_attention_matches_concatenated_softmax():
    """The reference's softmax over exact keys and ln 64-biased centroids
    (tau 0.5, no locality), with its own routes: the oracle on the same
    routes agrees to 1e-6."""
    seq, heads, qb = 260, 2, 32
    q, k, v = sol_inputs(seq, heads, seed=9)
    kc, vc = oracle.sol_summary(k, seq, heads, 64), oracle.sol_summary(v, seq, heads, 64)
    routes = vectors()["sol_masks_260"]
    assert 0 < routes.mean() < 1
    got = oracle.sol_attention(q, k, v, kc, vc, routes, seq, heads, qb, SCALE).reshape(seq, heads, 128)
    want = vectors()["sol_out_260"]
    rows = SOL_ATTENTION_ROWS
    assert np.max(np.abs(got[rows] - want)) < 1e-6
    qf, kf, vf = (synth.bf16_to_f32(a).reshape(seq, heads, 128) for a in (q, k, v))
    rng = np.random.default_rng(2)
    # All exact: the dense softmax.
    ones = np.ones_like(routes)
    full = oracle.sol_attention(q, k, v, kc, vc, ones, seq, heads, qb, SCALE).reshape(seq, heads, 128)
    dense = oracle.attention(qf, kf, vf, seq, heads, SCALE).reshape(seq, heads, 128)
    assert np.max(np.abs(full - dense)) < 1e-5
    # A centroid entry of a block whose keys all equal its centroid contributes
    # exactly as the 64 keys would (the ln 64 bias): constant K and V blocks.
    kk = synth.f32_to_bf16(np.broadcast_to(rng.normal(size=(5, 1, heads, 128)).astype(np.float32),
                                           (5, 64, heads, 128)).reshape(320, heads, 128)[:seq])
    vv = synth.f32_to_bf16(np.broadcast_to(rng.normal(size=(5, 1, heads, 128)).astype(np.float32),
                                           (5, 64, heads, 128)).reshape(320, heads, 128)[:seq])
    kcc, vcc = oracle.sol_summary(kk, seq, heads, 64), oracle.sol_summary(vv, seq, heads, 64)
    half = routes.copy()
    approx = oracle.sol_attention(q, kk, vv, kcc, vcc, half, seq, heads, qb, SCALE, rows=(0, 64))
    exact = oracle.sol_attention(q, kk, vv, kcc, vcc, ones, seq, heads, qb, SCALE, rows=(0, 64))
    assert np.max(np.abs(approx - exact)) < 1e-5
