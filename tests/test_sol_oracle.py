"""Pins of the SOL C restatement (oracle/sol.c) against the reference's own
NumPy oracle formulas (tests/cuda_sol_oracle.py, restated in
tests/sol_fixtures.py), closed forms and the routing rules one by one."""
import math

import numpy as np

from h3cli_amd import synth
from oracle import oracle
from tests.helpers import scale_bf16
from tests.sol_fixtures import attention64, inputs, metadata, routes64, summaries

SCALE = scale_bf16(1 / math.sqrt(128))


def _ulps(a, b):
    return np.abs(synth.f32_to_bf16(a).astype(np.int64) - synth.f32_to_bf16(b).astype(np.int64))


def test_summary_and_moments():
    seq, heads = 300, 2                       # ragged last blocks: 300 = 9*32 + 12 = 4*64 + 44
    q, k, _ = inputs(seq, heads, seed=3)
    for x, b in ((q, 32), (q, 64), (k, 64)):
        got = synth.bf16_to_f32(oracle.sol_summary(x, seq, heads, b)).reshape(heads, -1, 128)
        want = summaries(x, b).transpose(1, 0, 2)
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
    """Separated pairs (|dot - threshold| > 1e-5) route as the float64 rule;
    protection, locality, floor and tail force exact as the rule says."""
    seq, heads, qb = 1000, 3, 32
    q, k, _ = inputs(seq, heads, seed=5)
    meta = metadata(seq, qb, protected=True)
    qc, kc = oracle.sol_summary(q, seq, heads, qb), oracle.sol_summary(k, seq, heads, 64)
    kb = (seq + 63) // 64
    mom = oracle.sol_moments(kc, heads, kb)
    for minimum, tau, radius in ((0.0, 1.0, 1), (0.5, 1.0, 0), (0.0, 0.25, 3), (0.0, 16.0, 0)):
        floor_count = int(np.ceil(float(np.float32(minimum)) * kb))
        got, counts = oracle.sol_route(qc, kc, mom, meta[0], meta[1], heads, radius, floor_count, SCALE, tau)
        assert counts[0] + counts[1] == heads * len(meta[0]) * kb
        assert counts[0] == got.sum()
        qcf = synth.bf16_to_f32(qc).reshape(heads, -1, 128)
        kcf = synth.bf16_to_f32(kc).reshape(heads, -1, 128)
        for h in range(heads):
            want, dots, thr = routes64(qcf[h], kcf[h], meta, SCALE, minimum, tau, radius)
            sep = np.abs(dots - thr[:, None]) > 1e-5
            assert np.array_equal(got[h][sep], want[sep]), (minimum, tau, radius, h)
            assert (~sep).mean() < 0.02
    # Everything exact with force_exact; tail block (44 rows) always exact.
    got, _ = oracle.sol_route(qc, kc, mom, meta[0], meta[1], heads, 0, 0, SCALE, 16.0, True)
    assert got.all()
    meta0 = metadata(seq, qb)
    got, _ = oracle.sol_route(qc, kc, mom, meta0[0], meta0[1], heads, 0, 0, SCALE, 16.0)
    assert got[:, :, -1].all() and not got[:, :, :-1].all()


def test_attention_matches_concatenated_softmax():
    seq, heads, qb = 260, 2, 32
    q, k, v = inputs(seq, heads, seed=9)
    kc, vc = oracle.sol_summary(k, seq, heads, 64), oracle.sol_summary(v, seq, heads, 64)
    rng = np.random.default_rng(2)
    routes = (rng.random((heads, (seq + qb - 1) // qb, 5)) < 0.4).astype(np.uint8)
    routes[:, :, 4] = 1                      # the 4-row tail block is always exact
    got = oracle.sol_attention(q, k, v, kc, vc, routes, seq, heads, qb, SCALE).reshape(seq, heads, 128)
    qf, kf, vf = (synth.bf16_to_f32(a).reshape(seq, heads, 128) for a in (q, k, v))
    kcf = synth.bf16_to_f32(kc).reshape(heads, -1, 128)
    vcf = synth.bf16_to_f32(vc).reshape(heads, -1, 128)
    rows = [0, 31, 32, 100, 259]
    for h in range(heads):
        want = attention64(qf, kf, vf, kcf[h], vcf[h], routes[h], qb, SCALE, rows, h)
        assert np.max(np.abs(got[rows, h] - want)) < 1e-6
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
