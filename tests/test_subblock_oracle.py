"""Pins of the SubBlock router's C restatement (oracle/block.c: oracle_sb_pool,
oracle_sb_score, oracle_sb_select, oracle_attention_routed) against vectors
from the reference's own NumPy oracle (tests/subblock_oracle.py, run by
tests/golden/make_router_vectors.py), closed forms and brute force."""
import math

import numpy as np

from h3cli_amd import synth
from oracle import oracle
from tests.router_inputs import native_inputs, random_pool_inputs, select_inputs, vectors


def score_tolerance(expected):
    """The reference's contract tolerance of pooled scores (subblock_oracle.py:60)."""
    return 2e-4 + 2e-5 * np.abs(expected)


SCALE = np.float32(1 / math.sqrt(128))
QSCALE = np.float32(SCALE * np.float32(math.log2(math.e)))


def test_pool_matches_float64_means():
    """The fp32 tree sum agrees with the float64 mean to the BF16 rounding:
    at most one BF16 step apart, and identical almost everywhere. Ragged
    sequence: the last cell holds 5 rows, cells past it are zero."""
    seq, heads = 69, 3
    q, _, _ = native_inputs(seq, heads, 0)
    got = synth.bf16_to_f32(oracle.sb_pool(q, seq, heads, QSCALE)).reshape(heads, -1, 128)
    want = vectors()["sb_pool_69_q"]
    assert got.shape == want.shape == (heads, 8, 128)
    ulp = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64)) >> 16
    assert ulp.max() <= 1
    assert (got == want).mean() > 0.99
    assert np.all(got[:, 5:] == 0)


def test_pool_closed_forms():
    """Rows equal to c within each cell pool to bf16(c * scale) exactly; a
    cell of 3 rows (1, 2, 3) averages to 2."""
    seq, heads = 35, 1
    x = np.zeros((seq, heads, 128), np.float32)
    x[:16] = 0.75
    x[16:32] = -1.5
    x[32:] = np.array([1, 2, 3], np.float32)[:, None, None]
    p = synth.bf16_to_f32(oracle.sb_pool(synth.f32_to_bf16(x), seq, heads, 0.5)).reshape(heads, -1, 128)
    assert np.all(p[0, 0] == 0.375) and np.all(p[0, 1] == -0.75) and np.all(p[0, 2] == 1.0)
    assert np.all(p[0, 3:] == 0)


def test_score_within_reference_tolerance():
    """Scores from the same pooled cells agree with the float64 double
    log-sum-exp within the reference's contract tolerance, ragged last block
    included."""
    seq, heads = 300, 2
    q, k, _ = native_inputs(seq, heads, 0)
    blocks = (seq + 63) // 64
    got = oracle.sb_score(oracle.sb_pool(q, seq, heads, QSCALE), oracle.sb_pool(k, seq, heads, 1.0), seq,
                          heads).reshape(heads, blocks, blocks)
    want = vectors()["sb_scores_300"]
    assert np.all(np.abs(got - want) <= score_tolerance(want))
    # Random pools at a larger scale exercise the tolerance's relative term.
    seq = 200
    qr, kr = random_pool_inputs()
    blocks = (seq + 63) // 64
    got = oracle.sb_score(oracle.sb_pool(qr, seq, 1, QSCALE), oracle.sb_pool(kr, seq, 1, 1.0), seq,
                          1).reshape(1, blocks, blocks)
    want = vectors()["sb_scores_200r"]
    assert np.all(np.abs(got - want) <= score_tolerance(want))


def test_score_closed_form():
    """Equal cell dots d give (d + log2(nq * nk)) * ln 2: nq, nk are the valid
    cells of each block (seq 100: blocks of 4 and 3 cells; the 3rd cell of the
    second block holds 4 rows)."""
    seq, heads = 100, 1
    q = np.zeros((seq, heads, 128), np.float32)
    k = np.zeros((seq, heads, 128), np.float32)
    q[:, :, 0] = 1.0
    k[:, :, 0] = 2.0
    qp = oracle.sb_pool(synth.f32_to_bf16(q), seq, heads, 1.0)
    kp = oracle.sb_pool(synth.f32_to_bf16(k), seq, heads, 1.0)
    s = oracle.sb_score(qp, kp, seq, heads).reshape(2, 2)
    n = [4, 3]
    for i in range(2):
        for j in range(2):
            want = (2.0 + math.log2(n[i] * n[j])) * math.log(2)
            assert abs(s[i, j] - want) < 1e-6, (i, j, s[i, j], want)


def test_select_matches_lexsort_and_ties():
    scores, kp, qp, keep = select_inputs()
    heads, blocks = scores.shape[:2]
    got = oracle.sb_select(scores, heads, blocks, keep, qp, kp).reshape(heads, blocks, blocks)
    assert np.array_equal(got, vectors()["sb_select_routes"])
    # All scores equal: the first `keep` indices win.
    flat = np.zeros((1, blocks, blocks), np.float32)
    got = oracle.sb_select(flat, 1, blocks, keep).reshape(blocks, blocks)
    assert np.all(got[:, :keep] == 1) and np.all(got[:, keep:] == 0)
    # Signed zeros compare equal (ranked by index).
    z = np.tile(np.array([-0.0, 1.0, 0.0, -1.0], np.float32), (1, 4, 1))
    assert list(oracle.sb_select(z, 1, 4, 2)[:4]) == [1, 1, 0, 0]


def test_routed_attention_brute_force():
    """Per-head routed softmax vs a float64 brute force over the visible keys;
    all-ones routes equal the dense oracle."""
    seq, heads = 150, 2
    rng = np.random.default_rng(3)
    q, k, v = (rng.standard_normal((seq, heads, 128)).astype(np.float32) for _ in range(3))
    blocks = 3
    routes = (rng.random((heads, blocks, blocks)) < 0.5).astype(np.uint8)
    routes[:, :, 1] = 1
    scale = float(SCALE)
    got = oracle.attention_routed(q, k, v, seq, heads, scale, routes).reshape(seq, heads, 128)
    for h in range(heads):
        for i in (0, 63, 64, 100, 149):
            vis = np.repeat(routes[h, i // 64].astype(bool), 64)[:seq]
            logits = k[vis, h].astype(np.float64) @ q[i, h].astype(np.float64) * scale
            w = np.exp(logits - logits.max())
            w /= w.sum()
            want = w @ v[vis, h].astype(np.float64)
            assert np.max(np.abs(got[i, h] - want)) < 1e-5
    ones = np.ones((heads, blocks, blocks), np.uint8)
    dense = oracle.attention(q, k, v, seq, heads, scale).reshape(seq, heads, 128)
    full = oracle.attention_routed(q, k, v, seq, heads, scale, ones).reshape(seq, heads, 128)
    assert np.max(np.abs(full - dense)) < 1e-5
