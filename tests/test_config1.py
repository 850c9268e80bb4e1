"""BASELINE config 1, the reference's CPU-runnable plumbing case: non-causal
softmax(QK^T / sqrt(D)) V at B = 1, H = 8, S = 1024, D = 128, Q, K, V FP16
N(0, 1) from seed 0 (numpy default_rng(0), standard_normal, cast to float16,
in the order Q, K, V), FP32 accumulation, online softmax over 64-key blocks
(the reference's host oracle semantics, cuda_attention.cuh:7-51).

CPU: the oracle on the full case against float64 brute force on sampled rows
(tests/metal_attention.c:55-67 recipe). GPU: the DiT attention entry on the
same inputs, rounded to BF16 (the boundary's input type), against the oracle
on the FP16 values within BASELINE's gate (max-abs <= 2e-2, cosine >= 0.999).
"""
import math

import numpy as np
import pytest

from h3cli_amd import synth
from oracle import oracle
from tests.helpers import ATTN_COSINE, metrics, sdpa

SEQ, HEADS, D = 1024, 8, 128
SCALE = 1.0 / math.sqrt(D)


def inputs():
    rng = np.random.default_rng(0)
    return [rng.standard_normal((SEQ, HEADS, D)).astype(np.float16) for _ in range(3)]


def test_config1_oracle_against_float64():
    q, k, v = (x.astype(np.float32) for x in inputs())
    out = oracle.attention(q, k, v, SEQ, HEADS, SCALE, tile=64)
    rows = [0, 1, 63, 64, 511, 1000, 1023]
    qd, kd, vd = (x.astype(np.float64) for x in (q, k, v))
    for r in rows:
        s = np.einsum("hd,shd->hs", qd[r], kd) * SCALE
        p = np.exp(s - s.max(axis=1, keepdims=True))
        want = np.einsum("hs,shd->hd", p / p.sum(axis=1, keepdims=True), vd)
        assert np.max(np.abs(out[r] - want)) < 1e-5, r


@pytest.mark.gpu
def test_config1_gpu_against_oracle():
    from h3cli_amd.runtime import Gpu
    q, k, v = inputs()
    ref = oracle.attention(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), SEQ, HEADS, SCALE, tile=64)
    with Gpu() as g:
        bits = [synth.f32_to_bf16(x.astype(np.float32).reshape(-1)) for x in (q, k, v)]
        # The DiT entry rounds the scale to BF16 as the reference does; the
        # plain SDPA entry takes it as given, like the host op.
        got = synth.bf16_to_f32(sdpa(g, *bits, SEQ, HEADS, SCALE, dit=False)).reshape(SEQ, HEADS, D)
    m = metrics(got, ref)
    assert m["max_abs"] <= 2e-2 and m["cosine"] >= ATTN_COSINE, m
