"""SubBlock router fixtures and independent checks.

Inputs follow the reference's native operator test (tests/subblock_native.cu:
21-27, kinds 0-4); the float64 pooled-score formulation, the lexsort selection
and the contract tolerance follow the reference's independent oracle
(tests/subblock_oracle.py:21-83). These are the checkers the C restatement in
oracle/ and the HIP router are compared with.
"""
import ctypes as C

import numpy as np

from h3cli_amd import synth
from h3cli_amd._lib import SolBlock, SolLayout


def native_inputs(seq, heads, kind):
    """Q, K, V BF16 bits [seq, heads, 128] of subblock_native.cu:21-27:
    kind 0 integer ramps, 1 zero Q/K with V = 0.5, 2 kind 0 with a NaN in the
    last Q element, 3 Q = 100 and K = +-100 by element parity, 4 kind 0 (the
    first and last blocks are protected by the layout)."""
    n = seq * heads * 128
    i = np.arange(n, dtype=np.int64)
    if kind == 1:
        q = np.zeros(n, np.float32)
        k = np.zeros(n, np.float32)
        v = np.full(n, 0.5, np.float32)
    else:
        q = ((i * 7 + 3) % 71 - 35).astype(np.float32) * np.float32(0.03125)
        k = ((i * 11 + 1) % 67 - 33).astype(np.float32) * np.float32(0.03125)
        v = ((i * 13 + 5) % 79 - 39).astype(np.float32) * np.float32(0.025)
    q, k, v = (synth.f32_to_bf16(x) for x in (q, k, v))
    if kind == 2:
        q[-1] = 0x7FC0
    if kind == 3:
        q[:] = synth.f32_to_bf16(np.float32(100))
        k[:] = np.where(i % 2 == 1, synth.f32_to_bf16(np.float32(100)), synth.f32_to_bf16(np.float32(-100)))
    return (x.reshape(seq, heads, 128) for x in (q, k, v))


def protect_ends(seq):
    blocks = (seq + 63) // 64
    p = np.zeros(blocks, np.uint8)
    p[[0, -1]] = 1
    return p


class Layout:
    """A ctypes h3_sol_layout with 64-row query and key blocks."""

    def __init__(self, seq, q_protect=None, k_protect=None):
        blocks = (seq + 63) // 64
        self.q = (SolBlock * blocks)()
        self.k = (SolBlock * blocks)()
        for b in range(blocks):
            rows = min(64, seq - b * 64)
            self.q[b].rows = self.k[b].rows = rows
            self.q[b].protect = int(q_protect[b]) if q_protect is not None else 0
            self.k[b].protect = int(k_protect[b]) if k_protect is not None else 0
        self.layout = SolLayout(seq, blocks, blocks, 0, C.cast(self.q, C.POINTER(SolBlock)),
                                C.cast(self.k, C.POINTER(SolBlock)))

    @property
    def ptr(self):
        return C.addressof(self.layout)


def f64_pool(x, seq, heads, scale):
    """Cell means in float64, times scale in fp32, rounded to BF16
    (subblock_oracle.py:21-28). x: float32 [seq, heads, 128]."""
    cells = (seq + 63) // 64 * 4
    out = np.zeros((heads, cells, 128), np.float32)
    for c in range((seq + 15) // 16):
        mean = x[c * 16:min(seq, c * 16 + 16)].astype(np.float64).mean(axis=0).astype(np.float32)
        out[:, c] = synth.bf16_to_f32(synth.f32_to_bf16(mean * np.float32(scale)))
    return out


def _lse(x, axis):
    top = x.max(axis=axis, keepdims=True)
    return (top + np.log2(np.exp2(x - top).sum(axis=axis, keepdims=True))).squeeze(axis)


def f64_scores(qp, kp, seq):
    """Block scores from pooled cells [heads, cells, 128] in float64
    (subblock_oracle.py:47-54)."""
    heads = qp.shape[0]
    blocks = (seq + 63) // 64
    valid = (seq + 15) // 16
    out = np.empty((heads, blocks, blocks), np.float64)
    for h in range(heads):
        dots = qp[h].astype(np.float64) @ kp[h].astype(np.float64).T
        for i in range(blocks):
            for j in range(blocks):
                cell = dots[i * 4:min(i * 4 + 4, valid), j * 4:min(j * 4 + 4, valid)]
                out[h, i, j] = _lse(_lse(cell, 1), 0) * np.log(2)
    return out


def score_tolerance(expected):
    """Contract tolerance of pooled scores (subblock_oracle.py:60)."""
    return 2e-4 + 2e-5 * np.abs(expected)


def lexsort_routes(scores, keep, q_protect=None, k_protect=None, force=False):
    """Selection by descending score then ascending index, plus protection
    (subblock_oracle.py:64-74). scores: [heads, B, B]."""
    heads, blocks, _ = scores.shape
    kp = np.zeros(blocks, bool) if k_protect is None else np.asarray(k_protect, bool)
    qp = np.zeros(blocks, bool) if q_protect is None else np.asarray(q_protect, bool)
    routes = np.zeros((heads, blocks, blocks), np.uint8)
    for h in range(heads):
        for i in range(blocks):
            order = np.lexsort((np.arange(blocks), -scores[h, i]))
            row = kp.copy()
            row[order[:keep]] = True
            if force or qp[i]:
                row[:] = True
            routes[h, i] = row
    return routes


def separated_rows(expected, keep):
    """(h, i) rows whose keep-th and (keep+1)-th scores differ by more than
    twice the tolerance, where routes must match the float64 selection
    (subblock_oracle.py:75-80)."""
    heads, blocks, _ = expected.shape
    tol = score_tolerance(expected)
    rows = []
    if keep >= blocks:
        return rows
    for h in range(heads):
        for i in range(blocks):
            order = np.lexsort((np.arange(blocks), -expected[h, i]))
            if expected[h, i, order[keep - 1]] - expected[h, i, order[keep]] > 2 * tol[h, i].max():
                rows.append((h, i))
    return rows
