"""Inputs and layouts of the routed-attention tests (SubBlock mode 4, SOL mode 3).

Input recipes only: the expected values these inputs lead to come from the
C oracle and from vectors in tests/golden/router_vectors.npz, written by
tests/golden/make_router_vectors.py with the reference's own NumPy oracles."""
import ctypes as C
from pathlib import Path

import numpy as np

from h3cli_amd import synth
from h3cli_amd._lib import SolBlock, SolLayout

VECTORS = Path(__file__).resolve().parent / "golden" / "router_vectors.npz"


def vectors():
    """The committed golden vectors (plain arrays; no pickled objects)."""
    return np.load(VECTORS, allow_pickle=False)


def native_inputs(seq, heads, kind):
    """Q, K, V BF16 bits [seq, heads, 128] of the reference's native SubBlock
    operator test (tests/subblock_native.cu:21-27): kind 0 integer ramps
    scaled by 1/32 (V by 1/40); 1 zero Q and K with V = 0.5; 2 kind 0 with a
    NaN in the last Q element; 3 Q = 100 and K = -100/+100 by element parity;
    4 kind 0 (its layout protects the first and last blocks). Products are
    taken in float32 as that test does (the V step 0.025 is not a power of
    two)."""
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
        k[:] = synth.f32_to_bf16(np.where(i % 2 == 1, np.float32(100), np.float32(-100)))
    return tuple(x.reshape(seq, heads, 128) for x in (q, k, v))


# (seq, heads, kind) of the GPU router tests; kind 9 is seeded Gaussian input.
SUBBLOCK_GPU_CASES = [(4200, 2, 0), (4200, 2, 4), (5000, 3, 9), (4160, 1, 3)]
# (seq, q_block, protected, all_protected) of every SOL layout the tests bind.
SOL_EXACT = [(s, q) for s in (1, 31, 32, 33, 63, 64, 65, 127, 128, 129, 257, 1025) for q in (32, 64)]
SOL_LAYOUTS = sorted({(s, q, False, False) for s, q in SOL_EXACT} | {
    (513, 32, True, False), (513, 64, False, False), (257, 32, False, True), (257, 32, False, False),
    (128, 32, False, False), (4103, 32, False, False), (4103, 64, False, False), (65, 32, False, False),
    (300, 32, False, False), (300, 64, False, False), (1000, 32, True, False), (1000, 32, False, False)})
# (minimum_exact, tau, local_radius) option sets of the SOL route pins.
SOL_ROUTE_OPTIONS = [(0.0, 1.0, 1), (0.5, 1.0, 0), (0.0, 0.25, 3), (0.0, 16.0, 0)]
SOL_ATTENTION_ROWS = [0, 31, 32, 100, 200, 259]


def random_pool_inputs():
    """Q and K BF16 [200, 1, 128], 3 N(0,1), for the score pin at a scale where
    the contract tolerance's relative term matters."""
    rng = np.random.default_rng(5)
    q = synth.f32_to_bf16(rng.standard_normal((200, 1, 128)).astype(np.float32) * 3)
    k = synth.f32_to_bf16(rng.standard_normal((200, 1, 128)).astype(np.float32) * 3)
    return q, k


def select_inputs():
    """Tie-heavy integer scores [2, 37, 37], protected key blocks 3 and 30 and
    protected first/last query blocks, keep 8."""
    rng = np.random.default_rng(9)
    heads, blocks, keep = 2, 37, 8
    scores = rng.integers(-4, 4, (heads, blocks, blocks)).astype(np.float32)
    kp = np.zeros(blocks, np.uint8)
    kp[[3, 30]] = 1
    return scores, kp, protect_ends(blocks * 64), keep


def subblock_case_inputs(seq, heads, kind):
    """kind 9: seeded Gaussian Q, K, V (structure the router can rank)."""
    if kind == 9:
        return tuple(x.reshape(seq, heads, 128) for x in synth.attention_inputs(seq, heads, seed=seq, scale=1.0))
    return native_inputs(seq, heads, kind)


def protect_ends(seq):
    p = np.zeros((seq + 63) // 64, np.uint8)
    p[[0, -1]] = 1
    return p


def sol_inputs(seq, heads, seed=1701, pattern="random"):
    """BF16 bits Q, K, V [seq, heads, 128] for the SOL operator cases: 0.5 N(0,1)
    from the documented generator, and the acceptance patterns: zero (all
    zero), constant (K = 0.2, V = 0.7), extreme (Q and K x 40), spike (K of the
    middle row x 32), nan (the last Q element)."""
    n = seq * heads * 128
    x = np.stack([(synth.normal(seed * 16 + i, n) * 0.5).astype(np.float32).reshape(seq, heads, 128)
                  for i in range(3)])
    if pattern == "zero":
        x[:] = 0
    elif pattern == "constant":
        x[1] = 0.2
        x[2] = 0.7
    elif pattern == "extreme":
        x[:2] *= 40
    elif pattern == "spike":
        x[1, seq // 2] *= 32
    elif pattern == "nan":
        x[0, -1, -1, 0] = np.nan
    return [synth.f32_to_bf16(a) for a in x]


def sol_layout_name(seq, qb, protected=False, all_protected=False):
    """Key of a SOL layout in the golden vectors."""
    tag = "all" if all_protected else "prot" if protected else "open"
    return f"sol_layout_{seq}_{qb}_{tag}"


def sol_layout(seq, qb, protected=False, all_protected=False):
    """int32 [blocks, 4] (protect, first_frame, last_frame, rows) for query
    blocks of qb rows and 64-row key blocks: the reference's acceptance layouts
    as its oracle builds them, from the golden vectors."""
    v = vectors()
    key = sol_layout_name(seq, qb, protected, all_protected)
    return [np.asarray(v[key + "_q"]), np.asarray(v[key + "_k"])]


class Layout:
    """A ctypes h3_sol_layout. meta: [query, key] int32 [blocks, 4] arrays, or
    None with q_protect / k_protect flags for 64-row SubBlock blocks."""

    def __init__(self, seq, meta=None, q_protect=None, k_protect=None):
        if meta is None:
            blocks = (seq + 63) // 64
            rows = np.minimum(64, seq - 64 * np.arange(blocks))
            meta = []
            for flags in (q_protect, k_protect):
                m = np.zeros((blocks, 4), np.int32)
                m[:, 0] = 0 if flags is None else np.asarray(flags, np.int32)
                m[:, 3] = rows
                meta.append(m)
        self.arrays = []
        for m in meta:
            arr = (SolBlock * len(m))()
            for i, (p, f0, f1, rows) in enumerate(np.asarray(m)):
                arr[i].protect, arr[i].first_frame, arr[i].last_frame, arr[i].rows = int(p), int(f0), int(f1), int(rows)
            self.arrays.append(arr)
        self.layout = SolLayout(seq, len(meta[0]), len(meta[1]), 0, C.cast(self.arrays[0], C.POINTER(SolBlock)),
                                C.cast(self.arrays[1], C.POINTER(SolBlock)))

    @property
    def ptr(self):
        return C.addressof(self.layout)
