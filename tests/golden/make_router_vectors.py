"""Writes tests/golden/router_vectors.npz: expected values of the SubBlock and
SOL routers computed by the reference's own NumPy oracles,
/root/reference/tests/subblock_oracle.py and /root/reference/tests/cuda_sol_oracle.py,
imported from the reference tree in the build container (numpy only; this
script never runs on the GPU box, and the vectors are plain arrays).

    python tests/golden/make_router_vectors.py

What each vector is:
- sb_pool_*: the reference's `pool` (float64 cell means, fp32 scale, BF16).
- sb_scores_*: block scores as the reference's validator defines them
  (subblock_oracle.py:47-54: a log-sum-exp over key cells, then over query
  cells, of float64 dots of pooled cells, times ln 2), on the C oracle's
  pooled cells (which the GPU reproduces bit for bit).
- sb_routes_* / sb_separated_*: the reference's selection rule
  (subblock_oracle.py:64-80: descending score, ascending index, protected
  blocks) on those scores, and the rows whose keep-th gap exceeds twice the
  contract tolerance, where any implementation must agree with it.
- sol_layout_*: the acceptance layouts the reference's oracle builds
  (cuda_sol_oracle.py:14-22).
- sol_summary_*, sol_routes_*, sol_separated_*, sol_out_*: the reference's
  `summaries`, `routes` (on the C oracle's centroids) and `reference` softmax.

The script also runs the reference's validator (`validate`) on the C oracle's
SubBlock outputs for two native cases, so the oracle is accepted by the
reference's own checker before its vectors are written."""
import ctypes as C
import importlib.util
import math
import sys
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from h3cli_amd import _lib, synth  # noqa: E402
from oracle import oracle  # noqa: E402
from tests import router_inputs as ri  # noqa: E402

REF_TESTS = Path("/root/reference/tests")
OUT = Path(__file__).resolve().parent / "router_vectors.npz"
SCALE = np.float32(1 / math.sqrt(128))
QSCALE = np.float32(SCALE * np.float32(math.log2(math.e)))
SOL_SCALE = float(synth.bf16_to_f32(synth.f32_to_bf16(np.float32(1 / math.sqrt(128)))))


def reference_module(name):
    spec = importlib.util.spec_from_file_location(f"reference_{name}", REF_TESTS / f"{name}.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


sb = reference_module("subblock_oracle")
so = reference_module("cuda_sol_oracle")


def sb_scores(qp, kp, seq):
    """subblock_oracle.py:47-54 with the reference's `lse`."""
    heads, blocks = qp.shape[0], (seq + 63) // 64
    valid = (seq + 15) // 16
    out = np.empty((heads, blocks, blocks), np.float64)
    for h in range(heads):
        dots = qp[h].astype(np.float64) @ kp[h].astype(np.float64).T
        for i in range(blocks):
            for j in range(blocks):
                out[h, i, j] = sb.lse(sb.lse(dots[i * 4:min(i * 4 + 4, valid), j * 4:min(j * 4 + 4, valid)], 1),
                                      0) * np.log(2)
    return out


def sb_select(scores, keep, q_protect, k_protect):
    """subblock_oracle.py:64-74: routes of every (head, query block)."""
    heads, blocks, _ = scores.shape
    kp = np.zeros(blocks, bool) if k_protect is None else np.asarray(k_protect, bool)
    qp = np.zeros(blocks, bool) if q_protect is None else np.asarray(q_protect, bool)
    routes = np.zeros((heads, blocks, blocks), np.uint8)
    for h in range(heads):
        for i in range(blocks):
            order = np.lexsort((np.arange(blocks), -scores[h, i]))
            row = kp.copy()
            row[order[:keep]] = True
            if qp[i]:
                row[:] = True
            routes[h, i] = row
    return routes


def sb_separated(scores, keep):
    """subblock_oracle.py:75-80: rows whose keep-th gap exceeds twice the
    contract tolerance 2e-4 + 2e-5 |s|."""
    heads, blocks, _ = scores.shape
    tol = 2e-4 + 2e-5 * np.abs(scores)
    sep = np.zeros((heads, blocks), bool)
    if keep >= blocks:
        return sep
    for h in range(heads):
        for i in range(blocks):
            order = np.lexsort((np.arange(blocks), -scores[h, i]))
            sep[h, i] = scores[h, i, order[keep - 1]] - scores[h, i, order[keep]] > 2 * tol[h, i].max()
    return sep


def oracle_pools(q, k, seq, heads):
    qp = synth.bf16_to_f32(oracle.sb_pool(q, seq, heads, QSCALE)).reshape(heads, -1, 128)
    kp = synth.bf16_to_f32(oracle.sb_pool(k, seq, heads, 1.0)).reshape(heads, -1, 128)
    return qp, kp


def keep_of(blocks, sparsity=0.75):
    return _lib.load().h3_subblock_budget(blocks, C.c_float(sparsity))


def validate_oracle(seq, heads, kind, sparsity=0.75):
    """Run the reference's validator on the C oracle's scores, routes and
    routed outputs for one native case."""
    q, k, v = ri.native_inputs(seq, heads, kind)
    blocks = (seq + 63) // 64
    keep = min(blocks, 8 * int(np.ceil((1 - float(np.float32(sparsity))) * blocks / 8)))
    assert keep == keep_of(blocks, sparsity)
    scores = oracle.sb_score(oracle.sb_pool(q, seq, heads, QSCALE), oracle.sb_pool(k, seq, heads, 1.0), seq, heads)
    prot = ri.protect_ends(seq) if kind == 4 else None
    routes = oracle.sb_select(scores, heads, blocks, keep, prot, prot)
    out = oracle.attention_routed(synth.bf16_to_f32(q), synth.bf16_to_f32(k), synth.bf16_to_f32(v), seq, heads,
                                  float(SCALE), routes).reshape(seq, heads, 128)
    row = synth.f32_to_bf16(out)
    with tempfile.TemporaryDirectory() as d:
        base = Path(d) / "case"
        for name, x in (("q", q), ("k", k), ("v", v)):
            np.ascontiguousarray(x, np.uint16).tofile(str(base) + f".{name}.bf16")
        scores.astype(np.float32).tofile(str(base) + ".scores")
        routes.astype(np.uint8).tofile(str(base) + ".routes")
        row.tofile(str(base) + ".row.bf16")
        np.ascontiguousarray(row.transpose(1, 0, 2)).tofile(str(base) + ".head.bf16")
        result = sb.validate(base, seq, heads, sparsity, False, kind)
    print(f"reference validator accepted the oracle on S={seq} H={heads} kind={kind}: {result}")


def main():
    v = {}
    # ---- SubBlock (CPU oracle pins)
    q, _, _ = ri.native_inputs(69, 3, 0)
    v["sb_pool_69_q"] = sb.pool(synth.bf16_to_f32(q), QSCALE)
    q, k, _ = ri.native_inputs(300, 2, 0)
    v["sb_scores_300"] = sb_scores(*oracle_pools(q, k, 300, 2), 300)
    qr, kr = ri.random_pool_inputs()
    v["sb_scores_200r"] = sb_scores(*oracle_pools(qr, kr, 200, 1), 200)
    scores, kp, qp, keep = ri.select_inputs()
    v["sb_select_routes"] = sb_select(scores, keep, qp, kp)
    # ---- SubBlock (GPU cases: expected scores on the pooled cells the GPU reproduces)
    for seq, heads, kind in ri.SUBBLOCK_GPU_CASES:
        q, k, _ = ri.subblock_case_inputs(seq, heads, kind)
        expected = sb_scores(*oracle_pools(q, k, seq, heads), seq)
        blocks = (seq + 63) // 64
        keep = keep_of(blocks)
        prot = ri.protect_ends(seq) if kind == 4 else None
        tag = f"{seq}_{heads}_{kind}"
        v[f"sb_scores_{tag}"] = expected
        v[f"sb_routes_{tag}"] = sb_select(expected, keep, prot, prot)
        v[f"sb_separated_{tag}"] = sb_separated(expected, keep)
    for kind in (0, 4):
        validate_oracle(2048, 2, kind)

    # ---- SOL layouts of every case the tests bind
    for seq, qb, protected, all_protected in ri.SOL_LAYOUTS:
        meta = so.metadata(seq, qb, protected, all_protected)
        key = ri.sol_layout_name(seq, qb, protected, all_protected)
        v[key + "_q"], v[key + "_k"] = meta[0].astype(np.int32), meta[1].astype(np.int32)
    # ---- SOL centroids (CPU pin)
    seq, heads = 300, 2
    q, k, _ = ri.sol_inputs(seq, heads, seed=3)
    for name, x, b in (("q32", q, 32), ("q64", q, 64), ("k64", k, 64)):
        v[f"sol_summary_300_{name}"] = so.summaries(synth.bf16_to_f32(x), b)
    # ---- SOL routes on the C oracle's centroids, with the pairs a tiny change
    # of tau flips (near ties) marked as not separated.
    seq, heads, qb = 1000, 3, 32
    q, k, _ = ri.sol_inputs(seq, heads, seed=5)
    meta = so.metadata(seq, qb, True)
    qc = synth.bf16_to_f32(oracle.sol_summary(q, seq, heads, qb)).reshape(heads, -1, 128)
    kc = synth.bf16_to_f32(oracle.sol_summary(k, seq, heads, 64)).reshape(heads, -1, 128)
    for n, (minimum, tau, radius) in enumerate(ri.SOL_ROUTE_OPTIONS):
        routes, sep = [], []
        for h in range(heads):
            r = so.routes(qc[h], kc[h], meta, SOL_SCALE, minimum, tau, radius)
            lo = so.routes(qc[h], kc[h], meta, SOL_SCALE, minimum, tau * (1 - 1e-5), radius)
            hi = so.routes(qc[h], kc[h], meta, SOL_SCALE, minimum, tau * (1 + 1e-5), radius)
            routes.append(r)
            sep.append(lo == hi)
        v[f"sol_routes_{n}"] = np.array(routes, np.uint8)
        v[f"sol_separated_{n}"] = np.array(sep, bool)
    # ---- SOL attention: the reference's exact + centroid softmax and its routes
    seq, heads, qb = 260, 2, 32
    q, k, vv = ri.sol_inputs(seq, heads, seed=9)
    meta = so.metadata(seq, qb)
    rows = ri.SOL_ATTENTION_ROWS
    out, masks = so.reference(synth.bf16_to_f32(q), synth.bf16_to_f32(k), synth.bf16_to_f32(vv), meta, qb, 0.0,
                              0.5, 0, indices=rows)
    v["sol_out_260"] = out
    v["sol_masks_260"] = masks
    np.savez_compressed(OUT, **v)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(v)} arrays)")


if __name__ == "__main__":
    main()
