"""The synthetic DiT block of BASELINE config 5 composed through the C ABI
(include/h3_dit_synth.h, following the reference's run_block op sequence
src/denoise/dit.c:2286-2539) against the same block composed from the oracle's
ops, and the full 40-block config-5 step at its real size.

The small-geometry test traces one block (trace_block) and checks:
- every stage on the GPU's own input to that stage, at the per-op tolerances;
- the whole block chained through the oracle from the block input alone, so
  that composition errors (a wrong slot, operand or layout) cannot hide behind
  stage-local checks;
- the patch embedding, the output head and the Euler update around it."""
import math

import numpy as np
import pytest

from h3cli_amd import synth
from h3cli_amd.runtime import DitSynth
from oracle import oracle
from tests.helpers import ATTN_COSINE, ATTN_MAX_ABS, GEMM_REL_L2, bf16, metrics, scale_bf16
from tests.test_block_gpu import ulp_diff

pytestmark = pytest.mark.gpu

SMALL = dict(blocks=2, hidden=512, heads=4, mlp=1024, frames=2, height=8, width=32, audio_rows=128, latent=256,
             mask_density=0.25, seed=13, streamed_first=1, trace_block=1)
SLOTS = 6


def linear(x, codes, scales, rows, k, n, gelu=False):
    return oracle.linear_q8(x, codes, scales, rows, k, n, k, gelu=gelu)


def gemm_ok(got, x, codes, scales, rows, k, n, gelu=False):
    ref, ref64 = linear(x, codes, scales, rows, k, n, gelu)
    m = metrics(bf16(got), ref64)
    assert m["rel_l2"] < 0.006 and m["rel_l2"] <= GEMM_REL_L2, m
    assert np.mean(ulp_diff(got, ref) <= 1) > 0.99
    return ref


def attention_ok(mode, q, k, v, rows, heads, mask, got):
    """BF16 (mode 0) against the FP32 oracle; Sage (mode 1) against attention
    over the same quantized operands. V comes out of the projection at |v| of
    tens (BF16 step 0.125-0.25), so the absolute bound scales with the output
    magnitude. With BASELINE's weight distribution (int8 U[-127,127] x
    U[1e-3,1e-2], std ~0.4) the scores have a spread in the hundreds and the
    softmax is nearly one-hot: int8 Q/K rounding then moves which key wins on
    some rows, so Sage is held to the quantized-operand oracle here and to the
    BF16 oracle at config 3's inputs (tests/test_baseline_shapes_gpu.py)."""
    scale = scale_bf16(1 / math.sqrt(128))
    if mode == 0:
        ref = oracle.attention(bf16(q), bf16(k), bf16(v), rows, heads, scale, mask=mask, block=128)
    else:
        ref = oracle.sage_attention(oracle.sage_pack(q, k, v, rows, heads), rows, heads, scale, mask=mask, block=128)
    m = metrics(bf16(got), ref)
    print(f"[dit block] attention mode {mode}: {m}", flush=True)
    bound = ATTN_MAX_ABS * max(1.0, float(np.abs(ref).max()))
    assert m["cosine"] >= (ATTN_COSINE if mode == 0 else 0.9995) and m["max_abs"] <= bound, m


def bf16_attention(q, k, v, rows, heads, mask):
    scale = scale_bf16(1 / math.sqrt(128))
    ref = oracle.attention(bf16(q), bf16(k), bf16(v), rows, heads, scale, mask=mask, block=128)
    return synth.f32_to_bf16(ref.reshape(-1))


@pytest.mark.parametrize("mode", [1, 0])
def test_block_composition_against_oracle(mode):
    cfg = dict(SMALL, attention_mode=mode)
    print(f"[dit block] {cfg}", flush=True)
    dt = -0.05
    with DitSynth(**cfg) as m:
        R, H, I, F, L = m.rows, cfg["hidden"], cfg["heads"] * 128, cfg["mlp"], cfg["latent"]
        heads, eps = cfg["heads"], float(m.config.eps)
        latent0 = m.read("latent")
        w = {j: m.read_q8(f"blocks.0.{name}", n, k) for j, (name, n, k) in enumerate(
            [("attn.qkv_proj.weight", 3 * I, H), ("attn.out_proj.weight", H, I), ("mlp.fc1.weight", F, H),
             ("mlp.fc2.weight", H, F)])}
        norm1, norm2 = m.read("blocks.0.norm1.weight"), m.read("blocks.0.norm2.weight")
        mod = m.read("blocks.0.modulation")
        rmap, cos, sin = m.read("row_map"), m.read("rope_cos"), m.read("rope_sin")
        patch, head, head_norm, head_mod = m.read("patch"), m.read("head"), m.read("head_norm"), m.read("head_mod")
        m.step(step=0, dt=dt)
        t = {s: m.read(f"trace.{s}") for s in ("x0", "xn1", "qkv", "q", "k", "v", "attn", "o", "x1", "xn2", "h",
                                               "f", "x2")}
        latent_bf16, hidden, vel, latent1 = m.read("latent_bf16"), m.read("hidden"), m.read("velocity"), m.read("latent")
        video = cfg["frames"] * cfg["height"] * cfg["width"]
    mask = oracle.block_mask(R, video, 128, cfg["mask_density"], cfg["seed"])
    assert np.array_equal(rmap, (np.arange(R) >= video).astype(np.uint32))

    # Patch embedding of the BF16-rounded latent (BF16 weight).
    assert np.array_equal(latent_bf16, synth.f32_to_bf16(latent0))
    _, x0_64 = oracle.linear_bf16(latent_bf16, patch, R, L, H)
    assert metrics(bf16(t["x0"]), x0_64)["rel_l2"] < 0.006

    # Stage by stage on the GPU's own stage inputs.
    assert ulp_diff(t["xn1"], oracle.adaln(t["x0"], norm1, mod, rmap, R, H, SLOTS, 0, 1, eps)).max() <= 1
    gemm_ok(t["qkv"], t["xn1"], *w[0], R, H, 3 * I)
    rq, rk, rv = oracle.qkv_rope(t["qkv"], None, None, cos, sin, R, heads, 128, 64, eps, 0)
    assert np.array_equal(t["v"], rv)
    assert ulp_diff(t["q"], rq).max() <= 1 and ulp_diff(t["k"], rk).max() <= 1
    attention_ok(mode, t["q"], t["k"], t["v"], R, heads, mask, t["attn"])
    gemm_ok(t["o"], t["attn"], *w[1], R, I, H)
    assert np.array_equal(t["x1"], oracle.gate(t["x0"], t["o"], mod, rmap, R, H, SLOTS, 2))
    assert ulp_diff(t["xn2"], oracle.adaln(t["x1"], norm2, mod, rmap, R, H, SLOTS, 3, 4, eps)).max() <= 1
    gemm_ok(t["h"], t["xn2"], *w[2], R, H, F, gelu=True)
    gemm_ok(t["f"], t["h"], *w[3], R, F, H)
    assert np.array_equal(t["x2"], oracle.gate(t["x1"], t["f"], mod, rmap, R, H, SLOTS, 5))

    # The whole block chained through the oracle from the block input alone.
    xn1 = oracle.adaln(t["x0"], norm1, mod, rmap, R, H, SLOTS, 0, 1, eps)
    qkv, _ = linear(xn1, *w[0], R, H, 3 * I)
    q, k, v = oracle.qkv_rope(qkv, None, None, cos, sin, R, heads, 128, 64, eps, 0)
    # BF16 attention is chained too. Sage is not: one-ulp differences in the
    # chained projections change some int8 Q/K codes, and with the nearly
    # one-hot softmax of these weights a changed code moves a whole row's
    # winning key (2% rel-L2 measured), so in Sage mode the chain continues
    # from the GPU's attention output, which the stage check above holds to
    # the quantized-operand oracle.
    att = bf16_attention(q, k, v, R, heads, mask) if mode == 0 else t["attn"]
    o, _ = linear(att, *w[1], R, I, H)
    x1 = oracle.gate(t["x0"], o, mod, rmap, R, H, SLOTS, 2)
    xn2 = oracle.adaln(x1, norm2, mod, rmap, R, H, SLOTS, 3, 4, eps)
    h, _ = linear(xn2, *w[2], R, H, F, gelu=True)
    f, _ = linear(h, *w[3], R, F, H)
    x2 = oracle.gate(x1, f, mod, rmap, R, H, SLOTS, 5)
    for name, ref in (("qkv", qkv), ("attn", att), ("x1", x1), ("x2", x2)):
        met = metrics(bf16(t[name]), bf16(ref))
        print(f"[dit block] chained {name}: {met}", flush=True)
        # One-ulp differences in the projections move the chained inputs of
        # every later stage; each stays within the GEMM gate.
        assert met["cosine"] >= ATTN_COSINE and met["rel_l2"] <= GEMM_REL_L2, (name, met)

    # Output head on the last block's output, then the Euler update.
    hn = oracle.adaln(hidden, head_norm, head_mod, rmap, R, H, 2, 0, 1, eps)
    _, v64 = oracle.linear_bf16(hn, head, R, H, L)
    assert metrics(bf16(vel), v64)["rel_l2"] < 0.01
    expect = oracle.euler(latent0, vel, vel, dt, 0.0)
    assert np.array_equal(latent1.view(np.uint32), expect.view(np.uint32))


def test_full_config5_step():
    """BASELINE config 5 at its real size: 40 blocks, 33424 rows, hidden 5120,
    Sage attention over the 25%-density mask, blocks 20-39 streamed from
    pinned host memory. One step is finite and moves the latent; a second
    model with every block resident gives the same latent bit for bit (the
    streamed slots hold exactly the resident weights, and the ordering on the
    copy stream is right); a rerun of the streamed model is bit-identical."""
    outs = []
    for streamed_first in (20, 40, 20):
        print(f"[config5 step] streamed_first={streamed_first}", flush=True)
        with DitSynth(streamed_first=streamed_first) as m:
            assert m.rows == 33424 and m.config.blocks == 40 and m.config.hidden == 5120
            before = m.read("latent")
            m.step(step=0, dt=-0.02)
            outs.append((before, m.read("latent"), m.read("hidden")))
    before, lat, hid = outs[0]
    assert np.all(np.isfinite(lat)) and np.all(np.isfinite(bf16(hid)))
    assert not np.array_equal(before, lat)
    for other in outs[1:]:
        assert np.array_equal(other[1].view(np.uint32), lat.view(np.uint32))
        assert np.array_equal(other[2], hid)
