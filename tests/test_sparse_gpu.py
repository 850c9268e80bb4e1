"""Block-sparse DiT attention (BF16 and Sage) on the GPU vs the masked CPU oracle;
the synthetic mask builder bit-exact vs its numpy restatement."""
import math

import numpy as np
import pytest

from h3cli_amd import synth
from h3cli_amd.runtime import Gpu
from oracle import oracle
from tests.helpers import ATTN_COSINE, ATTN_MAX_ABS, bf16, metrics, scale_bf16, sdpa
from tests.test_sage_gpu import sage_inputs

pytestmark = pytest.mark.gpu


def bind_mask(gpu, mask):
    qb, kb = mask.shape
    m = np.ascontiguousarray(mask, np.uint8)
    gpu.check(gpu.lib.h3_hip_dit_block_mask(gpu.handle, m.ctypes.data, qb, kb, 128), "bind mask")


def make_gpu(mode):
    g = Gpu()
    g.check(g.lib.h3_gpu_dit_attention_configure(g.handle, mode), "configure")
    return g


@pytest.mark.parametrize("mode,seq,video", [(0, 1000, 900), (0, 2100, 1700), (4, 4200, 3800)])
def test_masked_bf16(mode, seq, video):
    print(f"[sparse bf16] mode={mode} seq={seq}", flush=True)
    g = make_gpu(mode)
    try:
        if mode == 4:
            g.check(g.lib.h3_gpu_dit_attention_noise(g.handle, 0, 0.5, 0.5), "noise")
            # Warmup off; block 1 of a sequence above the 4096-row "short"
            # threshold is not bypassed, so the bound mask applies.
            g.check(g.lib.h3_hip_dit_subblock_policy(g.handle, 0.75, -1), "policy")
        mask = oracle.block_mask(seq, video, 128, 0.25, seed=seq)
        bind_mask(g, mask)
        q, k, v = synth.attention_inputs(seq, 2, seed=seq, scale=1.0)
        out = bf16(sdpa(g, q, k, v, seq, 2))
        scale = scale_bf16(1 / math.sqrt(128))
        ref = oracle.attention(bf16(q), bf16(k), bf16(v), seq, 2, scale, mask=mask, block=128)
        m = metrics(out, ref)
        assert m["max_abs"] <= ATTN_MAX_ABS and m["cosine"] >= ATTN_COSINE, m
    finally:
        g.close()


def test_masked_sage():
    seq, video, heads = 1500, 1200, 2
    print(f"[sparse sage] seq={seq}", flush=True)
    g = make_gpu(1)
    try:
        mask = oracle.block_mask(seq, video, 128, 0.25, seed=3)
        bind_mask(g, mask)
        q, k, v = sage_inputs(seq, heads, seed=13)
        out = bf16(sdpa(g, q, k, v, seq, heads))
        scale = scale_bf16(1 / math.sqrt(128))
        ref = oracle.attention(bf16(q), bf16(k), bf16(v), seq, heads, scale, mask=mask, block=128)
        m = metrics(out, ref)
        assert m["cosine"] >= ATTN_COSINE, m
        pack = oracle.sage_pack(q, k, v, seq, heads)
        mq = metrics(out, oracle.sage_attention(pack, seq, heads, scale, mask=mask, block=128))
        assert mq["cosine"] >= 0.9995, mq
    finally:
        g.close()


def test_masked_sage_large_logit_scale():
    """Block-sparse Sage with Q and K at 400x (logit scale c ~ 30): every wave
    of the fast launch is flagged and the exact launch recomputes its rows
    over the same tile lists. Finite and within tolerance of the masked
    quantized-operand oracle."""
    seq, video, heads = 1500, 1200, 2
    print(f"[sparse sage large logits] seq={seq}", flush=True)
    g = make_gpu(1)
    try:
        mask = oracle.block_mask(seq, video, 128, 0.25, seed=3)
        bind_mask(g, mask)
        q, k, v = sage_inputs(seq, heads, seed=13)
        q = synth.f32_to_bf16(bf16(q) * 400.0)
        k = synth.f32_to_bf16(bf16(k) * 400.0)
        out = bf16(sdpa(g, q, k, v, seq, heads))
        assert np.all(np.isfinite(out))
        scale = scale_bf16(1 / math.sqrt(128))
        pack = oracle.sage_pack(q, k, v, seq, heads)
        mq = metrics(out, oracle.sage_attention(pack, seq, heads, scale, mask=mask, block=128))
        assert mq["cosine"] >= 0.99, mq
    finally:
        g.close()


@pytest.mark.parametrize("mode", [0, 1])
def test_masked_list_lengths(mode):
    """Tile lists of every length the kernels can meet: a query block with no
    kept block (its rows are zeros), one with only the last block (one tile
    with keys, one wholly past S: S = 960 ends on a tile boundary), one with
    only the first block, one with the first and the last; the other rows
    random. BF16 (mode 0) against the masked oracle; Sage (mode 1) against
    the masked quantized-operand oracle (rows that see only 128 or 256 keys
    have outputs near 1, where the int8/fp8 operands alone put the quantized
    oracle up to 0.057 from the FP32 one), with the same cosine gate against
    the FP32 oracle as the other masked Sage tests."""
    seq, heads = 960, 2
    print(f"[sparse list lengths] mode={mode} seq={seq}", flush=True)
    nb = (seq + 127) // 128
    rng = np.random.default_rng(5)
    mask = (rng.random((nb, nb)) < 0.3).astype(np.uint8)
    mask[0, :] = 0
    mask[1, :] = 0; mask[1, nb - 1] = 1
    mask[2, :] = 0; mask[2, 0] = 1
    mask[3, :] = 0; mask[3, 0] = 1; mask[3, nb - 1] = 1
    g = make_gpu(mode)
    try:
        bind_mask(g, mask)
        if mode == 1:
            q, k, v = sage_inputs(seq, heads, seed=17)
        else:
            q, k, v = synth.attention_inputs(seq, heads, seed=17, scale=1.0)
        out = bf16(sdpa(g, q, k, v, seq, heads))
        assert np.all(out[:128] == 0.0)
        scale = scale_bf16(1 / math.sqrt(128))
        ref = oracle.attention(bf16(q), bf16(k), bf16(v), seq, heads, scale, mask=mask, block=128)
        m = metrics(out, ref)
        if mode == 0:
            assert m["max_abs"] <= ATTN_MAX_ABS and m["cosine"] >= ATTN_COSINE, m
            return
        assert m["cosine"] >= ATTN_COSINE, m
        refq = oracle.sage_attention(oracle.sage_pack(q, k, v, seq, heads), seq, heads, scale, mask=mask, block=128)
        mq = metrics(out, refq)
        bound = ATTN_MAX_ABS * max(1.0, float(np.abs(refq).max()))
        assert mq["cosine"] >= 0.9995 and mq["max_abs"] <= bound, (mq, bound)
    finally:
        g.close()


def test_masked_sage_global_load_path(monkeypatch):
    """The block-sparse Sage kernel's buffer-load path and its global-load path
    (attention variant 13, what operands of 4 GiB and more take) agree bit for
    bit."""
    seq, video, heads = 1500, 1200, 2
    mask = oracle.block_mask(seq, video, 128, 0.25, seed=3)
    q, k, v = sage_inputs(seq, heads, seed=13)
    outs = []
    for variant in ("0", "13"):
        monkeypatch.setenv("H3_HIP_ATTENTION_VARIANT", variant)
        g = make_gpu(1)
        try:
            bind_mask(g, mask)
            outs.append(sdpa(g, q, k, v, seq, heads))
        finally:
            g.close()
    assert np.array_equal(outs[0], outs[1])


def test_subblock_requires_mask_and_step():
    g = make_gpu(4)
    try:
        seq = 4200
        q, k, v = synth.attention_inputs(seq, 1, seed=1)
        with pytest.raises(RuntimeError):
            sdpa(g, q, k, v, seq, 1, step=0)  # step not bound
        g.check(g.lib.h3_gpu_dit_attention_noise(g.handle, 12, 0.5, 0.5), "noise")
        with pytest.raises(RuntimeError):
            sdpa(g, q, k, v, seq, 1, step=12, block=3)  # sparse call without a bound mask
    finally:
        g.close()


def test_subblock_dense_bypass_matches_dense():
    """Calls for which the reference's bypass rules apply (warmup steps, probe
    block 0, short sequences) run dense even with a mask bound."""
    seq, video = 1000, 900
    g = make_gpu(4)
    d = Gpu()
    try:
        bind_mask(g, oracle.block_mask(seq, video, 128, 0.25, seed=1))
        q, k, v = synth.attention_inputs(seq, 2, seed=5)
        dense = sdpa(d, q, k, v, seq, 2)
        g.check(g.lib.h3_gpu_dit_attention_noise(g.handle, 3, 0.5, 0.5), "noise")
        for block in (0, 5):  # warmup (step 3 < 10) and probe / short
            assert np.array_equal(sdpa(g, q, k, v, seq, 2, step=3, block=block), dense)
    finally:
        g.close()
        d.close()
