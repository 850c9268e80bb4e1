"""The synthetic DiT denoise step (include/h3_dit_synth.h) end to end on the GPU:
finite, deterministic, and identical whether block weights are resident or
streamed from pinned host memory through the two device slots."""
import numpy as np
import pytest

from h3cli_amd.runtime import DitSynth

pytestmark = pytest.mark.gpu

SMALL = dict(blocks=3, hidden=256, heads=2, mlp=512, frames=2, height=4, width=16, audio_rows=100, latent=256,
             mask_density=0.5, seed=11)


def run(steps=2, **kw):
    cfg = dict(SMALL)
    cfg.update(kw)
    print(f"[dit step] {cfg}", flush=True)
    with DitSynth(**cfg) as m:
        before = m.read("latent")
        for s in range(steps):
            m.step(step=s, dt=-0.1)
        return before, m.read("latent"), m.read("hidden")


@pytest.mark.parametrize("mode", [1, 0])
def test_step_finite_and_deterministic(mode):
    b0, l0, h0 = run(attention_mode=mode, streamed_first=3)
    b1, l1, h1 = run(attention_mode=mode, streamed_first=3)
    assert np.all(np.isfinite(l0)) and np.all(np.isfinite(h0))
    assert not np.array_equal(b0, l0)          # the step moved the latent
    assert np.array_equal(l0, l1) and np.array_equal(h0, h1)


def test_streamed_blocks_match_resident():
    _, resident, _ = run(streamed_first=3)
    _, streamed, _ = run(streamed_first=1)
    _, all_streamed, _ = run(streamed_first=0)
    assert np.array_equal(resident, streamed)
    assert np.array_equal(resident, all_streamed)


def test_dense_and_sparse_differ_and_zero_dt_is_identity():
    _, sparse, _ = run(mask_density=0.0, steps=1)
    _, dense, _ = run(mask_density=-1.0, steps=1)
    assert not np.array_equal(sparse, dense)
    b, l, _ = run(steps=1, mask_density=-1.0, seed=3)
    with DitSynth(**dict(SMALL, seed=3)) as m:
        before = m.read("latent")
        m.step(step=0, dt=0.0)
        assert np.array_equal(before, m.read("latent"))
