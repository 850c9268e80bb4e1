"""CPU pins of the host-side DiT tables that feed the block: the 256-d timestep
features (reference src/denoise/dit_schedule.c:152-162) and the 3D RoPE cos/sin
tables (dit.c:1051-1090 structure, BASELINE config 2 split 44/42/42, theta 1e4).
Both are checked against closed forms computed here in float64, not against a
restatement of the C loops."""
import numpy as np

from h3cli_amd import _lib, synth


def features(times):
    lib = _lib.load()
    t = np.ascontiguousarray(times, np.float32)
    out = np.zeros((t.size, 256), np.float32)
    lib.h3_hip_dit_time_features(t.ctypes.data, t.size, out.ctypes.data)
    return out


def rope(frames, height, width, audio, half):
    lib = _lib.load()
    rows = frames * height * width + audio
    c = np.zeros((rows, half), np.uint16)
    s = np.zeros((rows, half), np.uint16)
    ok = lib.h3_hip_dit_rope_tables(frames, height, width, audio, half, c.ctypes.data, s.ctypes.data)
    return ok, synth.bf16_to_f32(c), synth.bf16_to_f32(s)


def test_time_features_closed_form():
    """cos for the first 128 features, sin for the last 128, frequency
    exp(-ln(1e4) i / 128) = 1e4^(-i/128); t = 0.5 is BASELINE config 5's."""
    t = np.array([0.5, 0.0, 1.0, 0.999, 0.125], np.float32)
    got = features(t)
    i = np.arange(128, dtype=np.float64)
    ang = t.astype(np.float64)[:, None] * 10000.0 ** (-i / 128.0)[None, :]
    assert np.max(np.abs(got[:, :128] - np.cos(ang))) < 2e-6
    assert np.max(np.abs(got[:, 128:] - np.sin(ang))) < 2e-6
    # t = 0: every cosine exactly 1, every sine exactly 0 (order check).
    assert np.all(got[1, :128] == 1.0) and np.all(got[1, 128:] == 0.0)
    # Frequency 0 is 1 for every t: feature 0 = cos t, feature 128 = sin t.
    assert np.allclose(got[:, 0], np.cos(t), atol=1e-7) and np.allclose(got[:, 128], np.sin(t), atol=1e-7)


def test_rope_split_and_frequencies():
    frames, height, width, audio, half = 27, 30, 40, 16, 64
    ok, c, s = rope(frames, height, width, audio, half)
    assert ok
    video = frames * height * width
    r = np.arange(video)
    pos = np.stack([r // (height * width), (r // width) % height, r % width], 1).astype(np.float64)
    # 22 frame pairs (44 channels), 21 row pairs, 21 column pairs.
    axis = np.repeat([0, 1, 2], [22, 21, 21])
    i = np.concatenate([np.arange(22), np.arange(21), np.arange(21)]).astype(np.float64)
    dim = np.array([44.0, 42.0, 42.0])[axis]
    inv = 10000.0 ** (-2.0 * i / dim)
    ang = pos[:, axis] * inv[None, :]
    ref_c = synth.bf16_to_f32(synth.f32_to_bf16(np.cos(ang).astype(np.float32)))
    ref_s = synth.bf16_to_f32(synth.f32_to_bf16(np.sin(ang).astype(np.float32)))
    # FP32 angle and libm differ from float64 only at rare BF16 rounding ties:
    # at most one BF16 step anywhere, and equal almost everywhere.
    step = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref_c), 1e-30))) - 7)
    assert np.all(np.abs(c[:video] - ref_c) <= step + 1e-30)
    assert np.mean(c[:video] == ref_c) > 0.999 and np.mean(s[:video] == ref_s) > 0.999
    # Axis split: a token at frame 5, row 0, column 0 rotates only the first 22 pairs.
    t = 5 * height * width
    assert np.all(c[t, 22:] == 1.0) and np.all(s[t, 22:] == 0.0) and np.all(s[t, 1:22] != 0.0)
    # Row 7 only: pairs 22..42; column 9 only: pairs 43..63.
    t = 7 * width
    assert np.all(c[t, :22] == 1.0) and np.all(c[t, 43:] == 1.0) and np.all(s[t, 22:43] != 0.0)
    t = 9
    assert np.all(c[t, :43] == 1.0) and np.all(s[t, 43:] != 0.0)
    # Pair 0 of each axis has inv_freq 1: angle = position exactly.
    assert np.array_equal(s[7 * width, 22], synth.bf16_to_f32(synth.f32_to_bf16(np.float32(np.sin(7.0)))))
    # Audio rows after the video rows: angle 0.
    assert np.all(c[video:] == 1.0) and np.all(s[video:] == 0.0)


def test_rope_even_split_and_invalid():
    """half = 48 (the real H3 block, 16 frequencies per axis): inv_freq
    1e4^(-i/16) on every axis; invalid halves are refused."""
    ok, c, s = rope(2, 3, 5, 0, 48)
    assert ok
    t = 1 * 15 + 2 * 5 + 3          # frame 1, row 2, column 3
    pos = np.repeat([1.0, 2.0, 3.0], 16)
    inv = np.tile(10000.0 ** (-np.arange(16) / 16.0), 3)
    ref = synth.bf16_to_f32(synth.f32_to_bf16(np.cos(pos * inv).astype(np.float32)))
    assert np.max(np.abs(c[t] - ref)) <= 2.0 ** -8
    for bad in (0, 50, 66):
        assert not rope(2, 3, 5, 0, bad)[0]
