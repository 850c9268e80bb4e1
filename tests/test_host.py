"""CPU tests of the C-ABI library: it loads, exports every declared symbol, and
its host-side logic (no GPU calls) matches the oracle."""
import ctypes as C
import re
from pathlib import Path

import numpy as np

from h3cli_amd import _lib
from oracle import oracle

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"\b(h3_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in sorted(declared_symbols()) if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_loads():
    lib = _lib.load()
    assert lib.h3_hip_version().startswith(b"h3hip gfx950")


def test_synthetic_mask_matches_oracle():
    lib = _lib.load()
    for seq, video, density, seed in [(33424, 32400, 0.25, 0), (1000, 900, 0.25, 7), (513, 513, 0.5, 1)]:
        blocks = (seq + 127) // 128
        m = np.zeros(blocks * blocks, np.uint8)
        kept = lib.h3_hip_synthetic_block_mask(m.ctypes.data, seq, video, 128, density, seed)
        ref = oracle.block_mask(seq, video, 128, density, seed)
        assert np.array_equal(m.reshape(blocks, blocks), ref)
        assert kept == int(ref.sum())
        assert np.all(np.diag(ref) == 1)


def test_synthetic_mask_density_and_audio_blocks():
    seq, video = 33424, 32400
    m = oracle.block_mask(seq, video, 128, 0.25, 0)
    b = m.shape[0]
    first_audio = video // 128
    assert np.all(m[first_audio:, first_audio:] == 1)
    off = m[:first_audio, :first_audio][~np.eye(first_audio, dtype=bool)]
    assert abs(off.mean() - 0.25) < 0.01
    assert b == 262


def test_v_position_is_a_permutation():
    lib = _lib.load()
    pos = [lib.h3_hip_sage_v_position(j) for j in range(64)]
    assert sorted(pos) == list(range(64))
    assert pos == [oracle.sage_v_position(j) for j in range(64)]


def test_exports_reference_link_contract():
    """Every symbol the reference's tests/test_gpu_contract.c links (non-Apple
    branch) is exported, so h3cli links against this library unchanged."""
    lib = C.CDLL(str(_lib.LIB_PATH))
    names = (ROOT / "tests" / "golden" / "gpu_contract_symbols.txt").read_text().split()
    assert len(names) == 166
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_context_free_surface_calls():
    """Calls that need no device: NULL contexts are rejected, host parses work."""
    lib = C.CDLL(str(_lib.LIB_PATH))
    lib.h3_qwen_gqa_scale_name.restype = C.c_char_p
    mode = C.c_int(-1)
    err = C.create_string_buffer(128)
    for text, want in ((None, 0), (b"", 0), (b"reference", 0), (b"scaled-q", 1), (b"legacy", 2)):
        assert lib.h3_qwen_gqa_scale_parse(text, C.byref(mode), err, 128) == 1 and mode.value == want
        assert lib.h3_qwen_gqa_scale_name(want) == (text or b"reference")
    assert lib.h3_qwen_gqa_scale_parse(b"bogus", C.byref(mode), err, 128) == 0
    assert err.value == b"invalid H3_QWEN_GQA_SCALE_MODE: bogus"
    assert lib.h3_gpu_prefers_device_sampler(None, 0) == 0
    assert lib.h3_gpu_should_retry_streaming(None) == 0
    assert lib.h3_gpu_is_m5(None) == 0 and lib.h3_gpu_has_int8_mlp(None) == 0
    # Out-of-path ops fail without a context rather than crash.
    assert lib.h3_gpu_conv3d_f32(None, None, None, None, None, *([1] * 13)) == 0
    assert lib.h3_gpu_video_graph_begin(None) == 0
    lib.h3_gpu_sglang_vae_weight.restype = C.c_void_p
    assert lib.h3_gpu_sglang_vae_weight(None, None) is None


def test_device_configure_validation(monkeypatch):
    lib = C.CDLL(str(_lib.LIB_PATH))
    err = C.create_string_buffer(128)
    monkeypatch.delenv("H3_CUDA_DEVICE", raising=False)
    monkeypatch.delenv("H3_CUDA_WEIGHT_MODE", raising=False)
    assert lib.h3_device_configure(b"x1", None, err, 128) == 0 and b"invalid HIP device index" in err.value
    assert lib.h3_device_configure(None, b"bogus", err, 128) == 0
    libc = C.CDLL(None)
    libc.getenv.restype = C.c_char_p
    try:
        assert lib.h3_device_configure(b"0", b"stream", err, 128) == 1
        assert libc.getenv(b"H3_CUDA_DEVICE") == b"0" and libc.getenv(b"H3_CUDA_WEIGHT_MODE") == b"stream"
    finally:  # the C-level environment is not restored by monkeypatch
        libc.unsetenv(b"H3_CUDA_DEVICE")
        libc.unsetenv(b"H3_CUDA_WEIGHT_MODE")
