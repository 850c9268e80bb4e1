"""Host side of the FP8 projection path: the packed descriptor sizes, checked
against closed forms and the reference's own residency.c compiled into
oracle/_ref/libh3ref.so, and SHA-256 (the artifact key) against hashlib."""
import ctypes as C
import hashlib
import os

import numpy as np
import pytest

from h3cli_amd import _lib

REF = os.path.join(os.path.dirname(__file__), "..", "oracle", "_ref", "libh3ref.so")
need_ref = pytest.mark.skipif(not os.path.exists(REF), reason="oracle/_ref/libh3ref.so not built")


def _bind(lib):
    lib.h3_weight_packed_size.restype = C.c_int
    lib.h3_weight_packed_size.argtypes = [C.c_uint32, C.c_uint32, C.c_int] + [C.POINTER(C.c_uint64)] * 3
    return lib


@pytest.fixture(scope="module")
def ours():
    return _bind(C.CDLL(str(_lib.LIB_PATH), mode=os.RTLD_LOCAL))


@pytest.fixture(scope="module")
def ref():
    if not os.path.exists(REF):
        pytest.skip("oracle/_ref/libh3ref.so not built")
    return _bind(C.CDLL(os.path.abspath(REF), mode=os.RTLD_LOCAL))


def _packed(lib, rows, cols, mode):
    s, g, b = C.c_uint64(), C.c_uint64(), C.c_uint64()
    ok = lib.h3_weight_packed_size(rows, cols, mode, C.byref(s), C.byref(g), C.byref(b))
    return ok, s.value, g.value, b.value


def test_packed_size_closed_form(ours):
    # FP8: codes, then the 4-byte scale at the next 256 boundary, then 16 bytes.
    assert _packed(ours, 21504, 5376, 1) == (1, 21504 * 5376, 21504 * 5376 + 256, 21504 * 5376 + 256 + 16)
    assert _packed(ours, 1, 1, 1) == (1, 256, 512, 528)
    # NVFP4 128 x 16: 1024 payload bytes, 128 rows x 4 padded block columns of scales.
    assert _packed(ours, 128, 16, 2) == (1, 1024, 1536, 1552)
    assert _packed(ours, 0, 128, 1)[0] == 0 and _packed(ours, 128, 128, 3)[0] == 0 and _packed(ours, 128, 8, 2)[0] == 0


@need_ref
def test_packed_size_matches_reference(ours, ref):
    rng = np.random.default_rng(3)
    cases = [(21504, 5376), (5376, 7168), (28672, 5376), (5376, 14336), (1, 1), (127, 16), (129, 48), (0, 16),
             (2**32 - 1, 2**32 - 1), (2**31, 3), (65536, 65536)]
    cases += [tuple(int(v) for v in rng.integers(1, 70000, 2)) for _ in range(200)]
    for rows, cols in cases:
        for mode in (0, 1, 2, 3):
            assert _packed(ours, rows, cols, mode) == _packed(ref, rows, cols, mode), (rows, cols, mode)


def test_sha256_matches_hashlib():
    lib = C.CDLL(str(_lib.LIB_PATH), mode=os.RTLD_LOCAL)
    lib.h3_hip_sha256.argtypes = [C.c_void_p, C.c_size_t, C.c_void_p]
    rng = np.random.default_rng(7)
    # Every length across the one- and two-block padding boundaries, then large.
    sizes = list(range(0, 200)) + [447, 448, 511, 512, 513, 4095, 65536, 1 << 20, (1 << 20) + 37]
    for n in sizes:
        data = rng.integers(0, 256, n, dtype=np.uint8)
        out = (C.c_ubyte * 32)()
        assert lib.h3_hip_sha256(data.ctypes.data if n else None, n, out)
        assert bytes(out) == hashlib.sha256(data.tobytes()).digest(), n
    # FIPS 180-2 appendix example: "abc".
    out = (C.c_ubyte * 32)()
    lib.h3_hip_sha256(C.c_char_p(b"abc"), 3, out)
    assert bytes(out).hex() == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
