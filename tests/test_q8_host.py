"""W8A16 packing on the host: the library's h3_q8_pack_rows / h3_q8_layout against
the reference's own known-answer cases (tests/metal_q8.c:19-35) and against the
oracle's independent restatement; the oracle's W8A16 GEMM against an exact
power-of-two pattern (tests/quant_native.c:31-50 recipe)."""
import ctypes as C

import numpy as np

from h3cli_amd import _lib, synth
from oracle import oracle


def lib():
    l = C.CDLL(str(_lib.LIB_PATH))
    l.h3_q8_pack_rows.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32]
    l.h3_q8_layout.argtypes = [C.c_uint32, C.c_uint32, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
    return l


def pack(l, w, rows, cols):
    w = np.ascontiguousarray(w, np.uint16)
    codes = np.zeros(rows * cols, np.int8)
    scales = np.zeros(rows * ((cols + 63) // 64), np.float32)
    ok = l.h3_q8_pack_rows(w.ctypes.data, codes.ctypes.data, scales.ctypes.data, rows, cols)
    return ok, codes, scales


def test_reference_known_answers():
    l = lib()
    src = np.zeros(65, np.uint16)
    vals = [127, -127, .5, 1.5, 2.5, -.5, -1.5, -2.5]
    src[:8] = synth.f32_to_bf16(np.float32(vals))
    ok, q, s = pack(l, src, 1, 65)
    assert ok
    assert list(q[:8]) == [127, -127, 0, 2, 2, 0, -2, -2]
    assert s[0] == 1 and s[1] == 1 and q[64] == 0
    off, total = C.c_size_t(), C.c_size_t()
    assert l.h3_q8_layout(1, 65, C.byref(off), C.byref(total)) and off.value == 68 and total.value == 76
    assert not l.h3_q8_layout(0, 65, C.byref(off), C.byref(total))
    assert not l.h3_q8_layout(0xFFFFFFFF, 0xFFFFFFFF, C.byref(off), C.byref(total))
    assert not l.h3_q8_layout(1, 0xFFFFFFFF - 31, C.byref(off), C.byref(total))
    for bad in (0x7FC0, 0x7F80):
        src[64] = bad
        assert not pack(l, src, 1, 65)[0]
    src[64] = 1  # smallest subnormal: scale stays finite
    ok, q, s = pack(l, src, 1, 65)
    assert ok and np.isfinite(s[1])
    # The oracle's restatement gives the same answers.
    codes, scales = oracle.q8_pack(src, 1, 65, 64)
    assert np.array_equal(codes, q) and np.array_equal(scales, s)


def test_library_pack_matches_oracle_random():
    l = lib()
    rows, cols = 37, 300
    w = synth.normal_bf16(5, rows * cols, scale=0.05)
    ok, q, s = pack(l, w, rows, cols)
    codes, scales = oracle.q8_pack(w, rows, cols, 64)
    assert ok and np.array_equal(q, codes) and np.array_equal(s.view(np.uint32), scales.view(np.uint32))
    # Every code is within half a step of w / scale and the extreme codes are +-127.
    wf = synth.bf16_to_f32(w).reshape(rows, cols)
    sc = np.repeat(s.reshape(rows, -1), 64, axis=1)[:, :cols]
    assert np.all(np.abs(q.reshape(rows, cols) - wf / sc) <= 0.5 + 1e-5)


def test_oracle_linear_exact_pattern():
    """Powers of two: every product and partial sum is exact, so the oracle's
    output must equal bf16 of the exact integer-arithmetic sum."""
    n, k, rows = 64, 256, 7
    j = np.arange(n)[:, None]
    c = np.arange(k)[None, :]
    w = np.ldexp(1.0, (j % 3) - 1 + (c // 16) % 3).astype(np.float32)
    r = np.arange(rows)[:, None]
    x = (np.where(r % 2, -1.0, 1.0) * np.ldexp(1.0, (r % 3) - 1 + (c // 16) % 2)).astype(np.float32)
    y, y64 = oracle.linear_bf16(synth.f32_to_bf16(x), synth.f32_to_bf16(w), rows, k, n)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.array_equal(y, synth.f32_to_bf16(exact.astype(np.float32)).reshape(-1))
    assert np.array_equal(y64.reshape(rows, n), exact)
