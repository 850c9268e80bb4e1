"""Pins of the FP8 projection restatement (oracle/quant.c): the tensorwide
E4M3 packing against torch's float8_e4m3fn cast, its scale closed forms, and
the GEMM against a float64 matrix product of torch-decoded codes; plus the
reference's exact-pattern case (tests/quant_native.c:29-52)."""
import ctypes as C

import numpy as np
import pytest

from h3cli_amd import synth
from oracle import oracle

torch = pytest.importorskip("torch")


def _torch_codes(x_bf16, scale):
    x = torch.from_numpy(synth.bf16_to_f32(x_bf16).astype(np.float32))
    return (x / torch.tensor(scale, dtype=torch.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def _decode(codes):
    return torch.from_numpy(np.ascontiguousarray(codes, np.uint8)).view(torch.float8_e4m3fn).float().numpy()


def test_pack_matches_torch_cast():
    rng = np.random.default_rng(11)
    for scale_exp in (-30, -8, 0, 6, 40):
        x = synth.f32_to_bf16((rng.standard_normal(4096) * 2.0 ** scale_exp).astype(np.float32))
        codes, scale, bad = oracle.fp8_pack(x)
        amax = np.abs(synth.bf16_to_f32(x)).max()
        assert not bad and scale == np.float32(max(np.float32(amax) / np.float32(448), np.float32(1e-20)))
        assert np.array_equal(codes, _torch_codes(x, scale)), scale_exp


def test_pack_closed_forms():
    x = synth.f32_to_bf16(np.array([448, -448, 1, -0.5, 3, 0, 2.0 ** -9, 2.0 ** -10] * 2, np.float32))
    codes, scale, _ = oracle.fp8_pack(x)
    assert scale == 1.0                                  # amax 448
    assert list(codes[:8]) == [0x7e, 0xfe, 0x38, 0xb0, 0x44, 0x00, 0x01, 0x00]   # 2^-10 ties to 0 (even)
    codes, scale, _ = oracle.fp8_pack(np.zeros(16, np.uint16))
    assert scale == np.float32(1e-20) and not codes.any()
    codes, scale, _ = oracle.fp8_pack(synth.f32_to_bf16(np.array([896.0] + [0.0] * 7, np.float32)))
    assert scale == 2.0 and codes[0] == 0x7e
    codes, _, _ = oracle.fp8_pack(np.zeros(8, np.uint16), 8, 24)       # padding rows pack as 0
    assert codes.size == 24 and not codes.any()
    bad = synth.f32_to_bf16(np.array([1.0, np.nan, 2.0, np.inf] * 2, np.float32))
    assert oracle.fp8_pack(bad)[2]


def test_gemm_matches_float64_product():
    rng = np.random.default_rng(12)
    m, n, k = 37, 48, 256
    x = synth.f32_to_bf16(rng.standard_normal(m * k).astype(np.float32))
    w = synth.f32_to_bf16((rng.standard_normal(n * k) * 0.05).astype(np.float32))
    x8, sx, _ = oracle.fp8_pack(x)
    w8, sw, _ = oracle.fp8_pack(w)
    got = oracle.fp8_gemm(x8, sx, w8, sw, m, n, k)
    exact = _decode(x8).reshape(m, k).astype(np.float64) @ _decode(w8).reshape(n, k).astype(np.float64).T
    want = synth.f32_to_bf16((exact.astype(np.float32) * np.float32(np.float32(sx) * np.float32(sw))).astype(np.float32))
    assert np.array_equal(got, want)
    # Transposition check: a single nonzero weight row selects one output column.
    w1 = np.zeros(n * k, np.uint8)
    w1[5 * k:6 * k] = 0x38                               # row 5 of W is all 1.0
    y = synth.bf16_to_f32(oracle.fp8_gemm(x8, 1.0, w1, 1.0, m, n, k))
    assert not np.delete(y, 5, axis=1).any()
    row_sums = _decode(x8).reshape(m, k).astype(np.float64).sum(axis=1).astype(np.float32)
    assert np.array_equal(y[:, 5], synth.bf16_to_f32(synth.f32_to_bf16(row_sums)))


def test_reference_exact_pattern():
    """tests/quant_native.c:29-52: power-of-two weights and inputs with tiled
    exponents; the FP8 product must equal bf16 of the exact sum."""
    n, k, rows = 256, 256, 129
    j, c = np.meshgrid(np.arange(n), np.arange(k), indexing="ij")
    w = synth.f32_to_bf16(np.ldexp(1.0, (j % 3) - 1 + (c // 16) % 3).astype(np.float32)).reshape(-1)
    r, c = np.meshgrid(np.arange(rows), np.arange(k), indexing="ij")
    x = synth.f32_to_bf16(np.ldexp(np.where(r % 2, -1.0, 1.0), (r % 3) - 1 + (c // 16) % 2).astype(np.float32)).reshape(-1)
    x8, sx, _ = oracle.fp8_pack(x)
    w8, sw, _ = oracle.fp8_pack(w)
    got = oracle.fp8_gemm(x8, sx, w8, sw, rows, n, k)
    exact = synth.bf16_to_f32(x).reshape(rows, k).astype(np.float64) @ synth.bf16_to_f32(w).reshape(n, k).astype(np.float64).T
    assert np.array_equal(got, synth.f32_to_bf16(exact.astype(np.float32)))


def test_e2m1_encoder_closed_forms():
    """E2M1 values {0, .5, 1, 1.5, 2, 3, 4, 6}: exact values, every midpoint
    tied to the even code, saturation at 6, the sign bit."""
    values = [0, 0.5, 1, 1.5, 2, 3, 4, 6]
    assert list(oracle.e2m1_decode(np.arange(16))) == values + [-v for v in values]
    enc = lambda x: int(oracle.load().oracle_f32_to_e2m1(C.c_float(x)))
    oracle.load().oracle_f32_to_e2m1.argtypes = [C.c_float]
    oracle.load().oracle_f32_to_e2m1.restype = C.c_uint8
    for c, v in enumerate(values):
        assert enc(v) == c
    ties = {0.25: 0, 0.75: 2, 1.25: 2, 1.75: 4, 2.5: 4, 3.5: 6, 5.0: 6}
    for x, c in ties.items():
        assert enc(x) == c, x
    assert enc(0.26) == 1 and enc(5.01) == 7 and enc(7.0) == 7 and enc(1e9) == 7
    assert enc(-0.75) == 8 | 2 and enc(-6.0) == 15


def test_nvfp4_scale_layout_is_a_bijection():
    """Every (row, block) of padded rows x blocks padded to 4 maps to its own
    byte of the plane, 512-byte tiles hold 128 rows x 4 blocks."""
    for rows, k in ((128, 64), (256, 512), (384, 1024)):
        blocks = (k // 16 + 3) // 4 * 4
        seen = {oracle.nvfp4_scale_index(r, b, k) for r in range(rows) for b in range(blocks)}
        assert len(seen) == rows * blocks and max(seen) == oracle.nvfp4_scale_bytes(rows, k) - 1
        for r in (0, 31, 32, 127):
            assert oracle.nvfp4_scale_index(r, 3, k) // 512 == 0


def test_nvfp4_exact_pattern_round_trips():
    """tests/quant_native.c's pattern: every value is 2^e with one e per 16
    columns, so g = amax / 2688, each block scale is 448 * 2^(e - emax), every
    code is 6 and the dequantized value code * sf * g is 2^e exactly."""
    n, k = 256, 256
    j, c = np.meshgrid(np.arange(n), np.arange(k), indexing="ij")
    e = (j % 3) - 1 + (c // 16) % 3
    w = synth.f32_to_bf16(np.ldexp(1.0, e).astype(np.float32)).reshape(-1)
    codes, scales, glob, _ = oracle.nvfp4_pack(w, n, k)
    assert glob[0] == np.float32(8.0 / 2688) and glob[1] == 1.0
    assert np.all(codes == 0x77)
    sf = oracle.e4m3_decode(scales)
    for r in (0, 1, 2, 200):
        for b in range(k // 16):
            assert sf[oracle.nvfp4_scale_index(r, b, k)] == 448 * 2.0 ** (e[r, b * 16] - 3)
    x = synth.f32_to_bf16(np.ldexp(np.where(j[:129] % 2, -1.0, 1.0), (j[:129] % 3) - 1 + (c[:129] // 16) % 2)
                          .astype(np.float32)).reshape(-1)
    x4, xs, xg, _ = oracle.nvfp4_pack(x, 129, k, weight_global=glob[0])
    assert xg[1] == np.float32(xg[0] * glob[0])
    y = oracle.nvfp4_gemm(x4, xs, codes, scales, xg[1], 129, n, k)
    exact = synth.bf16_to_f32(x).reshape(129, k).astype(np.float64) @ synth.bf16_to_f32(w).reshape(n, k).astype(np.float64).T
    assert np.array_equal(y, synth.f32_to_bf16(exact.astype(np.float32)))


def test_nvfp4_pack_error_bounds():
    """Random rows: each block scale is the E4M3 rounding of blockmax / (6 g)
    (floored at 2^-9); each dequantized value is within half an E2M1 step (or
    saturated at 6) of x / (sf g)."""
    rng = np.random.default_rng(13)
    rows, k = 128, 256
    x = synth.f32_to_bf16((rng.standard_normal(rows * k) * np.repeat(rng.uniform(0.01, 3, rows * k // 16), 16))
                          .astype(np.float32))
    codes, scales, glob, _ = oracle.nvfp4_pack(x, rows, k)
    xf = synth.bf16_to_f32(x).reshape(rows, k).astype(np.float64)
    g = float(glob[0])
    assert glob[0] == np.float32(max(np.float32(np.abs(xf).max()) / np.float32(2688), np.float32(1e-20)))
    sf = oracle.e4m3_decode(scales).astype(np.float64)
    vals = oracle.e2m1_decode(np.stack([codes & 15, codes >> 4], 1).reshape(-1)).astype(np.float64).reshape(rows, k)
    grid = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6, -0.5, -1, -1.5, -2, -3, -4, -6])
    for r in range(0, rows, 7):
        for b in range(k // 16):
            s = sf[oracle.nvfp4_scale_index(r, b, k)]
            m = np.abs(xf[r, b * 16:(b + 1) * 16]).max()
            t = max(m / (6 * g), 2.0 ** -9)
            assert abs(s - t) <= t * 2.0 ** -4 + 2.0 ** -10          # E4M3 rounding (3 mantissa bits)
            q = xf[r, b * 16:(b + 1) * 16] / (s * g)
            v = vals[r, b * 16:(b + 1) * 16]
            qc = np.clip(q, -6, 6)
            nearest = np.abs(grid[None, :] - qc[:, None]).min(axis=1)
            assert np.all(np.abs(v - qc) <= nearest + 1e-6), (r, b)         # a nearest E2M1 value
