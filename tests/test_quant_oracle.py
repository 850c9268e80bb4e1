"""Pins of the FP8 projection restatement (oracle/quant.c): the tensorwide
E4M3 packing against torch's float8_e4m3fn cast, its scale closed forms, and
the GEMM against a float64 matrix product of torch-decoded codes; plus the
reference's exact-pattern case (tests/quant_native.c:29-52)."""
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
