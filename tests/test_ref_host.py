"""Host-side restatements in libh3hip.so checked bit for bit against the
reference's own C sources, compiled where they lie by oracle/ref/Makefile into
oracle/_ref/libh3ref.so (src/weights/q8.c, src/denoise/subblock.c,
src/denoise/attention.c). Skipped when that library was not built (the GPU box
has no /root/reference; the prebuilt file travels with the tree when present)."""
import ctypes as C
import os

import numpy as np
import pytest

from h3cli_amd import _lib, synth

REF = os.path.join(os.path.dirname(__file__), "..", "oracle", "_ref", "libh3ref.so")

pytestmark = pytest.mark.skipif(not os.path.exists(REF), reason="oracle/_ref/libh3ref.so not built")


def _bind(lib):
    lib.h3_q8_layout.restype = C.c_int
    lib.h3_q8_layout.argtypes = [C.c_uint32, C.c_uint32, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
    lib.h3_q8_pack_rows.restype = C.c_int
    lib.h3_q8_pack_rows.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32]
    lib.h3_subblock_budget.restype = C.c_uint
    lib.h3_subblock_budget.argtypes = [C.c_uint, C.c_float]
    lib.h3_subblock_warmup.restype = C.c_int
    lib.h3_subblock_warmup.argtypes = [C.c_int]
    lib.h3_subblock_dense_reason.restype = C.c_char_p
    lib.h3_subblock_dense_reason.argtypes = [C.c_uint, C.c_uint, C.c_int, C.c_float, C.c_int]
    lib.h3_attention_name.restype = C.c_char_p
    lib.h3_attention_name.argtypes = [C.c_int]
    lib.h3_attention_parse.restype = C.c_int
    lib.h3_attention_parse.argtypes = [C.c_char_p, C.POINTER(C.c_int)]
    lib.h3_attention_options.restype = C.c_int
    lib.h3_attention_options.argtypes = [C.c_int, C.c_char_p, C.c_size_t]
    return lib


@pytest.fixture(scope="module")
def libs():
    # RTLD_LOCAL keeps the two libraries' same-named symbols apart.
    ref = _bind(C.CDLL(os.path.abspath(REF), mode=os.RTLD_LOCAL))
    ours = _bind(C.CDLL(str(_lib.LIB_PATH), mode=os.RTLD_LOCAL))
    return ours, ref


def _layout(lib, rows, cols):
    so, nb = C.c_size_t(), C.c_size_t()
    ok = lib.h3_q8_layout(rows, cols, C.byref(so), C.byref(nb))
    return ok, so.value, nb.value


def test_q8_layout_matches_reference(libs):
    ours, ref = libs
    cases = [(0, 0), (1, 1), (1, 63), (3, 64), (5, 65), (7, 129), (5120, 5120), (13824, 5120),
             (1, 2**31), (2**31, 2**31), (2**32 - 1, 2**32 - 1), (65536, 65536 * 4 + 3)]
    for rows, cols in cases:
        assert _layout(ours, rows, cols) == _layout(ref, rows, cols), (rows, cols)


def _pack(lib, src, rows, cols):
    codes = np.zeros(rows * cols, np.int8)
    groups = -(-cols // 64)
    scales = np.zeros(rows * groups, np.float32)
    ok = lib.h3_q8_pack_rows(src.ctypes.data, codes.ctypes.data, scales.ctypes.data, rows, cols)
    return ok, codes, scales


@pytest.mark.parametrize("rows,cols,seed", [(1, 1, 0), (3, 63, 1), (4, 64, 2), (5, 65, 3), (17, 300, 4),
                                            (64, 5120, 5)])
def test_q8_pack_matches_reference(libs, rows, cols, seed):
    ours, ref = libs
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(rows * cols) * rng.choice([1e-3, 1.0, 30.0], rows * cols)).astype(np.float32)
    x[rng.integers(0, x.size, max(1, x.size // 50))] = 0.0
    src = synth.f32_to_bf16(x)
    okr, cr, sr = _pack(ref, src, rows, cols)
    oko, co, so = _pack(ours, src, rows, cols)
    assert okr == oko == 1
    assert np.array_equal(cr, co)
    assert np.array_equal(sr.view(np.uint32), so.view(np.uint32))


def test_q8_pack_edge_values_match_reference(libs):
    ours, ref = libs
    bits = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x7F7F, 0xFF7F, 0x3F80, 0xBF80, 0x0080, 0x4000] * 13,
                    np.uint16)[:128]
    for rows, cols in ((1, 128), (2, 64), (128, 1)):
        okr, cr, sr = _pack(ref, bits, rows, cols)
        oko, co, so = _pack(ours, bits, rows, cols)
        assert okr == oko
        assert np.array_equal(cr, co) and np.array_equal(sr.view(np.uint32), so.view(np.uint32))
    for bad in (0x7F80, 0xFF80, 0x7FC0):  # +inf, -inf, NaN are rejected by both
        b = bits.copy()
        b[37] = bad
        assert _pack(ref, b, 2, 64)[0] == _pack(ours, b, 2, 64)[0] == 0


def test_subblock_budget_matches_reference(libs):
    ours, ref = libs
    sparsities = [0.0, 0.1, 0.5, 0.75, 0.875, 0.9, 0.99, 0.999999, 1.0, -0.1, float("nan"), float("inf")]
    for blocks in list(range(0, 80)) + [506, 507, 1000, 2**20, 2**32 - 1]:
        for s in sparsities:
            assert ours.h3_subblock_budget(blocks, s) == ref.h3_subblock_budget(blocks, s), (blocks, s)


def test_subblock_dense_reason_matches_reference(libs):
    ours, ref = libs
    for warmup in (-1, 0, 1, 10, 25):
        assert ours.h3_subblock_warmup(warmup) == ref.h3_subblock_warmup(warmup)
        for step in (-5, 0, 9, 10, 11, 30):
            for block in (0, 1, 39):
                for seq in (0, 64, 4095, 4096, 4097, 32400, 100000):
                    for s in (0.0, 0.5, 0.75, 0.99):
                        args = (seq, block, step, s, warmup)
                        assert ours.h3_subblock_dense_reason(*args) == ref.h3_subblock_dense_reason(*args), args


def test_attention_names_match_reference(libs):
    ours, ref = libs
    for mode in range(-2, 7):
        assert ours.h3_attention_name(mode) == ref.h3_attention_name(mode)
        eo, er = C.create_string_buffer(256), C.create_string_buffer(256)
        assert ours.h3_attention_options(mode, eo, 256) == ref.h3_attention_options(mode, er, 256)
        assert eo.value == er.value
    for text in (b"default", b"sage2++", b"sage3", b"sol", b"subblock", b"Sage2++", b"", b"dense"):
        mo, mr = C.c_int(-7), C.c_int(-7)
        assert ours.h3_attention_parse(text, C.byref(mo)) == ref.h3_attention_parse(text, C.byref(mr))
        assert mo.value == mr.value


class WeightOptions(C.Structure):
    _fields_ = [("mode", C.c_int), ("max_resident", C.c_int), ("capacity_limit", C.c_uint64),
                ("allocation_limit", C.c_uint64)]


class WeightPlan(C.Structure):
    _fields_ = [("options", WeightOptions), ("active_mask", C.c_uint64), ("resident_mask", C.c_uint64),
                ("free_bytes", C.c_uint64), ("live_bytes", C.c_uint64), ("reserve_bytes", C.c_uint64),
                ("future_bytes", C.c_uint64), ("block_bytes", C.c_uint64), ("resident_bytes", C.c_uint64),
                ("slot_bytes", C.c_uint64), ("active_count", C.c_uint), ("resident_count", C.c_uint),
                ("effective_mode", C.c_int)]


def _plan(lib, opts, *args):
    fn = lib.h3_weight_plan_build
    fn.restype = C.c_int
    fn.argtypes = [C.POINTER(WeightPlan), WeightOptions] + [C.c_uint64] * 6 + [C.c_char_p, C.c_size_t]
    p = WeightPlan()
    err = C.create_string_buffer(256)
    ok = fn(C.byref(p), opts, *args, err, 256)
    return ok, bytes(memoryview(p)), err.value


def test_weight_plan_matches_reference(libs):
    ours, ref = libs
    GiB = 1 << 30
    block = 246_400_000
    masks = [0, 1, (1 << 40) - 1, (1 << 50) - 1, 1 << 50, 0b1011 << 20]
    for mode in (0, 1, 2, 3):
        for max_res in (-2, -1, 0, 3, 50, 51):
            for cap in (0, 30 * GiB):
                opts = WeightOptions(mode, max_res, cap, 0)
                for mask in masks:
                    for avail in (0, 2 * GiB, 20 * GiB, 280 * GiB):
                        for blk in (0, block):
                            args = (mask, blk, avail, 5 * GiB, 8 * GiB, 28 * GiB)
                            assert _plan(ours, opts, *args) == _plan(ref, opts, *args), (mode, max_res, cap, mask, avail)


def test_weight_options_and_names_match_reference(libs, monkeypatch):
    ours, ref = libs
    for lib in (ours, ref):
        lib.h3_weight_mode_name.restype = C.c_char_p
        lib.h3_weight_options_read.argtypes = [C.POINTER(WeightOptions), C.c_int, C.c_char_p, C.c_size_t]
    for m in range(-1, 4):
        assert ours.h3_weight_mode_name(m) == ref.h3_weight_mode_name(m)
    for n in (0, 1, 2, 7, 100):
        assert ours.h3_weight_retry_cap(n) == ref.h3_weight_retry_cap(n)
    envs = [{}, {"H3_CUDA_WEIGHT_MODE": "stream"}, {"H3_CUDA_WEIGHT_MODE": "resident"},
            {"H3_CUDA_WEIGHT_MODE": "bogus"}, {"H3_TEST_CUDA_RESIDENT_BLOCKS": "7"},
            {"H3_TEST_CUDA_RESIDENT_BLOCKS": "51"}, {"H3_TEST_CUDA_CAPACITY_BYTES": "12x"},
            {"H3_TEST_CUDA_CAPACITY_BYTES": "123456", "H3_CUDA_TEST_MEMORY_BUDGET": "99"}]
    for env in envs:
        for k in ("H3_CUDA_WEIGHT_MODE", "H3_TEST_CUDA_RESIDENT_BLOCKS", "H3_TEST_CUDA_CAPACITY_BYTES",
                  "H3_CUDA_TEST_MEMORY_BUDGET"):
            monkeypatch.delenv(k, raising=False)
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        for force in (0, 1):
            out = []
            for lib in (ours, ref):
                o, e = WeightOptions(9, 9, 9, 9), C.create_string_buffer(256)
                ok = lib.h3_weight_options_read(C.byref(o), force, e, 256)
                out.append((ok, bytes(memoryview(o)) if ok else None, e.value))
            assert out[0] == out[1], (env, force)


class SolOptions(C.Structure):
    """h3_cuda_sol_options (cuda_sol_policy.h:12-15)."""
    _fields_ = [("q_block", C.c_int), ("kv_block", C.c_int), ("dense_layers", C.c_int), ("dense_steps", C.c_int),
                ("local_radius", C.c_int), ("tau", C.c_float), ("min_exact", C.c_float), ("dense_sigma", C.c_float)]


def _bind_sol(lib):
    lib.h3_cuda_sol_options_valid.restype = C.c_int
    lib.h3_cuda_sol_options_valid.argtypes = [SolOptions, C.c_char_p, C.c_size_t]
    lib.h3_cuda_sol_options_match.restype = C.c_int
    lib.h3_cuda_sol_options_match.argtypes = [SolOptions, SolOptions, C.c_uint]
    lib.h3_cuda_sol_dense_reason.restype = C.c_char_p
    lib.h3_cuda_sol_dense_reason.argtypes = [SolOptions, C.c_uint, C.c_int, C.c_float, C.c_float]
    lib.h3_cuda_sol_current.restype = SolOptions
    lib.h3_cuda_sol_current.argtypes = []
    lib.h3_cuda_sol_exchange.restype = SolOptions
    lib.h3_cuda_sol_exchange.argtypes = [SolOptions]
    return lib


def _opts(**kw):
    o = SolOptions(32, 64, 1, 1, 1, 1.0, 0.0, -1.0)
    for k, v in kw.items():
        setattr(o, k, v)
    return o


def test_sol_policy_matches_reference(libs):
    """SOL options validity, field matching, dense reasons and the thread's
    current options, against src/cuda/cuda_sol_policy.c, plus the reference's
    own assertions (tests/test_cuda_sol_policy.c:10-26)."""
    ours, ref = (_bind_sol(lib) for lib in libs)
    nan, inf = float("nan"), float("inf")
    grid = [dict()] + [{k: v} for k, vals in dict(
        q_block=[16, 31, 32, 33, 64, 128], kv_block=[32, 63, 64, 128], dense_layers=[-1, 0, 50, 51],
        dense_steps=[-1, 0, 1000, 1001], local_radius=[-1, 0, 10000, 10001], tau=[-0.1, 0, 16, 16.5, nan, inf],
        min_exact=[-0.1, 0, 0.5, 1, 1.1, nan], dense_sigma=[-1, -0.5, 0, 0.8, 1, 1.1, nan, inf]).items() for v in vals]
    for kw in grid:
        o = _opts(**kw)
        ea, eb = C.create_string_buffer(256), C.create_string_buffer(256)
        assert ours.h3_cuda_sol_options_valid(o, ea, 256) == ref.h3_cuda_sol_options_valid(o, eb, 256), kw
        assert ea.value == eb.value, kw
        for block in (0, 1, 49):
            for step in (-1, 0, 1, 5):
                for video, audio in ((0.2, 0.2), (0.2, 0.9), (nan, 0.1), (1.2, 0.1), (0.8, 0.0)):
                    args = (o, block, step, video, audio)
                    assert ours.h3_cuda_sol_dense_reason(*args) == ref.h3_cuda_sol_dense_reason(*args), (kw, args)
    base = _opts()
    for kw in grid[1:]:
        for mask in range(256):
            assert (ours.h3_cuda_sol_options_match(_opts(**kw), base, mask) ==
                    ref.h3_cuda_sol_options_match(_opts(**kw), base, mask))
    # tests/test_cuda_sol_policy.c:10-26
    d = ours.h3_cuda_sol_current()
    assert (d.q_block, d.kv_block, d.min_exact, d.dense_steps) == (32, 64, 0.0, 1)
    assert ours.h3_cuda_sol_dense_reason(d, 49, 0, 0.2, 0.2) == b"early-evaluation"
    assert ours.h3_cuda_sol_dense_reason(d, 0, 1, 0.2, 0.2) == b"early-layer"
    assert ours.h3_cuda_sol_dense_reason(d, 1, 1, 0.2, 0.2) is None
    assert ours.h3_cuda_sol_dense_reason(_opts(dense_sigma=0.8), 1, 1, 0.2, 0.9) == b"high-noise"
    assert ours.h3_cuda_sol_dense_reason(_opts(min_exact=1), 49, 1, 0.2, 0.2) == b"all-exact"
    saved = ours.h3_cuda_sol_exchange(_opts(min_exact=0.5))
    assert ours.h3_cuda_sol_current().min_exact == 0.5
    nested = ours.h3_cuda_sol_exchange(_opts())
    assert nested.min_exact == 0.5
    ours.h3_cuda_sol_exchange(nested)
    assert ours.h3_cuda_sol_current().min_exact == 0.5
    ours.h3_cuda_sol_exchange(saved)
    assert ours.h3_cuda_sol_current().min_exact == 0.0
