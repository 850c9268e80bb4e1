"""Host side of the FP8 projection path, checked against the reference's own C
sources compiled into oracle/_ref/libh3ref.so (src/weights/quant.c,
src/weights/quant_cache.c, src/weights/residency.c, src/digest.c) and against
hashlib: the packed descriptor sizes, the quantization policy, SHA-256, and the
metadata artifact cache (key, file name, header bytes, hit/miss/corruption
rules of tests/test_quant_cache.c), with artifacts written by one library read
by the other."""
import ctypes as C
import hashlib
import os

import numpy as np
import pytest

from h3cli_amd import _lib

REF = os.path.join(os.path.dirname(__file__), "..", "oracle", "_ref", "libh3ref.so")
need_ref = pytest.mark.skipif(not os.path.exists(REF), reason="oracle/_ref/libh3ref.so not built")


class Cache(C.Structure):
    """h3_quant_cache (quant_cache.h:13-21); struct stat is opaque here."""
    _fields_ = [("source", C.c_char_p), ("artifact", C.c_char_p), ("stamp", C.c_ubyte * 144),
                ("offset", C.c_uint64), ("bytes", C.c_uint64), ("scale", C.c_uint64), ("global_", C.c_uint64),
                ("mode", C.c_uint), ("rows", C.c_uint), ("columns", C.c_uint), ("key", C.c_ubyte * 32),
                ("lock", C.c_int)]


def _bind(lib):
    lib.h3_weight_packed_size.restype = C.c_int
    lib.h3_weight_packed_size.argtypes = [C.c_uint32, C.c_uint32, C.c_int] + [C.POINTER(C.c_uint64)] * 3
    lib.h3_quant_name.restype = C.c_char_p
    lib.h3_quant_name.argtypes = [C.c_int]
    lib.h3_quant_parse.argtypes = [C.c_char_p, C.POINTER(C.c_int)]
    lib.h3_quant_options.argtypes = [C.c_int, C.c_char_p, C.c_char_p, C.c_size_t]
    lib.h3_quant_projection.argtypes = [C.c_char_p, C.c_int]
    lib.h3_quant_recipe.restype = C.c_uint
    lib.h3_quant_recipe.argtypes = [C.c_int, C.c_int]
    lib.h3_quant_execution_recipe.restype = C.c_uint
    lib.h3_quant_execution_recipe.argtypes = [C.c_int, C.c_int, C.c_int]
    lib.h3_quant_projection_policy.argtypes = [C.c_char_p, C.c_int, C.c_int]
    lib.h3_quant_cache_open.restype = C.POINTER(Cache)
    lib.h3_quant_cache_open.argtypes = [C.c_char_p, C.c_char_p, C.c_uint64, C.c_uint, C.c_uint, C.c_int, C.c_uint64,
                                        C.c_uint64, C.c_uint64, C.c_char_p, C.c_size_t]
    lib.h3_quant_cache_read.argtypes = [C.POINTER(Cache), C.c_void_p, C.c_char_p, C.c_size_t]
    lib.h3_quant_cache_write.argtypes = [C.POINTER(Cache), C.c_void_p, C.c_char_p, C.c_size_t]
    lib.h3_quant_cache_unchanged.argtypes = [C.POINTER(Cache), C.c_char_p, C.c_size_t]
    lib.h3_quant_cache_close.argtypes = [C.POINTER(Cache)]
    lib.h3_quant_cache_close.restype = None
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


@need_ref
def test_quant_policy_matches_reference(ours, ref, tmp_path, monkeypatch):
    for m in range(-1, 5):
        assert ours.h3_quant_name(m) == ref.h3_quant_name(m)
    for text in (b"off", b"fp8", b"nvfp4", b"FP8", b"", b"invalid", b"fp4"):
        a, b = C.c_int(-7), C.c_int(-7)
        assert ours.h3_quant_parse(text, C.byref(a)) == ref.h3_quant_parse(text, C.byref(b)) and a.value == b.value
    names = [b"blocks.0.attn.qkv_proj.weight", b"blocks.49.mlp.fc2.weight", b"blocks.7.mlp.fc1.weight",
             b"blocks.12.attn.out_proj.weight", b"blocks..attn.qkv_proj.weight", b"blocks.x.mlp.fc1.weight",
             b"blocks.3.attn.q_norm.weight", b"block.3.mlp.fc1.weight", b"blocks.3.mlp.fc1.weight.x", b"",
             b"blocks.0.mlp.fc2.weight"]
    for name in names:
        for req in (0, 1, 2):
            assert ours.h3_quant_projection(name, req) == ref.h3_quant_projection(name, req), name
            for adaptive in (0, 1):
                assert ours.h3_quant_projection_policy(name, req, adaptive) == \
                    ref.h3_quant_projection_policy(name, req, adaptive), name
    for mode in range(0, 3):
        for adaptive in (0, 1):
            assert ours.h3_quant_recipe(mode, adaptive) == ref.h3_quant_recipe(mode, adaptive)
            for attention in range(0, 5):
                assert ours.h3_quant_execution_recipe(mode, adaptive, attention) == \
                    ref.h3_quant_execution_recipe(mode, adaptive, attention)
    writable = tmp_path / "w"
    writable.mkdir()
    readonly = tmp_path / "r"
    readonly.mkdir()
    os.chmod(readonly, 0o500)
    afile = tmp_path / "file"
    afile.write_bytes(b"x")
    caches = [None, b"", str(writable).encode(), str(writable / "a" / "b").encode(), str(afile).encode(),
              str(afile / "sub").encode()]
    if os.geteuid() != 0:
        caches.append(str(readonly / "sub").encode())
    for verify in (None, "0", "1", "bad"):
        if verify is None:
            monkeypatch.delenv("H3_QUANT_VERIFY", raising=False)
        else:
            monkeypatch.setenv("H3_QUANT_VERIFY", verify)
        for mode in (-1, 0, 1, 2, 3):
            for cache in caches:
                ea, eb = C.create_string_buffer(256), C.create_string_buffer(256)
                a = ours.h3_quant_options(mode, cache, ea, 256)
                b = ref.h3_quant_options(mode, cache, eb, 256)
                assert a == b and ea.value == eb.value, (verify, mode, cache, ea.value, eb.value)
        assert ours.h3_quant_verify() == ref.h3_quant_verify()
    os.chmod(readonly, 0o700)


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


def _entry(lib, d, source, offset=0, mode=2, err=None):
    err = err if err is not None else C.create_string_buffer(512)
    return lib.h3_quant_cache_open(str(d).encode(), str(source).encode(), offset, 128, 128, mode, 9232, 8192, 9216,
                                   err, 512), err


def _flip(path, offset):
    with open(path, "r+b") as f:
        f.seek(offset)
        b = f.read(1)
        f.seek(offset)
        f.write(bytes([b[0] ^ 1]))


def test_metadata_cache_rules(ours, tmp_path):
    """The checks of the reference's tests/test_quant_cache.c:26-91, on this
    library: miss then hit, stable key, aliases share it, offset and mode change
    it, range errors, every header field and the exact length validated,
    payload bits not hashed, a changed source refused, no staging files left."""
    lib = ours
    source = tmp_path / "source"
    source.write_bytes(bytes(65536))
    payload = np.full(9232, 17, np.uint8)
    back = np.zeros(9232, np.uint8)
    err = C.create_string_buffer(512)
    c, _ = _entry(lib, tmp_path, source)
    assert c
    artifact = c.contents.artifact.decode()
    key = bytes(c.contents.key)
    assert lib.h3_quant_cache_read(c, back.ctypes.data, err, 512) == 0
    assert lib.h3_quant_cache_write(c, payload.ctypes.data, err, 512)
    assert lib.h3_quant_cache_read(c, back.ctypes.data, err, 512) == 1 and np.array_equal(back, payload)
    lib.h3_quant_cache_close(c)
    assert os.path.basename(artifact) == f"m2-nvfp4-128x128-{key.hex()}.h3q"
    c, _ = _entry(lib, tmp_path, source)
    assert bytes(c.contents.key) == key and lib.h3_quant_cache_read(c, back.ctypes.data, err, 512) == 1
    lib.h3_quant_cache_close(c)
    os.symlink(source, tmp_path / "alias")
    c, _ = _entry(lib, tmp_path, tmp_path / "alias")
    assert bytes(c.contents.key) == key
    lib.h3_quant_cache_close(c)
    for kw in (dict(offset=2), dict(mode=1)):
        c, _ = _entry(lib, tmp_path, source, **kw)
        assert bytes(c.contents.key) != key
        lib.h3_quant_cache_close(c)
    c, e = _entry(lib, tmp_path, source, offset=65536)
    assert not c and b"range" in e.value
    for field in (8, 12, 16, 20, 24, 28, 32, 40, 48, 56, 88, 96, 127):
        c, _ = _entry(lib, tmp_path, source)
        _flip(artifact, field)
        assert lib.h3_quant_cache_read(c, back.ctypes.data, err, 512) == -1, field
        assert b"corrupt/incompatible metadata quantization artifact" in err.value
        assert lib.h3_quant_cache_write(c, payload.ctypes.data, err, 512)
        lib.h3_quant_cache_close(c)
    c, _ = _entry(lib, tmp_path, source)
    os.truncate(artifact, 128 + 9232 - 1)
    assert lib.h3_quant_cache_read(c, back.ctypes.data, err, 512) == -1
    assert lib.h3_quant_cache_write(c, payload.ctypes.data, err, 512)
    with open(artifact, "ab") as f:
        f.write(b"x")
    assert lib.h3_quant_cache_read(c, back.ctypes.data, err, 512) == -1
    assert lib.h3_quant_cache_write(c, payload.ctypes.data, err, 512)
    with open(artifact, "r+b") as f:          # payload bytes are not hashed
        f.seek(128)
        f.write(bytes([18]))
    assert lib.h3_quant_cache_read(c, back.ctypes.data, err, 512) == 1 and back[0] == 18
    st = os.stat(source)
    with open(source, "r+b") as f:
        f.write(bytes([42]))
    os.utime(source, ns=(st.st_atime_ns, st.st_mtime_ns))
    assert not lib.h3_quant_cache_unchanged(c, err, 512) and b"source changed" in err.value
    assert not lib.h3_quant_cache_write(c, payload.ctypes.data, err, 512)
    lib.h3_quant_cache_close(c)
    c, _ = _entry(lib, tmp_path, source)       # ctime moved: a new key, a miss
    assert bytes(c.contents.key) != key and lib.h3_quant_cache_read(c, back.ctypes.data, err, 512) == 0
    lib.h3_quant_cache_close(c)
    c, e = _entry(lib, tmp_path, source, mode=3)
    assert not c and b"invalid quantization metadata arguments" in e.value
    assert not any(".tmp." in n for n in os.listdir(tmp_path))


@need_ref
def test_metadata_cache_interchangeable_with_reference(ours, ref, tmp_path):
    """Same key, artifact path and file bytes as the reference's cache, and an
    artifact written by either library is a hit for the other."""
    source = tmp_path / "weights.bin"
    rng = np.random.default_rng(5)
    source.write_bytes(rng.integers(0, 256, 1 << 17, dtype=np.uint8).tobytes())
    payload = rng.integers(0, 256, 9232, dtype=np.uint8)
    back = np.zeros(9232, np.uint8)
    err = C.create_string_buffer(512)
    for mode, offset in ((1, 0), (2, 0), (1, 4096), (2, 777)):
        d_ours, d_ref = tmp_path / f"o{mode}{offset}", tmp_path / f"r{mode}{offset}"
        d_ours.mkdir()
        d_ref.mkdir()
        a, _ = _entry(ours, d_ours, source, offset, mode)
        b, _ = _entry(ref, d_ref, source, offset, mode)
        assert bytes(a.contents.key) == bytes(b.contents.key)
        assert os.path.basename(a.contents.artifact) == os.path.basename(b.contents.artifact)
        assert ours.h3_quant_cache_write(a, payload.ctypes.data, err, 512)
        assert ref.h3_quant_cache_write(b, payload.ctypes.data, err, 512)
        name = os.path.basename(a.contents.artifact.decode())
        assert (d_ours / name).read_bytes() == (d_ref / name).read_bytes()
        ours.h3_quant_cache_close(a)
        ref.h3_quant_cache_close(b)
        # Cross reads: ours reads the reference's directory and vice versa.
        a, _ = _entry(ours, d_ref, source, offset, mode)
        assert ours.h3_quant_cache_read(a, back.ctypes.data, err, 512) == 1 and np.array_equal(back, payload)
        ours.h3_quant_cache_close(a)
        b, _ = _entry(ref, d_ours, source, offset, mode)
        assert ref.h3_quant_cache_read(b, back.ctypes.data, err, 512) == 1 and np.array_equal(back, payload)
        ref.h3_quant_cache_close(b)
    for bad in (dict(offset=1 << 17), dict(mode=0)):
        ea, eb = C.create_string_buffer(512), C.create_string_buffer(512)
        a, _ = _entry(ours, tmp_path, source, err=ea, **bad)
        b, _ = _entry(ref, tmp_path, source, err=eb, **bad)
        assert not a and not b and ea.value == eb.value
