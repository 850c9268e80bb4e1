"""The safetensors reader (h3cli_amd/host/safetensors.c, include/h3_safetensors.h).

Pinned two ways:
- files written by the `safetensors` package (the format's reference writer):
  every tensor's dtype, shape, byte range and bytes, and the metadata;
- the reference's own reader (src/weights/safetensors.c, compiled in place into
  oracle/_ref/libh3ref.so): the same verdict, error text and tensor table on a
  corpus of valid and malformed headers and on seeded byte mutations of a
  valid file. Skipped when libh3ref.so was not built.
"""
import ctypes as C
import json
import os
import random
import struct

import numpy as np
import pytest

from h3cli_amd import _lib

REF = os.path.join(os.path.dirname(__file__), "..", "oracle", "_ref", "libh3ref.so")


class StTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("dtype", C.c_int), ("ndim", C.c_int), ("shape", C.c_uint64 * 8),
                ("data_begin", C.c_uint64), ("data_end", C.c_uint64), ("file_offset", C.c_uint64)]


class StHeader(C.Structure):
    _fields_ = [("path", C.c_char_p), ("file_size", C.c_uint64), ("header_size", C.c_uint64),
                ("tensors", C.POINTER(StTensor)), ("tensor_count", C.c_size_t),
                ("metadata_keys", C.POINTER(C.c_char_p)), ("metadata_values", C.POINTER(C.c_char_p)),
                ("metadata_count", C.c_size_t)]


DTYPES = ["UNKNOWN", "BOOL", "I8", "U8", "I16", "U16", "F16", "BF16", "I32", "U32", "F32", "I64", "U64", "F64"]


def bind(lib):
    lib.h3_st_read_header.restype = C.c_int
    lib.h3_st_read_header.argtypes = [C.c_char_p, C.POINTER(StHeader), C.c_char_p, C.c_size_t]
    lib.h3_st_free_header.restype = None
    lib.h3_st_free_header.argtypes = [C.POINTER(StHeader)]
    lib.h3_st_read_data.restype = C.c_int
    lib.h3_st_read_data.argtypes = [C.POINTER(StHeader), C.POINTER(StTensor), C.c_void_p, C.c_size_t, C.c_char_p,
                                    C.c_size_t]
    lib.h3_st_find.restype = C.POINTER(StTensor)
    lib.h3_st_find.argtypes = [C.POINTER(StHeader), C.c_char_p]
    lib.h3_st_tensor_elements.restype = C.c_uint64
    lib.h3_st_tensor_elements.argtypes = [C.POINTER(StTensor)]
    lib.h3_dtype_size.restype = C.c_size_t
    lib.h3_dtype_size.argtypes = [C.c_int]
    lib.h3_dtype_name.restype = C.c_char_p
    lib.h3_dtype_name.argtypes = [C.c_int]
    lib.h3_st_file_range.restype = C.c_int
    lib.h3_st_file_range.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64]
    return lib


@pytest.fixture(scope="module")
def ours():
    return bind(_lib.load())


@pytest.fixture(scope="module")
def ref():
    if not os.path.exists(REF):
        pytest.skip("oracle/_ref/libh3ref.so not built")
    return bind(C.CDLL(REF))


def read(lib, path, with_data=False):
    """(ok, error, tensors, metadata) with tensors as tuples; data bytes if asked."""
    h = StHeader()
    err = C.create_string_buffer(512)
    ok = lib.h3_st_read_header(str(path).encode(), C.byref(h), err, 512)
    tensors, meta = [], []
    if ok:
        for i in range(h.tensor_count):
            t = h.tensors[i]
            row = (t.name.decode("utf-8"), DTYPES[t.dtype], tuple(t.shape[:t.ndim]), t.data_begin, t.data_end,
                   t.file_offset)
            if with_data:
                buf = (C.c_uint8 * max(1, t.data_end - t.data_begin))()
                e2 = C.create_string_buffer(256)
                assert lib.h3_st_read_data(C.byref(h), C.byref(t), buf, t.data_end - t.data_begin, e2, 256), e2.value
                row = row + (bytes(buf)[: t.data_end - t.data_begin],)
            tensors.append(row)
        meta = [(h.metadata_keys[i].decode("utf-8"), h.metadata_values[i].decode("utf-8"))
                for i in range(h.metadata_count)]
        lib.h3_st_free_header(C.byref(h))
    return bool(ok), err.value.decode("utf-8", "replace"), tensors, meta


def write_raw(path, header_text, payload=b"", size_field=None):
    body = header_text.encode("utf-8") if isinstance(header_text, str) else header_text
    n = len(body) if size_field is None else size_field
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", n) + body + payload)


def test_files_written_by_safetensors_package(ours, tmp_path):
    torch = pytest.importorskip("torch")
    from safetensors import safe_open
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(3)
    tensors = {
        "blocks.0.attn.qkv_proj.weight": torch.randn(96, 64, generator=g).to(torch.bfloat16),
        "blocks.0.norm1.weight": torch.randn(64, generator=g).to(torch.bfloat16),
        "f16": torch.randn(3, 5, generator=g).to(torch.float16),
        "f32": torch.randn(2, 3, 4, generator=g),
        "f64": torch.randn(7, generator=g).double(),
        "i8": torch.randint(-128, 127, (9,), generator=g).to(torch.int8),
        "u8": torch.randint(0, 255, (4, 4), generator=g).to(torch.uint8),
        "i16": torch.randint(-1000, 1000, (5,), generator=g).to(torch.int16),
        "i32": torch.randint(-10 ** 6, 10 ** 6, (6,), generator=g).to(torch.int32),
        "i64": torch.randint(-10 ** 9, 10 ** 9, (3,), generator=g),
        "flags": torch.tensor([True, False, True]),
        "scalar": torch.tensor(2.5),
        "empty": torch.zeros(0, 3),
        "nested.name/with\"quote": torch.ones(2),
    }
    meta = {"format": "pt", "note": "ünïcode ✓", "escaped": "tab\there"}
    path = tmp_path / "model.safetensors"
    save_file(tensors, str(path), metadata=meta)
    ok, err, table, got_meta = read(ours, path, with_data=True)
    assert ok, err
    header = json.loads(path.read_bytes()[8:8 + struct.unpack("<Q", path.read_bytes()[:8])[0]])
    base = 8 + struct.unpack("<Q", path.read_bytes()[:8])[0]
    by_name = {row[0]: row for row in table}
    assert set(by_name) == set(tensors)
    with safe_open(str(path), framework="pt") as f:
        assert f.metadata() == meta and dict(got_meta) == meta
        for name, ref in tensors.items():
            _, dtype, shape, begin, end, off, data = by_name[name]
            assert dtype == header[name]["dtype"] and list(shape) == header[name]["shape"], name
            assert [begin, end] == header[name]["data_offsets"] and off == base + begin
            t = f.get_tensor(name)
            expect = t.reshape(-1).contiguous().view(torch.uint8).numpy().tobytes() if t.numel() else b""
            assert data == expect, name


def test_api_helpers(ours):
    assert [ours.h3_dtype_size(d) for d in range(14)] == [0, 1, 1, 1, 2, 2, 2, 2, 4, 4, 4, 8, 8, 8]
    assert [ours.h3_dtype_name(d).decode() for d in range(14)] == DTYPES
    assert ours.h3_dtype_name(99) == b"UNKNOWN" and ours.h3_dtype_size(99) == 0
    assert ours.h3_st_file_range(8, 10, 18) and not ours.h3_st_file_range(8, 11, 18)
    assert not ours.h3_st_file_range(2 ** 63, 0, 2 ** 64 - 1)


def test_read_data_errors(ours, tmp_path):
    path = tmp_path / "a.safetensors"
    write_raw(path, '{"x":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', b"\0" * 8)
    h = StHeader()
    err = C.create_string_buffer(256)
    assert ours.h3_st_read_header(str(path).encode(), C.byref(h), err, 256)
    t = ours.h3_st_find(C.byref(h), b"x")
    assert t and ours.h3_st_tensor_elements(t) == 2 and not ours.h3_st_find(C.byref(h), b"y")
    buf = (C.c_uint8 * 8)()
    assert not ours.h3_st_read_data(C.byref(h), t, buf, 4, err, 256)
    assert err.value == b"x: expected 8 bytes, got 4"
    ours.h3_st_free_header(C.byref(h))


TENSOR = '"t":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}'
CORPUS = [
    ("{" + TENSOR + "}", 8),
    ("{" + TENSOR + "}    ", 8),
    (" {" + TENSOR + "}", 8),
    ("{}", 0),
    ("{}", 4),
    ('{"__metadata__":{}}', 0),
    ('{"__metadata__":{"a":"1","b":"2"},' + TENSOR + "}", 8),
    ('{"__metadata__":{"a":"1","a":"2"}}', 0),
    ('{"__metadata__":{},"__metadata__":{}}', 0),
    ('{"__metadata__":{"a":1}}', 0),
    ('{"__metadata__":{"a":"1",}}', 0),
    ('{"__metadata__":"x"}', 0),
    ("{" + TENSOR + "," + TENSOR + "}", 8),
    ('{"t":{"dtype":"F32","shape":[2],"data_offsets":[0,8]},"u":{"dtype":"F32","shape":[1],"data_offsets":[4,8]}}', 8),
    ('{"t":{"dtype":"F32","shape":[2],"data_offsets":[0,8]},"u":{"dtype":"F32","shape":[1],"data_offsets":[12,16]}}', 16),
    ('{"t":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}', 8),
    ('{"t":{"dtype":"F32","shape":[3],"data_offsets":[0,8]}}', 8),
    ('{"t":{"dtype":"F33","shape":[2],"data_offsets":[0,8]}}', 8),
    ('{"t":{"dtype":"BF16","shape":[1,1,1,1,1,1,1,1,4],"data_offsets":[0,8]}}', 8),
    ('{"t":{"dtype":"BF16","shape":[1,1,1,1,1,1,1,4],"data_offsets":[0,8]}}', 8),
    ('{"t":{"dtype":"F32","shape":[02],"data_offsets":[0,8]}}', 8),
    ('{"t":{"dtype":"F32","shape":[-2],"data_offsets":[0,8]}}', 8),
    ('{"t":{"dtype":"F32","shape":[2.0],"data_offsets":[0,8]}}', 8),
    ('{"t":{"dtype":"F32","shape":[18446744073709551616],"data_offsets":[0,8]}}', 8),
    ('{"t":{"dtype":"U8","shape":[4294967296,4294967296],"data_offsets":[0,8]}}', 8),
    ('{"t":{"dtype":"F64","shape":[2305843009213693952,8],"data_offsets":[0,8]}}', 8),
    ('{"t":{"dtype":"F32","shape":[2],"data_offsets":[8,0]}}', 8),
    ('{"t":{"dtype":"F32","shape":[2],"data_offsets":[0,9]}}', 8),
    ('{"t":{"dtype":"F32","dtype":"F32","shape":[2],"data_offsets":[0,8]}}', 8),
    ('{"t":{"dtype":"F32","shape":[2],"shape":[2],"data_offsets":[0,8]}}', 8),
    ('{"t":{"dtype":"F32","shape":[2],"data_offsets":[0,8],"data_offsets":[0,8]}}', 8),
    ('{"t":{"dtype":"F32","shape":[2],"data_offsets":[0,8],"extra":1}}', 8),
    ('{"t":{"dtype":"F32","shape":[2]}}', 8),
    ('{"t":{}}', 0),
    ('{"t":{"dtype":"F32","shape":[2],"data_offsets":[0,8],}}', 8),
    ('{"t":{"dtype":"F32" "shape":[2],"data_offsets":[0,8]}}', 8),
    ('{"t":{"dtype":"F32","shape":[2 3],"data_offsets":[0,8]}}', 8),
    ('{"t":{"dtype":"F32","shape":[2', 0),
    ('{"t":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}', 8),
    ('{"t":{"dtype":"F32","shape":[2],"data_offsets":[0,8]} x', 8),
    ('{"t":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}}', 8),
    ('{"t":{"dtype":"F32","shape":[2],"data_offsets":[0,8]};', 8),
    ('{"t":{"dtype":"F32","shape":[2],"data_offsets":[0 8]}}', 8),
    ('{t:1}', 0),
    ('[]', 0),
    ('{"\\u00e9\\ud83d\\ude00":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', 8),
    ('{"\\u0000":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', 8),
    ('{"\\ud83d":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', 8),
    ('{"\\ude00":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', 8),
    ('{"\\ud83d\\u0041":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', 8),
    ('{"\\x41":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', 8),
    ('{"\\u12G4":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', 8),
    ('{"a\\"b\\\\c\\/d\\b\\f\\n\\r\\t":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', 8),
    (b'{"\xc3\xa9":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', 8),
    (b'{"\xc0\x80":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', 8),
    (b'{"\xed\xa0\x80":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', 8),
    (b'{"\xe0\x80\x80":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', 8),
    (b'{"\xf4\x90\x80\x80":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', 8),
    (b'{"\xf0\x9f\x98\x80":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', 8),
    (b'{"\xe2\x82":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', 8),
    (b'{"a\x01":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', 8),
    (b'{"a\tb":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', 8),
    ('{"e":{"dtype":"F32","shape":[0],"data_offsets":[0,0]},' + TENSOR + "}", 8),
    ('{"s":{"dtype":"F64","shape":[],"data_offsets":[0,8]}}', 8),
]


def test_corpus_matches_reference(ours, ref, tmp_path):
    path = tmp_path / "c.safetensors"
    for i, (text, payload) in enumerate(CORPUS):
        write_raw(path, text, b"\x5a" * payload)
        a, b = read(ours, path), read(ref, path)
        assert a == b, (i, text, a, b)
    # Header-size field and file-size cases.
    for size_field, body, payload in ((0, "{}", 0), (10 ** 12, "{}", 0), (4, '{}  ', 0), (300 * 2 ** 20, "{}", 0)):
        write_raw(path, body, b"\0" * payload, size_field=size_field)
        assert read(ours, path) == read(ref, path), size_field
    path.write_bytes(b"\x02\0\0")
    assert read(ours, path) == read(ref, path)
    missing = tmp_path / "missing.safetensors"
    assert read(ours, missing) == read(ref, missing) and not read(ours, missing)[0]


def test_mutations_match_reference(ours, ref, tmp_path):
    """Seeded byte mutations of a valid multi-tensor header: both readers give
    the same verdict, error text and table."""
    base = ('{"__metadata__":{"format":"pt","k\\u00e9y":"v"},'
            '"a.weight":{"dtype":"BF16","shape":[2,3],"data_offsets":[0,12]},'
            '"b":{"dtype":"F32","shape":[3],"data_offsets":[12,24]},'
            '"c":{"data_offsets":[24,32],"shape":[1],"dtype":"I64"}}  ').encode()
    payload = bytes(range(32))
    alphabet = b'{}[]":,\\u0123456789abcdefFI -.\x00\x1f\x80\xc3\xe2\xed\xf0\xff'
    rng = random.Random(12345)
    path = tmp_path / "m.safetensors"
    accepted = 0
    for trial in range(3000):
        body = bytearray(base)
        for _ in range(rng.randint(1, 3)):
            op, at = rng.randrange(3), rng.randrange(len(body))
            if op == 0:
                body[at] = rng.choice(alphabet)
            elif op == 1:
                del body[at]
            else:
                body.insert(at, rng.choice(alphabet))
        extra = rng.choice((0, 0, 0, 4, -4))
        write_raw(path, bytes(body), payload[: max(0, 32 + extra)] + (b"\0" * max(0, extra)))
        a, b = read(ours, path), read(ref, path)
        assert a == b, (trial, bytes(body), a, b)
        accepted += a[0]
    assert 0 < accepted < 3000
