"""File -> device fills (h3_gpu_tensor_read_file_bf16 / _stream_file_bf16 /
h3_gpu_tensor_load_bf16, reference src/gpu.h:220-236, behaviour of
src/cuda/gpu_cuda.cu:761-846): the device tensor holds the file's bytes exactly,
at any offset and for ranges that wrap the staging ring several times; short
files and missing files fail with the reference's messages; repeated streamed
fills of one tensor, each read by a kernel, stay ordered."""
import ctypes as C

import numpy as np
import pytest

from h3cli_amd import _lib
from h3cli_amd.runtime import Gpu, H3Error

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[stream-file] {msg}", flush=True)


def write(path, data, offset):
    with open(path, "wb") as f:
        f.write(bytes(range(256)) * (offset // 256) + bytes(offset % 256))
        f.write(np.ascontiguousarray(data, np.uint16).tobytes())


@pytest.mark.parametrize("n,offset", [(1, 0), (4097, 2), (3 * (4 << 20) + 123, 4096 + 6),
                                      (9 * (4 << 20) + 1, 10)])
def test_read_file_exact(tmp_path, n, offset):
    say(f"read_file n={n} offset={offset}")
    rng = np.random.default_rng(n)
    data = rng.integers(0, 1 << 16, n, dtype=np.uint16)
    path = tmp_path / "w.bin"
    write(path, data, offset)
    with Gpu() as g:
        t = g.empty(n + 7)
        err = C.create_string_buffer(512)
        assert g.lib.h3_gpu_tensor_read_file_bf16(t.handle, str(path).encode(), offset, n, err, 512), err.value
        assert g.lib.h3_gpu_synchronize(g.handle), g.error()
        got = t.read(n)
        assert np.array_equal(got, data)
        h = g.lib.h3_gpu_tensor_load_bf16(g.handle, str(path).encode(), offset, n)
        assert h, g.error()
        u = g._track(h, n, _lib.BF16)
        assert g.lib.h3_gpu_synchronize(g.handle), g.error()
        assert np.array_equal(u.read(n), data)


def test_short_and_missing_file(tmp_path):
    say("short and missing files")
    path = tmp_path / "short.bin"
    n = 3 * (4 << 20)
    write(path, np.zeros(n - 5, np.uint16), 0)
    with Gpu() as g:
        t = g.empty(n)
        err = C.create_string_buffer(512)
        assert not g.lib.h3_gpu_tensor_read_file_bf16(t.handle, str(path).encode(), 0, n, err, 512)
        msg = err.value.decode()
        assert msg.startswith(f"read weight {path} at ") and msg.endswith("unexpected EOF"), msg
        # The failing offset is the first byte the file does not hold.
        assert f" at {2 * (n - 5)}:" in msg, msg
        assert not g.lib.h3_gpu_tensor_read_file_bf16(t.handle, str(tmp_path / "none").encode(), 0, 4, err, 512)
        assert err.value.decode().startswith(str(tmp_path / "none") + ": No such file"), err.value
        # The context still works after a failed fill.
        ok = np.arange(1000, dtype=np.uint16)
        write(path, ok, 0)
        assert g.lib.h3_gpu_tensor_read_file_bf16(t.handle, str(path).encode(), 0, 1000, err, 512), err.value
        assert g.lib.h3_gpu_synchronize(g.handle), g.error()
        assert np.array_equal(t.read(1000), ok)


def test_streamed_fills_ordered_with_compute(tmp_path):
    """Fill one tensor from file generations 0..5 in turn; after each fill a
    copy kernel on the compute stream reads it into a result row. Every row
    must equal its own generation: a fill that overtook the previous read, or
    a read that ran before its fill, would show another generation."""
    say("streamed fills ordered with compute")
    n = 5 * (4 << 20) + 17
    gens = 6
    with Gpu() as g:
        slot = g.empty(n)
        out = g.empty(n * gens)
        lib = g.lib
        err = C.create_string_buffer(512)
        for i in range(gens):
            path = tmp_path / f"g{i}.bin"
            write(path, np.full(n, 0x3f80 + i, np.uint16), 2 * i)
        g.begin()
        for i in range(gens):
            ok = lib.h3_gpu_tensor_stream_file_bf16(slot.handle, str(tmp_path / f"g{i}.bin").encode(), 2 * i, n, err, 512)
            assert ok, err.value
            assert lib.h3_gpu_copy_bf16(g.handle, out.handle, i * n, slot.handle, 0, n), g.error()
        g.submit()
        got = out.read().reshape(gens, n)
        for i in range(gens):
            assert (got[i] == 0x3f80 + i).all(), i
        st = _lib.GpuStats()
        assert lib.h3_gpu_get_stats(g.handle, C.byref(st))
        assert st.streamed_bytes >= gens * n * 2
