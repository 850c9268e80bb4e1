"""Thin Python wrapper over the C ABI: a context object that owns tensors and
raises on errors. Every call goes straight to libh3hip.so."""
import ctypes as C

import numpy as np

from . import _lib
from ._lib import BF16, F32, I8, U32


class H3Error(RuntimeError):
    pass


_DTYPE_NP = {F32: np.float32, BF16: np.uint16, I8: np.int8, U32: np.uint32}


class Tensor:
    def __init__(self, gpu, handle, elements, dtype):
        self.gpu, self.handle, self.elements, self.dtype = gpu, handle, elements, dtype

    def free(self):
        if self.handle:
            self.gpu.lib.h3_gpu_tensor_free(self.handle)
            self.handle = None

    def read(self, count=None):
        count = self.elements if count is None else count
        lib = self.gpu.lib
        if self.dtype == I8:
            # int8 tensors are read through their device contents as raw bytes.
            raise H3Error("int8 tensors are read with read_bytes()")
        out = np.empty(count, dtype=_DTYPE_NP[self.dtype])
        fn = {F32: lib.h3_gpu_tensor_read_f32, BF16: lib.h3_gpu_tensor_read_bf16,
              U32: lib.h3_gpu_tensor_read_u32}[self.dtype]
        self.gpu.check(fn(self.handle, out.ctypes.data, count), "tensor read")
        return out

    def read_bytes(self):
        """Raw contents of any tensor (int8 included) via a u32/f32 alias read."""
        lib = self.gpu.lib
        nbytes = self.elements * np.dtype(_DTYPE_NP[self.dtype]).itemsize
        out = np.empty(nbytes, dtype=np.uint8)
        ok = lib.h3_hip_tensor_read_bytes(self.handle, out.ctypes.data, nbytes)
        self.gpu.check(ok, "tensor byte read")
        return out


class Gpu:
    def __init__(self):
        self.lib = _lib.load()
        err = C.create_string_buffer(1024)
        self.handle = self.lib.h3_gpu_create(None, err, 1024)
        if not self.handle:
            raise H3Error(f"h3_gpu_create: {err.value.decode()}")
        self.tensors = []

    # -- errors
    def error(self):
        return self.lib.h3_gpu_error(self.handle).decode()

    def check(self, ok, what=""):
        if not ok:
            raise H3Error(f"{what}: {self.error()}")
        return ok

    # -- lifecycle
    def close(self):
        for t in self.tensors:
            t.free()
        self.tensors.clear()
        if self.handle:
            self.lib.h3_gpu_free(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def begin(self):
        self.check(self.lib.h3_gpu_begin(self.handle), "begin")

    def submit(self):
        self.check(self.lib.h3_gpu_submit(self.handle), "submit")

    def cancel(self):
        self.lib.h3_gpu_cancel(self.handle)

    # -- tensors
    def _track(self, handle, n, dtype):
        if not handle:
            raise H3Error(f"tensor allocation: {self.error()}")
        t = Tensor(self, handle, n, dtype)
        self.tensors.append(t)
        return t

    def empty(self, n, dtype=BF16):
        return self._track(self.lib.h3_gpu_tensor_alloc(self.handle, n, dtype, _lib.DEVICE_ONLY), n, dtype)

    def from_bf16(self, a):
        a = np.ascontiguousarray(a, dtype=np.uint16).reshape(-1)
        return self._track(self.lib.h3_gpu_tensor_from_bf16(self.handle, a.ctypes.data, a.size), a.size, BF16)

    def from_f32(self, a):
        a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
        return self._track(self.lib.h3_gpu_tensor_from_f32(self.handle, a.ctypes.data, a.size), a.size, F32)

    def from_u32(self, a):
        a = np.ascontiguousarray(a, dtype=np.uint32).reshape(-1)
        return self._track(self.lib.h3_gpu_tensor_from_u32(self.handle, a.ctypes.data, a.size), a.size, U32)

    def free(self, t):
        t.free()
        if t in self.tensors:
            self.tensors.remove(t)

    # -- timing
    def timing_event(self):
        e = self.lib.h3_hip_timing_event_new(self.handle)
        if not e:
            raise H3Error(self.error())
        return e

    def record(self, event):
        self.check(self.lib.h3_gpu_event_record(self.handle, event), "event record")

    def elapsed_ms(self, a, b):
        ms = C.c_float()
        self.check(self.lib.h3_hip_event_elapsed_ms(self.handle, a, b, C.byref(ms)), "elapsed")
        return ms.value


class DitSynth:
    """The synthetic DiT denoise step of include/h3_dit_synth.h on its own context."""

    def __init__(self, geometry="synthetic", **overrides):
        """geometry: "synthetic" or "h3" (the real H3 block)."""
        self.lib = _lib.load()
        cfg = self.lib.h3_hip_dit_synth_h3() if geometry == "h3" else self.lib.h3_hip_dit_synth_default()
        for k, v in overrides.items():
            setattr(cfg, k, v)
        self.config = cfg
        self.gpu = Gpu()
        err = C.create_string_buffer(1024)
        self.handle = self.lib.h3_hip_dit_synth_create(self.gpu.handle, C.byref(cfg), err, 1024)
        if not self.handle:
            msg = err.value.decode()
            self.gpu.close()
            raise H3Error(f"h3_hip_dit_synth_create: {msg}")

    @property
    def rows(self):
        return self.lib.h3_hip_dit_synth_rows(self.handle)

    def kept_blocks(self):
        total = C.c_uint64()
        kept = self.lib.h3_hip_dit_synth_kept_blocks(self.handle, C.byref(total))
        return kept, total.value

    def load(self, path):
        """Load block weights from a safetensors checkpoint (reference names)."""
        err = C.create_string_buffer(1024)
        if not self.lib.h3_hip_dit_synth_load(self.handle, str(path).encode(), err, 1024):
            raise H3Error(err.value.decode())

    def step(self, step=0, dt=-0.05):
        if not self.lib.h3_hip_dit_synth_step(self.handle, step, dt):
            raise H3Error(f"step: {self.gpu.error()}")

    def read(self, name):
        h = self.lib.h3_hip_dit_synth_tensor(self.handle, name.encode())
        if not h:
            raise H3Error(f"no tensor {name}")
        n = self.lib.h3_gpu_tensor_elements(h)
        dtype = self.lib.h3_gpu_tensor_dtype(h)
        out = np.empty(n, dtype=_DTYPE_NP[dtype])
        fn = {F32: self.lib.h3_gpu_tensor_read_f32, BF16: self.lib.h3_gpu_tensor_read_bf16,
              U32: self.lib.h3_gpu_tensor_read_u32}[dtype]
        if not fn(h, out.ctypes.data, n):
            raise H3Error(self.gpu.error())
        return out

    def read_q8(self, name, rows, columns):
        """A resident per-output-channel W8A16 weight: (int8 codes [rows *
        columns], fp32 scales [rows])."""
        h = self.lib.h3_hip_dit_synth_tensor(self.handle, name.encode())
        if not h:
            raise H3Error(f"no tensor {name}")
        raw = np.empty(rows * columns + rows * 4, np.uint8)
        if not self.lib.h3_hip_tensor_copy_to_host(h, raw.ctypes.data, raw.size):
            raise H3Error(self.gpu.error())
        return raw[:rows * columns].view(np.int8).copy(), raw[rows * columns:].view(np.float32).copy()

    def close(self):
        if self.handle:
            self.lib.h3_hip_dit_synth_free(self.handle)
            self.handle = None
        self.gpu.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
