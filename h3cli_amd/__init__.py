"""h3cli_amd — MI355X (gfx950) backend for h3cli's DiT denoise hot path.

The product is the C-ABI shared library libh3hip.so (include/h3_gpu.h,
include/h3_hip_ext.h). This package builds it (h3cli_amd.build), binds it with
ctypes (h3cli_amd._lib) and wraps it for Python callers (h3cli_amd.runtime).
"""
from ._lib import LIB_PATH, load  # noqa: F401

__all__ = ["LIB_PATH", "load"]
