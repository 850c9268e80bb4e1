"""Device query and weight planning on the GPU box (reference src/device.h,
src/gpu.h:36-40)."""
import ctypes as C

import pytest

from h3cli_amd import _lib
from h3cli_amd.runtime import Gpu

pytestmark = pytest.mark.gpu


class DeviceInfo(C.Structure):
    _fields_ = [("name", C.c_char * 128), ("architecture", C.c_char * 128), ("physical_memory", C.c_uint64),
                ("recommended_working_set", C.c_uint64), ("max_buffer_length", C.c_uint64),
                ("apple_gpu_family", C.c_int), ("metal4", C.c_int), ("unified_memory", C.c_int),
                ("backend", C.c_char * 16), ("device_index", C.c_int), ("cuda_compute_major", C.c_int),
                ("cuda_compute_minor", C.c_int), ("cuda_driver_version", C.c_int),
                ("cuda_runtime_version", C.c_int), ("device_memory", C.c_uint64),
                ("free_device_memory", C.c_uint64), ("multiprocessor_count", C.c_int), ("cuda_uuid", C.c_uint8 * 16)]


def test_device_query_reports_mi355x():
    lib = _lib.load()
    info, err = DeviceInfo(), C.create_string_buffer(256)
    assert lib.h3_device_query(C.byref(info), err, 256) == 1, err.value
    print(f"[device] {info.name.decode()} {info.architecture.decode()} CUs={info.multiprocessor_count} "
          f"HBM={info.device_memory / 2**30:.1f} GiB", flush=True)
    assert info.backend == b"hip" and info.architecture.startswith(b"gfx950")
    assert info.multiprocessor_count == 256 and info.device_memory > 250 * 2**30
    assert lib.h3_device_memory_fits(1 << 30) == 1 and lib.h3_device_memory_fits(1 << 50) == 0


def test_weight_planner_on_device(monkeypatch):
    from tests.test_ref_host import WeightPlan
    monkeypatch.delenv("H3_CUDA_WEIGHT_MODE", raising=False)
    g = Gpu()
    try:
        block = 246_400_000
        # 40 synthetic blocks (9.9 GB) fit in 288 GB: resident, no slots.
        assert g.lib.h3_gpu_plan_weights(g.handle, 40 * block, 20 << 30) == 0
        plan = WeightPlan()
        mask = (1 << 40) - 1
        assert g.lib.h3_gpu_plan_bf16_weights(g.handle, mask, block, 20 << 30, 0, -1, C.byref(plan)) == 1, g.error()
        assert plan.effective_mode == 1 and plan.resident_count == 40 and plan.slot_bytes == 0
        # Forced streaming keeps two slots and no resident blocks.
        assert g.lib.h3_gpu_plan_bf16_weights(g.handle, mask, block, 20 << 30, 1, -1, C.byref(plan)) == 1
        assert plan.effective_mode == 2 and plan.resident_count == 0 and plan.slot_bytes == 2 * block
        # A retry cap of 5 keeps the five lowest blocks resident.
        assert g.lib.h3_gpu_plan_bf16_weights(g.handle, mask, block, 20 << 30, 0, 5, C.byref(plan)) == 1
        assert plan.effective_mode == 0 and plan.resident_mask == 0b11111
        assert g.lib.h3_gpu_weight_plan_compatible(g.handle, 0) == 0  # partial automatic plan is recomputed
    finally:
        g.close()
