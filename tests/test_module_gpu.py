"""Module entries of the C-ABI (ts_hip_module_load_data / _get_function /
_launch / _unload: hipModuleLoadData, hipModuleGetFunction,
hipModuleLaunchKernel): a stand-alone gfx950 code object built with the
package (ts_probe.hsaco, y = a*x + y) is loaded from memory, launched on the
library stream and checked bit for bit against numpy's fp32 a*x + y."""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import pytest

from conftest import assert_bits_equal

pytestmark = pytest.mark.gpu

PROBE = Path(__file__).resolve().parents[1] / "train-station_amd" / "ts_probe.hsaco"


def test_load_launch_unload():
    from gpu_util import Dev, sync
    from train_station_amd._ffi import hip, hip_check
    import train_station_amd as T

    assert PROBE.exists(), "ts_probe.hsaco is built by train-station_amd/Makefile"
    image = PROBE.read_bytes()
    buf = ctypes.create_string_buffer(image, len(image))
    mod, fn = ctypes.c_void_p(), ctypes.c_void_p()
    hip_check(hip.ts_hip_module_load_data(buf, ctypes.byref(mod)))
    try:
        hip_check(hip.ts_hip_module_get_function(mod, b"ts_probe_axpy", ctypes.byref(fn)))
        assert hip.ts_hip_module_get_function(mod, b"no_such_kernel", ctypes.byref(ctypes.c_void_p())) != 0
        # that failure was reported once: the next launch of the library reports its own status
        scratch = Dev(16)
        assert hip.ts_hip_fill(scratch.ptr, 1.0, 16, T.stream()) == 0
        rng = np.random.default_rng(3)
        for n in (1, 255, 4099, 1 << 20):
            x = rng.standard_normal(n).astype(np.float32)
            y = rng.standard_normal(n).astype(np.float32)
            dx, dy = Dev.of(x), Dev.of(y)
            a = ctypes.c_float(1.75)
            px, py, pn = ctypes.c_void_p(dx.ptr), ctypes.c_void_p(dy.ptr), ctypes.c_ulonglong(n)
            params = (ctypes.c_void_p * 4)(*[ctypes.cast(ctypes.pointer(v), ctypes.c_void_p) for v in (a, px, py, pn)])
            hip_check(hip.ts_hip_module_launch(fn, (n + 255) // 256, 1, 1, 256, 1, 1, 0, T.stream(), params))
            sync()
            want = np.float32(1.75) * x + y  # fp32 multiply, then fp32 add
            assert_bits_equal(dy.get(), want, f"n={n}")
        # a block over 1024 threads is refused before reaching HIP
        assert hip.ts_hip_module_launch(fn, 1, 1, 1, 2048, 1, 1, 0, T.stream(), params) != 0
    finally:
        hip_check(hip.ts_hip_module_unload(mod))
