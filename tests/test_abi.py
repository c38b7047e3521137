"""The C-ABI libraries load and export every function include/*.h declares.
CPU only: nothing here launches a kernel."""
from __future__ import annotations

import ctypes
import re

from conftest import ROOT

PKG = ROOT / "train-station_amd"


def declared(header: str) -> set[str]:
    text = (ROOT / "include" / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(ts_[a-z0-9_]+)\s*\(", text))


def test_headers_declare_the_boundary():
    hip = declared("ts_hip.h")
    # the replacements of the reference FFI block (train-station/src/cuda/mod.rs:139-208)
    for name in ("ts_hip_initialize", "ts_hip_cleanup", "ts_hip_get_device_count",
                 "ts_hip_set_device", "ts_hip_get_device", "ts_hip_malloc", "ts_hip_free",
                 "ts_hip_memcpy", "ts_hip_memcpy_async", "ts_hip_stream_create",
                 "ts_hip_stream_destroy", "ts_hip_add", "ts_hip_sub", "ts_hip_mul", "ts_hip_matmul",
                 "ts_hip_gemm", "ts_hip_adam_step", "ts_hip_sum_dim0", "ts_hip_relu_backward"):
        assert name in hip, name


def test_libraries_export_every_declared_symbol():
    for lib, header in (("libts_hip.so", "ts_hip.h"), ("libts_gradtrack.so", "ts_gradtrack.h")):
        dll = ctypes.CDLL(str(PKG / lib))
        missing = [n for n in sorted(declared(header)) if not hasattr(dll, n)]
        assert not missing, (lib, missing)


def test_python_bindings_cover_the_headers():
    import train_station_amd._ffi as ffi

    assert set(ffi.HIP_SIGNATURES) == declared("ts_hip.h")
    assert set(ffi.GRADTRACK_SIGNATURES) == declared("ts_gradtrack.h")


def test_error_strings_without_a_device():
    import train_station_amd._ffi as ffi

    assert ffi.hip.ts_hip_error_string(0) == b"success"
    assert b"invalid argument" in ffi.hip.ts_hip_error_string(100001)
    assert b"workspace" in ffi.hip.ts_hip_error_string(100003)


def test_workspace_queries_are_host_only():
    import train_station_amd._ffi as ffi

    assert ffi.hip.ts_hip_sum_workspace_floats(1 << 26) >= 2
    assert ffi.hip.ts_hip_sum_dim0_workspace_floats(8192, 4096) >= 2 * 4096
