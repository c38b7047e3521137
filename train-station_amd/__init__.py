"""train-station's gradtrack training step on AMD Instinct MI355X (gfx950).

Layers, bottom up:

* ``libts_hip.so`` -- hand-written HIP kernels for gfx950 behind the C-ABI of
  ``include/ts_hip.h``: fp32-MFMA GEMMs (forward and both backward
  contractions), bit-exact elementwise and ReLU-mask kernels, deterministic
  wave/LDS reductions, one fused Adam kernel, device randn, checkpoint
  record encoding, plus malloc / async copy / stream / event wrappers.
* ``libts_gradtrack.so`` -- the reference's Tensor / gradtrack engine / Adam
  restated in C++ over that C-ABI (``include/ts_gradtrack.h``).
* this package -- a ctypes face of the same API for Python callers.

Importing the package loads both libraries; it raises if they are not built.
"""
from ._ffi import TsError, gradtrack as native_gradtrack, hip as native_hip, hip_check
from .tensor import (Adam, NoGradTrack, Profile, StepGraph, Tensor, adam_config_from_binary,
                     adam_config_from_json, adam_config_to_binary, adam_config_to_json,
                     clear_gradients, empty_cache, fusion_enabled, is_grad_enabled, pool_stats, recording,
                     set_fusion, set_grad_enabled, stream, synchronize, with_no_grad)

__all__ = [
    "Adam", "NoGradTrack", "Profile", "StepGraph", "Tensor", "TsError", "adam_config_from_binary",
    "adam_config_from_json", "adam_config_to_binary", "adam_config_to_json", "clear_gradients",
    "empty_cache", "fusion_enabled",
    "hip_check", "is_grad_enabled", "native_gradtrack", "native_hip", "pool_stats", "recording", "set_fusion",
    "set_grad_enabled", "stream", "synchronize", "with_no_grad",
]
