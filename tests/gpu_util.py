"""Device buffers for the GPU tests, through the C-ABI of include/ts_hip.h only."""
from __future__ import annotations

import ctypes

import numpy as np

import train_station_amd as T
from train_station_amd._ffi import F, hip, hip_check

_initialised = False


def init() -> None:
    global _initialised
    if not _initialised:
        hip_check(hip.ts_hip_initialize(), "ts_hip_initialize")
        _initialised = True


class Dev:
    """A device buffer of n floats (optionally offset by `offset` floats to
    exercise unaligned pointers)."""

    def __init__(self, n: int, offset: int = 0):
        init()
        self.n = int(n)
        self.offset = offset
        self._base = F()
        hip_check(hip.ts_hip_malloc(ctypes.byref(self._base), self.n + offset + 4), "ts_hip_malloc")

    @property
    def ptr(self) -> int:
        return ctypes.cast(self._base, ctypes.c_void_p).value + 4 * self.offset

    @staticmethod
    def of(arr, offset: int = 0) -> "Dev":
        a = np.ascontiguousarray(arr, dtype=np.float32)
        d = Dev(a.size, offset)
        d.put(a)
        return d

    def put(self, arr) -> None:
        a = np.ascontiguousarray(arr, dtype=np.float32)
        assert a.size == self.n
        if a.size:
            hip_check(hip.ts_hip_memcpy(self.ptr, a.ctypes.data, a.size, 0), "H2D")

    def get(self, shape=None) -> np.ndarray:
        out = np.empty(self.n, dtype=np.float32)
        if self.n:
            hip_check(hip.ts_hip_device_synchronize(), "sync")
            hip_check(hip.ts_hip_memcpy(out.ctypes.data, self.ptr, self.n, 1), "D2H")
        return out.reshape(shape) if shape is not None else out

    def __del__(self):
        try:
            hip.ts_hip_free(self._base)
        except Exception:
            pass


class ZeroIndex:
    """Device uint64 for the division-by-zero report, initialised to UINT64_MAX."""

    def __init__(self):
        self.d = Dev(2)
        self.reset()

    def reset(self):
        self.d.put(np.frombuffer(np.uint64(np.iinfo(np.uint64).max).tobytes(), dtype=np.float32))

    @property
    def ptr(self) -> int:
        return self.d.ptr

    def value(self):
        raw = self.d.get().tobytes()
        v = int(np.frombuffer(raw, dtype=np.uint64)[0])
        return None if v == np.iinfo(np.uint64).max else v


def sync() -> None:
    hip_check(hip.ts_hip_device_synchronize(), "sync")


__all__ = ["Dev", "ZeroIndex", "hip", "hip_check", "init", "sync", "T"]
