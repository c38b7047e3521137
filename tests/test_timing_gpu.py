"""Kernel-attached timing (ts_hip_timing_begin/end) and the host profiler
built on it: the events ride in the kernels' own dispatches, so a window spans
exactly the kernels launched inside it."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import normal

pytestmark = pytest.mark.gpu


def _events(n):
    from gpu_util import hip, hip_check

    evs = []
    for _ in range(n):
        e = ctypes.c_void_p()
        hip_check(hip.ts_hip_event_create(ctypes.byref(e)), "ts_hip_event_create")
        evs.append(e)
    return evs


def _elapsed(a, b):
    from gpu_util import hip, hip_check

    ms = ctypes.c_float()
    hip_check(hip.ts_hip_event_elapsed_ms(ctypes.byref(ms), a, b), "ts_hip_event_elapsed_ms")
    return ms.value


def test_window_counts_and_spans_its_kernels():
    from gpu_util import Dev, hip, hip_check, init, sync

    init()
    M = N = K = 2048
    a, b = Dev.of(normal((M, K), 1)), Dev.of(normal((K, N), 2))
    c = Dev(M * N)
    r0, k0, k1, r1 = _events(4)
    n = ctypes.c_int(-1)
    # nothing launched: no kernel stamped
    hip_check(hip.ts_hip_timing_begin(k0, k1), "ts_hip_timing_begin")
    hip_check(hip.ts_hip_timing_end(ctypes.byref(n)), "ts_hip_timing_end")
    assert n.value == 0
    # end without begin: no window, 0 kernels
    hip_check(hip.ts_hip_timing_end(ctypes.byref(n)), "ts_hip_timing_end")
    assert n.value == 0
    assert hip.ts_hip_timing_begin(None, k1) != 0
    # warm-up: the first launch of a kernel also loads its code
    hip_check(hip.ts_hip_gemm(0, 0, M, N, K, a.ptr, K, b.ptr, N, c.ptr, N, None), "ts_hip_gemm")
    sync()
    for rep in range(3):
        print(f"[timing] rep {rep}: two products of {M}x{N}x{K} in one window", flush=True)
        hip_check(hip.ts_hip_event_record(r0, None), "ts_hip_event_record")
        hip_check(hip.ts_hip_timing_begin(k0, k1), "ts_hip_timing_begin")
        for _ in range(2):
            hip_check(hip.ts_hip_gemm(0, 0, M, N, K, a.ptr, K, b.ptr, N, c.ptr, N, None), "ts_hip_gemm")
        hip_check(hip.ts_hip_timing_end(ctypes.byref(n)), "ts_hip_timing_end")
        hip_check(hip.ts_hip_event_record(r1, None), "ts_hip_event_record")
        sync()
        assert n.value == 2
        kern, outer = _elapsed(k0, k1), _elapsed(r0, r1)
        print(f"[timing] kernels {kern * 1e3:.1f} us, recorded around them {outer * 1e3:.1f} us", flush=True)
        # the window starts at the first kernel and ends with the last: inside
        # the recorded pair, and most of it for two ~0.1 ms products
        assert 0.0 < kern <= outer + 1e-3
        assert kern >= 0.5 * outer
    # launches after the window are plain again
    hip_check(hip.ts_hip_gemm(0, 0, M, N, K, a.ptr, K, b.ptr, N, c.ptr, N, None), "ts_hip_gemm")
    sync()
    got = c.get((M, N))
    assert np.isfinite(got).all()


def test_profiler_times_a_product_and_nested_deferred_work():
    import train_station_amd as T

    x = T.Tensor.from_slice(normal((512, 256), 3), (512, 256))
    w = T.Tensor.from_slice(normal((256, 384), 4), (256, 384)).with_requires_grad()
    T.Profile.reset()
    T.Profile.enable(True)
    y = x.matmul(w).relu()
    s = y.sum()
    T.Profile.enable(False)
    g = T.Profile.read(T.Profile.GEMM)
    assert g["launches"] == 1 and g["ms"] > 0.0
    assert g["work"] == 2.0 * 512 * 384 * 256
    assert s.value() == pytest.approx(float(np.maximum(normal((512, 256), 3) @ normal((256, 384), 4), 0).sum()),
                                      rel=1e-4)
    T.Profile.reset()
