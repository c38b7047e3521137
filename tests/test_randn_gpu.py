"""Device randn (ts_hip_randn / Tensor::randn) against the oracle.

The reference takes ln and cos from the host libm (glibc 2.35's logf /
cosf); the device restates those evaluations, so it must equal the oracle's
host-libm mode (and its restated mode) bit for bit at every size, seed and
alignment.  The 2^28-element case draws every one of the 2^23 possible u1
and u2 values with overwhelming probability, so it checks the device's ln
and cos on their whole input domain.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import assert_bits_equal

pytestmark = pytest.mark.gpu

SEEDS = [0, 1, 42, 12345, 0xFFFFFFFFFFFFFFFF, 0x9E3779B97F4A7C15]
SIZES = [1, 3, 4, 5, 63, 64, 65, 1000, 4096 + 7, 100_480, (1 << 20) + 13]


def _device_randn(n, seed, offset=0):
    from gpu_util import Dev, sync
    from train_station_amd._ffi import hip, hip_check

    d = Dev(n, offset)
    hip_check(hip.ts_hip_randn(d.ptr, n, ctypes.c_uint64(seed), None), "ts_hip_randn")
    sync()
    return d.get()


@pytest.mark.parametrize("n", SIZES)
def test_randn_bit_exact(oracle, n):
    for seed in SEEDS:
        print(f"randn n={n} seed={seed:#x}", flush=True)
        got = _device_randn(n, seed)
        assert_bits_equal(got, oracle.randn(n, seed), f"randn n={n} seed={seed} (host libm)")
        assert_bits_equal(got, oracle.randn(n, seed, restated=True), f"randn n={n} seed={seed} (restated)")


@pytest.mark.parametrize("offset", [1, 2, 3])
def test_randn_unaligned_output(oracle, offset):
    n = 10_001
    assert_bits_equal(_device_randn(n, 42, offset), oracle.randn(n, 42))


def test_randn_zero_size_is_noop():
    from train_station_amd._ffi import hip

    assert hip.ts_hip_randn(None, 0, ctypes.c_uint64(1), None) == 0
    assert hip.ts_hip_randn(None, 5, ctypes.c_uint64(1), None) != 0  # NULL output is rejected


def test_randn_prefix_across_run_lengths(oracle):
    # thread run lengths change with n; the stream must not
    big = _device_randn(1 << 24, 7)
    for n in (1 << 12, 1 << 18, (1 << 20) + 1, (1 << 22) - 3):
        assert_bits_equal(_device_randn(n, 7), big[:n], f"prefix {n}")


def test_randn_full_domain_and_host_libm(oracle):
    n = 1 << 28
    seed = 20260101
    print(f"randn n={n}", flush=True)
    got = _device_randn(n, seed)
    assert_bits_equal(got, oracle.randn(n, seed), "randn 2^28 (host logf / cosf, as the reference)")


def test_tensor_randn_api(oracle):
    import train_station_amd as T

    t = T.Tensor.randn([2, 3], seed=42)
    assert t.shape == (2, 3)
    assert_bits_equal(t.data(), oracle.randn(6, 42).reshape(2, 3))
    e = T.Tensor.randn([0], seed=42)
    assert e.size() == 0 and e.shape == (0,)
    # without a seed: clock-seeded, not all zeros, different per call
    a, b = T.Tensor.randn([10]).data(), T.Tensor.randn([10]).data()
    assert np.any(a != 0.0) and np.any(a != b)
    f = T.Tensor.zeros([4, 5])
    f.fill_randn(seed=9)
    assert_bits_equal(f.data(), oracle.randn(20, 9).reshape(4, 5))
    # the reference's own tests, random.rs:622-750, on the device values
    big = T.Tensor.randn([100, 100], seed=42).data()
    assert abs(float(big.mean())) < 0.1 and big.min() > -4.0 and big.max() < 4.0
