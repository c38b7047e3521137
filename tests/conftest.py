"""Shared test setup.

Markers: ``gpu`` -- needs an MI355X (run with ``-m gpu``); everything else runs
on the CPU.  The oracle (``oracle/``) is the checker for both.
"""
from __future__ import annotations

import json
import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (gfx950)")


def golden(name: str) -> dict:
    return json.loads((GOLDEN / name).read_text())


@pytest.fixture(scope="session")
def oracle():
    import oracle as O

    O.lib()
    return O


def rng(seed: int = 0) -> np.random.Generator:
    return np.random.default_rng(seed)


def normal(shape, seed=0, scale=1.0) -> np.ndarray:
    return (rng(seed).standard_normal(shape) * scale).astype(np.float32)


def uniform(shape, lo, hi, seed=0) -> np.ndarray:
    return rng(seed).uniform(lo, hi, shape).astype(np.float32)


def bits(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_bits_equal(got, want, what=""):
    """Bit-for-bit equality, except that any two NaNs match: IEEE 754 leaves
    the sign and payload of a generated NaN to the implementation (x86 SSE/AVX
    produce 0xFFC00000 for inf - inf, gfx950 produces 0x7FC00000)."""
    g, w = bits(got), bits(want)
    assert g.shape == w.shape, (what, g.shape, w.shape)
    both_nan = np.isnan(np.asarray(got, np.float32)) & np.isnan(np.asarray(want, np.float32))
    bad = np.flatnonzero((g != w).reshape(-1) & ~both_nan.reshape(-1))
    assert bad.size == 0, (
        f"{what}: {bad.size} of {g.size} elements differ in bits; first at {bad[0]}: "
        f"got {np.asarray(got).reshape(-1)[bad[0]]!r} want {np.asarray(want).reshape(-1)[bad[0]]!r}")


def max_rel(got, want) -> float:
    """Normwise max relative error: max|got - want| / max|want|."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    den = max(np.max(np.abs(want)), 1e-30)
    return float(np.max(np.abs(got - want)) / den)


def rel_l2(got, want) -> float:
    """Normwise L2 relative error ||got - want||_2 / ||want||_2.  Used for
    parameters after many optimizer steps: a ReLU pre-activation within GEMM
    rounding of zero can flip its mask in one of two correct GEMMs, moving a
    single element by about one Adam step (~lr), which a max-norm measure
    would report as the whole tensor's error."""
    got = np.asarray(got, dtype=np.float64).reshape(-1)
    want = np.asarray(want, dtype=np.float64).reshape(-1)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def sum_order_model(values, mean=False, aligned=True, times=None) -> np.float32:
    """The fp32 result of ts_hip_sum / ts_hip_mean (and of a fused sum in
    ts_hip_map) over `values`, in the partition's order, restated in numpy:
    R float4 groups per thread (1 while ceil(n / 1024) <= 2048, else
    max(4, ceil(n / 2^26))) and ceil(n / (1024 R)) first-pass workgroups of
    256 threads; thread t of workgroup b adds, in f64 from +0, the groups
    g = 256 R b + t + 256 j, j = 0 .. R - 1 (those below n4), each as
    ((x0 + x1) + x2) + x3 (no groups when the input is not 16-byte aligned),
    then the elements 4 * n4 + T, T + 256 * blocks, ... past the groups
    (T = 256 b + t); a workgroup's sum is the
    xor butterfly over each wave's 64 lanes, the four wave sums added from +0;
    the second pass's thread t adds partials t, t + 256, ... from +0, then the
    same workgroup sum; one rounding to fp32 (divided by (float)n for the
    mean).  With `times`, the sum of products x[i] * times[i] (ts_hip_dot),
    each product formed in f64 (exact).  Whatever kernels run, the bits are
    these."""
    x = np.asarray(values, np.float32).astype(np.float64)
    if times is not None:
        x = x * np.asarray(times, np.float32).astype(np.float64)
    n = x.size
    if n == 0:
        return np.float32(0.0)
    run = 1 if (n + 1023) // 1024 <= 2048 else max(4, -(-n // (1024 * 65536)))
    blocks = max(-(-n // (1024 * run)), 1)
    threads = blocks * 256
    n4 = n // 4 if aligned else 0
    q = x[: 4 * n4].reshape(n4, 4)
    quad = np.zeros(threads * run)  # padded with +0: adding it to an f64 sum from +0 changes nothing
    quad[:n4] = ((q[:, 0] + q[:, 1]) + q[:, 2]) + q[:, 3]
    runs = quad.reshape(blocks, run, 256)
    acc = np.zeros((blocks, 256))
    for j in range(run):
        acc += runs[:, j, :]
    acc = acc.reshape(threads)
    for i0 in range(4 * n4, n, threads):
        part = x[i0: i0 + threads]
        acc[: part.size] += part

    def workgroup_sums(v):  # v: [workgroups, 256]
        w = v.reshape(v.shape[0], 4, 64).copy()
        for off in (32, 16, 8, 4, 2, 1):
            w = w + w[:, :, np.arange(64) ^ off]
        r = np.zeros(v.shape[0])
        for k in range(4):
            r = r + w[:, k, 0]
        return r

    partial = workgroup_sums(acc.reshape(blocks, 256))
    acc2 = np.zeros(256)
    for i0 in range(0, blocks, 256):
        part = partial[i0: i0 + 256]
        acc2[: part.size] += part
    s = np.float32(workgroup_sums(acc2.reshape(1, 256))[0])
    return np.float32(s / np.float32(n)) if mean else s
