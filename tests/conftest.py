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
