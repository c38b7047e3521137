"""CPU oracle for train-station's gradtrack training step.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import this package, and only as
the checker or as the reported CPU baseline.  The product path
(``train-station_amd/``) never imports, links or calls it.

``libts_oracle.so`` (built from ``ts_oracle.c`` by ``make -C oracle``) holds
the fp32 arithmetic restated from the reference in its operation order;
``gradtrack.py`` restates the reference's graph recording, LIFO backward
worklist and Adam on top of it.  Arrays are numpy float32, C-contiguous.
"""
from __future__ import annotations

import ctypes
import os
import pathlib

import numpy as np

_HERE = pathlib.Path(__file__).resolve().parent
_LIB: ctypes.CDLL | None = None

_F = ctypes.POINTER(ctypes.c_float)
_D = ctypes.POINTER(ctypes.c_double)
_SZ = ctypes.c_size_t


def lib() -> ctypes.CDLL:
    """Load libts_oracle.so (built by ``make -C oracle``)."""
    global _LIB
    if _LIB is None:
        path = _HERE / "libts_oracle.so"
        if not path.exists():
            raise RuntimeError(f"{path} is missing: run `make -C oracle` (or __graft_entry__.build())")
        L = ctypes.CDLL(str(path))
        for name in ("o_add", "o_sub", "o_mul"):
            getattr(L, name).argtypes = [_F, _F, _F, _SZ]
        L.o_div.argtypes = [_F, _F, _F, _SZ]
        L.o_div.restype = ctypes.c_longlong
        for name in ("o_add_scalar", "o_sub_scalar", "o_mul_scalar", "o_div_scalar"):
            getattr(L, name).argtypes = [_F, ctypes.c_float, _F, _SZ]
        L.o_neg.argtypes = [_F, _F, _SZ]
        L.o_relu.argtypes = [_F, _F, _SZ]
        L.o_pow2.argtypes = [_F, _F, _SZ]
        L.o_bias_add.argtypes = [_F, _F, _F, _SZ, _SZ, ctypes.c_int]
        L.o_fill.argtypes = [_F, ctypes.c_float, _SZ]
        L.o_relu_bwd.argtypes = [_F, _F, _F, _SZ]
        L.o_pow_bwd.argtypes = [_F, _F, _F, _SZ, ctypes.c_float]
        L.o_sum.argtypes = [_F, _SZ]
        L.o_sum.restype = ctypes.c_float
        L.o_mean.argtypes = [_F, _SZ]
        L.o_mean.restype = ctypes.c_float
        L.o_sum_f64.argtypes = [_F, _SZ]
        L.o_sum_f64.restype = ctypes.c_double
        L.o_sum_dim0.argtypes = [_F, _SZ, _SZ, _F]
        L.o_sum_dim0_f64.argtypes = [_F, _SZ, _SZ, _D]
        L.o_gemm_f64.argtypes = [ctypes.c_int, ctypes.c_int, _SZ, _SZ, _SZ, _F, _SZ, _F, _SZ, _D]
        L.o_gemm_f32.argtypes = [ctypes.c_int, ctypes.c_int, _SZ, _SZ, _SZ, _F, _SZ, _F, _SZ, _F, _F, _F]
        L.o_adam_correction_factor.argtypes = [ctypes.c_float, ctypes.c_uint64]
        L.o_adam_correction_factor.restype = ctypes.c_float
        L.o_adam_step.argtypes = [_F, _F, _F, _F, _F, _SZ, ctypes.c_float, ctypes.c_float,
                                  ctypes.c_float, ctypes.c_float, ctypes.c_float, ctypes.c_uint64,
                                  ctypes.c_int]
        L.o_randn.argtypes = [_F, _SZ, ctypes.c_uint64, ctypes.c_int]
        L.o_unary.argtypes = [ctypes.c_int, _F, _F, _SZ, ctypes.c_float, ctypes.c_int]
        L.o_unary_bwd.argtypes = [ctypes.c_int, _F, _F, _F, _SZ, ctypes.c_float]
        L.o_softmax.argtypes = [_F, _F, _SZ, _SZ, _SZ, ctypes.c_int]
        L.o_softmax_bwd.argtypes = [_F, _F, _F, _SZ, _SZ, _SZ]
        L.o_sum_dims.argtypes = [_F, ctypes.POINTER(_SZ), _SZ, ctypes.c_uint, _F, _D]
        for name in ("o_unary_cr_check", "o_unary_glibc_diff"):
            getattr(L, name).argtypes = [ctypes.c_int, ctypes.c_uint]
            getattr(L, name).restype = ctypes.c_long
        L.o_xorshift_next.argtypes = [ctypes.c_uint64]
        L.o_xorshift_next.restype = ctypes.c_uint64
        L.o_xorshift_advance.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
        L.o_xorshift_advance.restype = ctypes.c_uint64
        L.o_libm_cr_check.argtypes = [ctypes.c_int]
        L.o_libm_cr_check.restype = ctypes.c_long
        L.o_libm_glibc_diff.argtypes = [ctypes.c_int]
        L.o_libm_glibc_diff.restype = ctypes.c_long
        L.o_glibc_restated_diff.argtypes = [ctypes.c_int, ctypes.c_uint, ctypes.c_uint]
        L.o_glibc_restated_diff.restype = ctypes.c_long
        _LIB = L
    return _LIB


def _f32(x) -> np.ndarray:
    a = np.ascontiguousarray(x, dtype=np.float32)
    return a


def _p(a: np.ndarray):
    return a.ctypes.data_as(_F)


def _binary(name: str, a, b) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    assert a.shape == b.shape, (a.shape, b.shape)
    out = np.empty_like(a)
    getattr(lib(), name)(_p(a), _p(b), _p(out), a.size)
    return out


def add(a, b):
    return _binary("o_add", a, b)


def sub(a, b):
    return _binary("o_sub", a, b)


def mul(a, b):
    return _binary("o_mul", a, b)


class DivisionByZero(ArithmeticError):
    """Raised where the reference panics on a zero divisor (ops/div.rs:378-417)."""


def div(a, b):
    a, b = _f32(a), _f32(b)
    assert a.shape == b.shape
    out = np.empty_like(a)
    idx = lib().o_div(_p(a), _p(b), _p(out), a.size)
    if idx >= 0:
        raise DivisionByZero(f"Division by zero detected at index {idx}")
    return out


def _scalar(name, x, s):
    x = _f32(x)
    out = np.empty_like(x)
    getattr(lib(), name)(_p(x), ctypes.c_float(s), _p(out), x.size)
    return out


def add_scalar(x, s):
    return _scalar("o_add_scalar", x, s)


def sub_scalar(x, s):
    return _scalar("o_sub_scalar", x, s)


def mul_scalar(x, s):
    return _scalar("o_mul_scalar", x, s)


def div_scalar(x, s):
    if np.float32(s) == 0:
        raise DivisionByZero("Division by zero: cannot divide tensor by zero scalar")
    return _scalar("o_div_scalar", x, s)


def _unary(name, x):
    x = _f32(x)
    out = np.empty_like(x)
    getattr(lib(), name)(_p(x), _p(out), x.size)
    return out


def neg(x):
    return _unary("o_neg", x)


def relu(x):
    return _unary("o_relu", x)


def pow2(x):
    return _unary("o_pow2", x)


def bias_add(x, bias, bias_first=False):
    x, bias = _f32(x), _f32(bias)
    rows, cols = x.shape
    assert bias.shape == (cols,)
    out = np.empty_like(x)
    lib().o_bias_add(_p(x), _p(bias), _p(out), rows, cols, int(bias_first))
    return out


def fill(shape, v):
    out = np.empty(shape, dtype=np.float32)
    lib().o_fill(_p(out), ctypes.c_float(v), out.size)
    return out


def relu_bwd(x, go):
    x, go = _f32(x), _f32(go)
    gi = np.empty_like(x)
    lib().o_relu_bwd(_p(x), _p(go), _p(gi), x.size)
    return gi


def pow_bwd(x, go, exponent):
    x, go = _f32(x), _f32(go)
    gi = np.empty_like(x)
    lib().o_pow_bwd(_p(x), _p(go), _p(gi), x.size, ctypes.c_float(exponent))
    return gi


def sum_(x) -> np.float32:
    x = _f32(x)
    return np.float32(lib().o_sum(_p(x), x.size))


def mean(x) -> np.float32:
    x = _f32(x)
    return np.float32(lib().o_mean(_p(x), x.size))


def sum_f64(x) -> float:
    x = _f32(x)
    return float(lib().o_sum_f64(_p(x), x.size))


def sum_dim0(x):
    x = _f32(x)
    rows, cols = x.shape
    out = np.empty(cols, dtype=np.float32)
    lib().o_sum_dim0(_p(x), rows, cols, _p(out))
    return out


def sum_dim0_f64(x):
    x = _f32(x)
    rows, cols = x.shape
    out = np.empty(cols, dtype=np.float64)
    lib().o_sum_dim0_f64(_p(x), rows, cols, out.ctypes.data_as(_D))
    return out


# The device's column-sum order (ts_hip_sum_dim0, and the bias gradient the
# weight-gradient product writes alongside it): chunks of 64 rows, each added
# row by row; groups of 8 consecutive chunk sums added in chunk order; the
# group sums added in group order -- every sum in f64 from +0 -- and one
# rounding to fp32.  Its bits are the device's; the value is the reference's
# sum_dims(&[0]) (reductions/sum.rs:225-306) to within the f64 rounding of the
# partials, far inside the 1e-4 the reference's own fp32 row order allows.
COLSUM_ROWS = 64
COLSUM_GROUP = 8


def sum_dim0_chunked(x, weights=None):
    """Column sums (weights: row r scaled by weights[r] in f64, the transposed
    matrix-vector product) in the device's fixed order; fp32 result."""
    x = _f32(x)
    rows, cols = x.shape
    w = None if weights is None else np.asarray(weights, dtype=np.float32).astype(np.float64)
    chunks = []
    for c0 in range(0, rows, COLSUM_ROWS):
        s = np.zeros(cols, dtype=np.float64)
        for r in range(c0, min(c0 + COLSUM_ROWS, rows)):
            row = x[r].astype(np.float64)
            s = s + (row if w is None else w[r] * row)
        chunks.append(s)
    total = np.zeros(cols, dtype=np.float64)
    for g0 in range(0, len(chunks), COLSUM_GROUP):
        g = np.zeros(cols, dtype=np.float64)
        for s in chunks[g0:g0 + COLSUM_GROUP]:
            g = g + s
        total = total + g
    return total.astype(np.float32)


# Products of at least this many multiply-adds take numpy's float64 matmul
# (multi-threaded BLAS) instead of the C triple loop: both accumulate exactly
# representable f32 products in f64, differing only in f64 summation order
# (pinned against each other in tests/test_oracle.py).  Many-step training
# comparisons at the configuration shapes need the speed.
GEMM_F64_BLAS_MIN_MACS = 1 << 22


def gemm_f64(a, b, ta=False, tb=False, path: str = "auto") -> np.ndarray:
    """op(a) @ op(b) with f64 accumulation; op transposes a [K,M] / b [N,K] view.
    ``path``: "loop" (C), "blas" (numpy float64 matmul) or "auto" (by size)."""
    a, b = _f32(a), _f32(b)
    M = a.shape[1] if ta else a.shape[0]
    K = a.shape[0] if ta else a.shape[1]
    N = b.shape[0] if tb else b.shape[1]
    Kb = b.shape[1] if tb else b.shape[0]
    assert K == Kb, (a.shape, b.shape, ta, tb)
    if path == "blas" or (path == "auto" and M * N * K >= GEMM_F64_BLAS_MIN_MACS):
        a64 = a.astype(np.float64)
        b64 = b.astype(np.float64)
        return np.ascontiguousarray((a64.T if ta else a64) @ (b64.T if tb else b64))
    out = np.empty((M, N), dtype=np.float64)
    lib().o_gemm_f64(int(ta), int(tb), M, N, K, _p(a), a.shape[1], _p(b), b.shape[1],
                     out.ctypes.data_as(_D))
    return out


def gemm_f32(a, b, ta=False, tb=False) -> np.ndarray:
    """op(a) @ op(b) in fp32 with the reference's sequential-k FMA order."""
    a, b = _f32(a), _f32(b)
    M = a.shape[1] if ta else a.shape[0]
    K = a.shape[0] if ta else a.shape[1]
    N = b.shape[0] if tb else b.shape[1]
    out = np.empty((M, N), dtype=np.float32)
    sa = np.empty(M * K if ta else 1, dtype=np.float32)
    sb = np.empty(K * N if tb else 1, dtype=np.float32)
    lib().o_gemm_f32(int(ta), int(tb), M, N, K, _p(a), a.shape[1], _p(b), b.shape[1],
                     _p(out), _p(sa), _p(sb))
    return out


def adam_correction_factor(beta: float, step_count: int) -> np.float32:
    return np.float32(lib().o_adam_correction_factor(ctypes.c_float(beta), step_count))


def adam_step(p, g, m, v, step_count, lr=1e-3, b1=0.9, b2=0.999, eps=1e-8, weight_decay=0.0,
              vmax=None, amsgrad_first=False):
    """In-place Adam update of float32 arrays p, m, v (and vmax under AMSGrad)."""
    for arr in (p, g, m, v) + ((vmax,) if vmax is not None else ()):
        assert arr.dtype == np.float32 and arr.flags.c_contiguous
    lib().o_adam_step(_p(p), _p(g), _p(m), _p(v), _p(vmax) if vmax is not None else None, p.size,
                      ctypes.c_float(lr), ctypes.c_float(b1), ctypes.c_float(b2),
                      ctypes.c_float(eps), ctypes.c_float(weight_decay), step_count,
                      int(amsgrad_first))


def build() -> None:
    """Compile libts_oracle.so in place."""
    import subprocess
    subprocess.run(["make", "-B", "-C", str(_HERE)], check=True,
                   stdout=subprocess.DEVNULL if not os.environ.get("TS_VERBOSE") else None)


def _libm_mode(correctly_rounded: bool, restated: bool) -> int:
    """0: the host libm, as the reference; 1: f64 rounded once; 2: glibc 2.35's
    evaluation restated in ts_oracle.c (the host libm's bits on this image)."""
    return 1 if correctly_rounded else (2 if restated else 0)


def randn(n: int, seed: int, correctly_rounded: bool = False, restated: bool = False) -> np.ndarray:
    """Tensor::randn(n, Some(seed)) values.  ``correctly_rounded`` evaluates ln
    and cos in f64 and rounds once; ``restated`` takes glibc 2.35's logf / cosf
    restated; otherwise the host libm's logf / cosf."""
    out = np.empty(n, dtype=np.float32)
    lib().o_randn(_p(out), n, ctypes.c_uint64(seed), _libm_mode(correctly_rounded, restated))
    return out


GLIBC_RESTATED = {"exp": 0, "log": 1, "tanh": 2, "cos": 3, "expm1": 4}


def glibc_restated_diff(fn: str, stride: int, offset: int = 0) -> int:
    """Inputs (f32 bit patterns offset + k * stride; cos below 120 only) where
    ts_oracle.c's restatement of glibc 2.35's expf / logf / tanhf / cosf /
    expm1f differs from the host libm's."""
    return int(lib().o_glibc_restated_diff(GLIBC_RESTATED[fn], stride, offset))


def xorshift_next(s: int) -> int:
    return int(lib().o_xorshift_next(ctypes.c_uint64(s)))


def xorshift_advance(s: int, k: int) -> int:
    return int(lib().o_xorshift_advance(ctypes.c_uint64(s), ctypes.c_uint64(k)))


def libm_cr_check(which: int) -> int:
    """Inputs (of 2^23) where f64-rounded ln (0) / cos (1) disagrees with long double."""
    return int(lib().o_libm_cr_check(which))


def libm_glibc_diff(which: int) -> int:
    """Inputs (of 2^23) where the host's logf (0) / cosf (1) differ from the
    correctly rounded value."""
    return int(lib().o_libm_glibc_diff(which))


UNARY = {"exp": 0, "log": 1, "sqrt": 2, "tanh": 3, "sigmoid": 4, "leaky_relu": 5}


def unary(op: str, x, slope: float = 0.0, correctly_rounded: bool = False, restated: bool = False) -> np.ndarray:
    """tensor/ops/{exp,log,sqrt,tanh,sigmoid,leaky_relu}.rs forward.  exp / ln /
    tanh come from the host libm unless ``correctly_rounded`` (f64 rounded
    once) or ``restated`` (glibc 2.35's evaluation restated)."""
    x = _f32(x)
    out = np.empty_like(x)
    lib().o_unary(UNARY[op], _p(x), _p(out), x.size, ctypes.c_float(slope), _libm_mode(correctly_rounded, restated))
    return out


def unary_bwd(op: str, saved, go, slope: float = 0.0) -> np.ndarray:
    """grad_fn/ops/{exp,log,sqrt,tanh,sigmoid,leaky_relu}.rs; saved = output for
    exp / sqrt / tanh / sigmoid, input for log / leaky_relu."""
    saved, go = _f32(saved), _f32(go)
    gi = np.empty_like(go)
    lib().o_unary_bwd(UNARY[op], _p(saved), _p(go), _p(gi), go.size, ctypes.c_float(slope))
    return gi


def _axis_view(shape, dim):
    outer = int(np.prod(shape[:dim], dtype=np.int64))
    inner = int(np.prod(shape[dim + 1:], dtype=np.int64))
    return outer, int(shape[dim]), inner


def softmax(x, dim: int, correctly_rounded: bool = False, restated: bool = False) -> np.ndarray:
    x = _f32(x)
    y = np.empty_like(x)
    outer, red, inner = _axis_view(x.shape, dim)
    lib().o_softmax(_p(x), _p(y), outer, red, inner, _libm_mode(correctly_rounded, restated))
    return y


def softmax_bwd(y, go, dim: int) -> np.ndarray:
    y, go = _f32(y), _f32(go)
    gi = np.empty_like(go)
    outer, red, inner = _axis_view(y.shape, dim)
    lib().o_softmax_bwd(_p(y), _p(go), _p(gi), outer, red, inner)
    return gi


def sum_dims_shape(shape, dims, keepdim: bool) -> list:
    """reductions/sum.rs:237-252 (every zero-size axis is dropped when not keepdim)"""
    out = list(shape)
    for d in sorted(set(dims)):
        out[d] = 1 if keepdim else 0
    if not keepdim:
        out = [v for v in out if v != 0]
    return out or [1]


def sum_dims(x, dims, keepdim: bool = False, f64: bool = False) -> np.ndarray:
    """sum_dims (reductions/sum.rs:225-306): fp32 accumulation in input order
    (or the same sums in f64)."""
    x = _f32(x)
    reduced = sorted(set(dims))
    out_shape = sum_dims_shape(x.shape, dims, keepdim)
    if x.size == 0:
        return np.zeros(out_shape, np.float64 if f64 else np.float32)
    mask = 0
    for d in reduced:
        mask |= 1 << d
    kd = [1 if k in reduced else v for k, v in enumerate(x.shape)]
    out = np.empty(int(np.prod(kd, dtype=np.int64)), np.float32)
    out64 = np.empty(out.size, np.float64)
    dims_arr = (_SZ * max(x.ndim, 1))(*x.shape)
    lib().o_sum_dims(_p(x), dims_arr, x.ndim, mask, _p(out), out64.ctypes.data_as(_D))
    return (out64 if f64 else out).reshape(out_shape)


def unary_cr_check(op: str, stride: int) -> int:
    return int(lib().o_unary_cr_check(UNARY[op], stride))


def unary_glibc_diff(op: str, stride: int) -> int:
    return int(lib().o_unary_glibc_diff(UNARY[op], stride))
