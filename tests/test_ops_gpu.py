"""Activations, softmax, general broadcasting and axis sums on the device,
through the C-ABI (kernels) and the handle API (recorded ops + backward),
against the oracle.

Bars: bit-exact for every elementwise formula and for softmax, against the
host libm's exp / ln / tanh (what the reference computes: glibc 2.35's expf /
logf / tanhf, whose evaluations the device restates) and against the oracle's
restatement of them; axis sums and reduced gradients within 1e-6 relative of
f64 (the oracle's fp32 chains differ from f64 by their own rounding, bounded
below 1e-4).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import assert_bits_equal, normal

import oracle as O
from oracle import gradtrack as G

pytestmark = pytest.mark.gpu

SIZES = [1, 5, 4096 + 3, (1 << 20) + 7]
SPECIAL = np.array([0.0, -0.0, 1.0, -1.0, 0.5, 88.7, 88.8, -87.3, -103.0, -104.0, 1e-30, -1e-30, 1e-41,
                    20.0, -20.0, 9.0, -9.0, 1e-8, 3.4e38, -3.4e38, np.inf, -np.inf, np.nan], np.float32)


def _x(n, seed, scale=4.0):
    x = normal(n, seed, scale)
    k = min(n, SPECIAL.size)
    x[:k] = SPECIAL[:k]
    return x


def _hip():
    from train_station_amd._ffi import hip, hip_check
    return hip, hip_check


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("op", ["exp", "log", "sqrt", "tanh", "sigmoid", "leaky_relu"])
def test_unary_forward_bit_exact(op, n):
    from gpu_util import Dev, sync
    hip, check = _hip()
    x = _x(n, 1)
    if op in ("log", "sqrt"):
        x = np.abs(x)
    for offset in (0, 1):
        dx, dy = Dev.of(x, offset), Dev(n, offset)
        if op == "leaky_relu":
            check(hip.ts_hip_leaky_relu(dx.ptr, ctypes.c_float(0.01), dy.ptr, n, None))
        else:
            check(getattr(hip, f"ts_hip_{op}")(dx.ptr, dy.ptr, n, None))
        sync()
        got = dy.get()
        assert_bits_equal(got, O.unary(op, x, 0.01), f"{op} n={n} (host libm)")
        assert_bits_equal(got, O.unary(op, x, 0.01, restated=True), f"{op} n={n} (restated)")


@pytest.mark.parametrize("op", ["exp", "log", "tanh", "sigmoid"])
def test_unary_forward_on_a_sweep_of_every_float(op):
    # every 4099th f32 bit pattern (about a million values of every sign,
    # exponent and NaN kind): the device equals the host libm bit for bit
    from gpu_util import Dev, sync
    hip, check = _hip()
    x = (np.arange(0, 1 << 32, 4099, dtype=np.uint64) + 17).astype(np.uint32).view(np.float32)
    n = x.size
    dx, dy = Dev.of(x), Dev(n)
    check(getattr(hip, f"ts_hip_{op}")(dx.ptr, dy.ptr, n, None))
    sync()
    assert_bits_equal(dy.get(), O.unary(op, x), f"{op} sweep")


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("op", ["log", "sqrt", "tanh", "sigmoid", "leaky_relu"])
def test_unary_backward_bit_exact(op, n):
    from gpu_util import Dev, sync
    hip, check = _hip()
    go = normal(n, 2)
    saved = np.abs(_x(n, 3)) + np.float32(0.01) if op in ("log", "sqrt") else np.tanh(normal(n, 4))
    if op == "leaky_relu":
        saved = _x(n, 5)
    ds, dg, dgi = Dev.of(saved), Dev.of(go), Dev(n)
    if op == "leaky_relu":
        check(hip.ts_hip_leaky_relu_backward(ds.ptr, dg.ptr, dgi.ptr, n, ctypes.c_float(0.2), None))
    else:
        check(getattr(hip, f"ts_hip_{op}_backward")(ds.ptr, dg.ptr, dgi.ptr, n, None))
    sync()
    assert_bits_equal(dgi.get(), O.unary_bwd(op, saved, go, 0.2), op)


@pytest.mark.parametrize("shape,dim", [((64, 10), 1), ((7, 33, 5), 1), ((1000,), 0), ((3, 4, 257), 2),
                                       ((2, 3, 4, 5), 0), ((4096, 128), 1)])
def test_softmax_bit_exact(shape, dim):
    from gpu_util import Dev, sync
    hip, check = _hip()
    x = normal(shape, 6, 5.0)
    outer, red, inner = O._axis_view(shape, dim)
    dx, dy = Dev.of(x), Dev(x.size)
    check(hip.ts_hip_softmax(dx.ptr, dy.ptr, outer, red, inner, None))
    sync()
    y = dy.get(shape)
    assert_bits_equal(y, O.softmax(x, dim))
    assert_bits_equal(y, O.softmax(x, dim, restated=True))
    go = normal(shape, 7)
    dgo, dgi = Dev.of(go), Dev(x.size)
    check(hip.ts_hip_softmax_backward(dy.ptr, dgo.ptr, dgi.ptr, outer, red, inner, None))
    sync()
    assert_bits_equal(dgi.get(shape), O.softmax_bwd(y, go, dim))


@pytest.mark.parametrize("src,out", [((6,), (4, 5, 6)), ((5, 1), (5, 7)), ((1,), (3, 3)), ((4, 1, 6), (4, 5, 6)),
                                     ((), (2, 3)), ((3, 1, 1, 2), (2, 3, 4, 5, 2)), ((7, 8), (7, 8))])
def test_broadcast_copy(src, out):
    from gpu_util import Dev, sync
    hip, check = _hip()
    from train_station_amd._ffi import SZ
    x = normal(src if src else (1,), 8)
    dx, dy = Dev.of(x), Dev(int(np.prod(out)))
    sd = (SZ * max(len(src), 1))(*src)
    od = (SZ * len(out))(*out)
    check(hip.ts_hip_broadcast_copy(dx.ptr, sd, len(src), dy.ptr, od, len(out), ctypes.c_float(1.0), 0, None))
    sync()
    want = np.broadcast_to(x.reshape(src), out)
    assert_bits_equal(dy.get(out), np.ascontiguousarray(want))
    check(hip.ts_hip_broadcast_copy(dx.ptr, sd, len(src), dy.ptr, od, len(out), ctypes.c_float(0.25), 1, None))
    sync()
    assert_bits_equal(dy.get(out), np.ascontiguousarray(want) * np.float32(0.25))


@pytest.mark.parametrize("shape,mask", [((8192, 4096), 0b01), ((4096, 8192), 0b10), ((64, 33, 17), 0b101),
                                        ((5, 7, 9), 0b010), ((3, 4, 5, 6), 0b1111), ((1 << 22,), 0b1),
                                        ((257, 3), 0b00)])
def test_reduce_sum(shape, mask):
    from gpu_util import Dev, sync
    hip, check = _hip()
    from train_station_amd._ffi import SZ
    x = normal(shape, 9)
    axes = tuple(k for k in range(len(shape)) if (mask >> k) & 1)
    want = x.astype(np.float64).sum(axis=axes, keepdims=True) if axes else x.astype(np.float64)
    dx, dy = Dev.of(x), Dev(want.size)
    dims = (SZ * len(shape))(*shape)
    check(hip.ts_hip_reduce_sum(dx.ptr, dims, len(shape), mask, dy.ptr, ctypes.c_float(1.0), 0, None))
    sync()
    got = dy.get(want.shape).astype(np.float64)
    assert np.max(np.abs(got - want)) <= 1e-6 * max(1.0, float(np.max(np.abs(want))))
    if not axes:
        assert_bits_equal(dy.get(want.shape), x)


# ---- recorded ops through the handle API ----------------------------------------------

def _T():
    import train_station_amd as T
    return T


@pytest.mark.parametrize("sa,sb", [((4, 5, 6), (6,)), ((4, 1, 6), (5, 6)), ((5, 1), (1, 7)), ((3, 4), (3, 4)),
                                   ((1,), (2, 3)), ((2, 3, 4), (3, 1))])
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
def test_broadcast_binary_ops_and_gradients(op, sa, sb):
    T = _T()
    a = normal(sa, 1)
    b = np.abs(normal(sb, 2)) + np.float32(0.5)
    ta = T.Tensor.from_slice(a, sa).with_requires_grad()
    tb = T.Tensor.from_slice(b, sb).with_requires_grad()
    oa, ob = G.OTensor(a.copy(), True), G.OTensor(b.copy(), True)
    y = getattr(ta, f"{op}_tensor")(tb)
    oy = getattr(oa, f"{op}_tensor")(ob)
    assert_bits_equal(y.data(), oy.data, f"{op} {sa} {sb}")
    go = normal(oy.shape, 3)
    y.backward(T.Tensor.from_slice(go, oy.shape))
    G.backward(oy, go)
    for mine, theirs in ((ta, oa), (tb, ob)):
        g, w = mine.grad_by_value().data(), theirs.grad_by_value()
        assert g.shape == w.shape
        # reduced gradients: the oracle chains fp32 sums, the device sums in f64
        assert np.max(np.abs(g - w)) <= 1e-5 * max(1.0, float(np.max(np.abs(w)))), (op, sa, sb)
        if mine.shape == tuple(oy.shape):
            assert_bits_equal(g, w)
    T.clear_gradients()
    G.clear_gradients()


def test_broadcast_errors_and_division_by_zero():
    T = _T()
    a = T.Tensor.from_slice(normal((3, 4), 1), [3, 4])
    b = T.Tensor.from_slice(normal((5,), 2), [5])
    with pytest.raises(T.TsError, match="Cannot broadcast tensor shapes"):
        a.add_tensor(b)
    # a zero divisor broadcast into the last 32 elements of the result panics
    num = T.Tensor.from_slice(np.ones((40, 1), np.float32), [40, 1])
    den = T.Tensor.from_slice(np.array([0.0], np.float32), [1])
    with pytest.raises(T.TsError, match="Division by zero"):
        num.div_tensor(den).data()


def test_graph_against_oracle():
    T = _T()
    G.CORRECTLY_ROUNDED = False  # the host libm, as the reference and the device
    try:
        a = normal((4, 1, 6), 1)
        b = normal((5, 6), 2)
        c = np.abs(normal((6,), 3)) + np.float32(0.5)
        ta, tb, tc = (T.Tensor.from_slice(v, v.shape).with_requires_grad() for v in (a, b, c))
        oa, ob, oc = (G.OTensor(v.copy(), True) for v in (a, b, c))

        def run(A, B, C):
            h = A.add_tensor(B).mul_tensor(C).sigmoid().div_tensor(C).sub_tensor(B.tanh())
            return h.softmax(2).log().mean_dims([0, 2]).leaky_relu(0.2).exp().sqrt().sum()

        s, os_ = run(ta, tb, tc), run(oa, ob, oc)
        assert abs(s.value() - os_.value()) <= 1e-6 * abs(os_.value())
        s.backward()
        G.backward(os_)
        for mine, theirs in ((ta, oa), (tb, ob), (tc, oc)):
            g, w = mine.grad_by_value().data(), theirs.grad_by_value()
            assert np.max(np.abs(g - w)) <= 1e-4 * float(np.max(np.abs(w)))
    finally:
        G.CORRECTLY_ROUNDED = False
        G.clear_gradients()
        T.clear_gradients()


def test_sum_dims_and_mean_dims():
    T = _T()
    x = normal((6, 7, 8), 4)
    for dims, keepdim in (([1], False), ([0, 2], True), ([2, 0, 2], False), ([0, 1, 2], False)):
        t = T.Tensor.from_slice(x, x.shape).with_requires_grad()
        s = t.sum_dims(dims, keepdim)
        want = O.sum_dims(x, dims, keepdim, f64=True)
        assert list(s.shape) == list(want.shape)
        assert np.max(np.abs(s.data() - want)) <= 1e-5 * max(1.0, float(np.max(np.abs(want))))
        m = t.mean_dims(dims, keepdim)
        factor = int(np.prod([x.shape[d] for d in dims]))
        assert np.max(np.abs(m.data() - want / factor)) <= 1e-5 * max(1.0, float(np.max(np.abs(want / factor))))
        go = normal(want.shape, 5)
        m.backward(T.Tensor.from_slice(go, want.shape))
        o = G.OTensor(x.copy(), True)
        G.backward(o.mean_dims(dims, keepdim), go)
        assert_bits_equal(t.grad_by_value().data(), o.grad_by_value())
        T.clear_gradients()
        G.clear_gradients()
    # the reference's quirks: zero-size axes are dropped from the output shape
    z = T.Tensor.zeros([0, 3]).sum_dims([1], False)
    assert list(z.shape) == [1] and z.data()[0] == 0.0
    with pytest.raises(T.TsError, match="out of bounds"):
        T.Tensor.zeros([2, 3]).sum_dims([2], False)
    with pytest.raises(T.TsError, match="softmax dim 2 out of bounds for rank 2"):
        T.Tensor.zeros([2, 3]).softmax(2)
