"""Pins of the restated activations, softmax, axis sums and broadcasting
(oracle/ts_oracle.c, oracle/gradtrack.py) against facts from outside it:

* the reference's own tests (tensor/ops/{sigmoid,tanh,leaky_relu,log,sqrt,
  softmax}.rs, reductions/sum.rs) -- their known answers;
* torch on the CPU: float64 values rounded once (the correctly rounded
  result), float32 elementwise arithmetic in the reference's order (IEEE,
  an independent implementation), float64 autograd for the gradients;
* long double over a strided sweep of all 2^32 inputs for exp / ln / tanh.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import assert_bits_equal, normal

import oracle as O
from oracle import gradtrack as G

SPECIAL = np.array([0.0, -0.0, 1.0, -1.0, 0.5, 88.7, 88.8, -87.3, -103.0, -104.0, 1e-30, -1e-30, 1e-41,
                    20.0, -20.0, 9.0, -9.0, 1e-8, 3.4e38, -3.4e38, np.inf, -np.inf, np.nan], np.float32)


def _inputs(n=4099, seed=0):
    return np.concatenate([SPECIAL, normal(n, seed, 4.0)]).astype(np.float32)


def test_reference_known_answers():
    tol = 1e-6
    s = O.unary("sigmoid", [-1.0, 0.0, 1.0])
    assert np.allclose(s, [0.26894143, 0.5, 0.7310586], atol=tol)          # sigmoid.rs tests
    t = O.unary("tanh", [-1.0, 0.0, 1.0])
    assert np.allclose(t, [-0.7615942, 0.0, 0.7615942], atol=tol)           # tanh.rs tests
    lr = O.unary("leaky_relu", [-2.0, -1.0, 0.0, 1.5], slope=0.1)
    assert np.allclose(lr, [-0.2, -0.1, 0.0, 1.5], atol=tol)                 # leaky_relu.rs tests
    assert np.array_equal(O.unary("sqrt", [0.0, 1.0, 4.0, 9.0]), [0.0, 1.0, 2.0, 3.0])  # sqrt.rs tests
    x = np.array([1.0, 2.0, 4.0], np.float32)                                # log.rs backward test
    assert np.allclose(O.unary_bwd("log", x, np.ones(3, np.float32)), [1.0, 0.5, 0.25], atol=tol)
    assert abs(float(O.softmax(np.array([0.0, 1.0, 2.0], np.float32), 0).sum()) - 1.0) < tol  # softmax.rs
    m = np.array([[1, 2, 3], [4, 5, 6]], np.float32)                         # sum.rs tests
    assert np.array_equal(O.sum_dims(m.T.copy(), [0]), [6.0, 15.0])
    assert np.array_equal(O.sum_dims(m.T.copy(), [1]), [5.0, 7.0, 9.0])
    assert np.array_equal(O.sum_dims(m, [0]), [5.0, 7.0, 9.0])


@pytest.mark.parametrize("op", ["exp", "log", "tanh", "sqrt"])
def test_correctly_rounded_mode_equals_torch_f64_rounded(op):
    x = _inputs()
    if op in ("log", "sqrt"):
        x = np.abs(x)
    want = getattr(torch, op)(torch.from_numpy(x.astype(np.float64))).numpy().astype(np.float32)
    assert_bits_equal(O.unary(op, x, correctly_rounded=True), want, op)


def test_sigmoid_both_branches_against_torch_f32_steps():
    x = _inputs()
    tx = torch.from_numpy(x)
    z_pos = torch.from_numpy(O.unary("exp", -x, correctly_rounded=True))
    z_neg = torch.from_numpy(O.unary("exp", x, correctly_rounded=True))
    want = torch.where(tx >= 0, 1.0 / (1.0 + z_pos), z_neg / (1.0 + z_neg)).numpy()
    assert_bits_equal(O.unary("sigmoid", x, correctly_rounded=True), want)
    # and it is the logistic function to within a few ulps of f64
    ref = torch.sigmoid(torch.from_numpy(x[np.isfinite(x)].astype(np.float64))).numpy()
    got = O.unary("sigmoid", x[np.isfinite(x)], correctly_rounded=True).astype(np.float64)
    assert np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)) < 3e-7


@pytest.mark.parametrize("op", ["exp", "log", "tanh"])
def test_f64_rounded_once_is_correctly_rounded(op):
    # every 1021st bit pattern of the f32 line against long double
    assert O.unary_cr_check(op, 1021) == 0


@pytest.mark.parametrize("op,limit", [("exp", 1e-4), ("log", 1e-3), ("tanh", 0.05)])
def test_host_libm_is_close_to_correct_rounding(op, limit):
    # glibc's expf / logf / tanhf are not correctly rounded everywhere: this is
    # where the device (correctly rounded) and the reference can differ
    n = (1 << 32) // 1021
    d = O.unary_glibc_diff(op, 1021)
    assert d / n < limit


def test_backward_formulas_against_torch_f32_in_reference_order():
    rng = np.random.default_rng(3)
    go = normal(4099, 7)
    x = np.abs(normal(4099, 8)) + np.float32(0.1)
    y = rng.uniform(-0.99, 0.99, 4099).astype(np.float32)
    t = torch.from_numpy
    cases = {
        "exp": (y, t(go) * t(y)),
        "log": (x, t(go) * (1.0 / t(x))),
        "sqrt": (x, t(go) * ((1.0 / t(x)) * 0.5)),
        "tanh": (y, t(go) * (1.0 - t(y) * t(y))),
        "sigmoid": (y, t(go) * t(y) * (1.0 - t(y))),
    }
    for op, (saved, want) in cases.items():
        assert_bits_equal(O.unary_bwd(op, saved, go), want.numpy(), op)
    xs = normal(4099, 9)
    want = torch.where(t(xs) > 0, t(go), 0.01 * t(go)).numpy()
    assert_bits_equal(O.unary_bwd("leaky_relu", xs, go, slope=0.01), want)


@pytest.mark.parametrize("shape,dim", [((7, 10), 1), ((4, 5, 6), 1), ((33,), 0), ((3, 4, 5), 0)])
def test_softmax_against_torch(shape, dim):
    x = normal(shape, 11, 3.0)
    y = O.softmax(x, dim, correctly_rounded=True)
    tx = torch.from_numpy(x.astype(np.float64)).requires_grad_(True)
    ty = torch.softmax(tx, dim)
    assert np.max(np.abs(y - ty.detach().numpy())) < 2e-7
    go = normal(shape, 12)
    ty.backward(torch.from_numpy(go.astype(np.float64)))
    gi = O.softmax_bwd(y, go, dim)
    assert np.max(np.abs(gi - tx.grad.numpy())) / np.max(np.abs(tx.grad.numpy())) < 1e-5


@pytest.mark.parametrize("shape,dims,keepdim", [
    ((4, 5, 6), [1], False), ((4, 5, 6), [0, 2], True), ((4, 5, 6), [2, 0, 2], False),
    ((3, 1, 7), [1], False), ((8,), [0], False), ((2, 3, 4, 5), [1, 3], True), ((0, 3), [1], False),
])
def test_sum_dims_shapes_and_values(shape, dims, keepdim):
    x = normal(shape, 5)
    got = O.sum_dims(x, dims, keepdim)
    want = x.astype(np.float64).sum(axis=tuple(sorted(set(dims))), keepdims=keepdim)
    if shape == (0, 3):
        assert list(got.shape) == [1]  # the reference drops zero-size axes from the output shape
        return
    assert list(got.shape) == (list(want.shape) or [1])
    assert np.max(np.abs(got - want.reshape(got.shape))) < 1e-5 * max(1.0, np.max(np.abs(want)))


def test_graph_with_broadcasting_and_new_ops_against_torch_autograd():
    G.CORRECTLY_ROUNDED = True
    try:
        a = normal((4, 1, 6), 1)
        b = normal((5, 6), 2)
        c = np.abs(normal((6,), 3)) + np.float32(0.5)
        ta, tb, tc = (torch.from_numpy(v.astype(np.float64)).requires_grad_(True) for v in (a, b, c))
        A, B, C = (G.OTensor(v.copy(), True) for v in (a, b, c))
        # ((a + b) * c).sigmoid() / c - tanh(b) -> softmax(dim 2) -> log -> mean_dims([0, 2])
        h = A.add_tensor(B).mul_tensor(C).sigmoid().div_tensor(C).sub_tensor(B.tanh())
        s = h.softmax(2).log().mean_dims([0, 2]).leaky_relu(0.2).exp().sum()
        s.backward()
        th = ((ta + tb) * tc).sigmoid() / tc - torch.tanh(tb)
        ts = torch.nn.functional.leaky_relu(torch.log(torch.softmax(th, 2)).mean(dim=(0, 2)), 0.2).exp().sum()
        ts.backward()
        assert abs(s.value() - ts.item()) < 1e-5 * abs(ts.item())
        for mine, theirs in ((A, ta), (B, tb), (C, tc)):
            g = mine.grad_by_value()
            want = theirs.grad.numpy()
            assert g.shape == want.shape
            assert np.max(np.abs(g - want)) / np.max(np.abs(want)) < 1e-4
    finally:
        G.CORRECTLY_ROUNDED = False
        G.clear_gradients()


MATMUL_CASES = [((7,), (7,)), ((7,), (7, 5)), ((6, 7), (7,)), ((6, 7), (7, 5)), ((3, 6, 7), (3, 7, 5)),
                ((2, 1, 6, 7), (4, 7, 5)), ((6, 7), (4, 7, 5)), ((2, 3, 6, 7), (7, 5)), ((1, 6, 7), (7, 5)),
                ((6, 7), (1, 7, 5))]


@pytest.mark.parametrize("sa,sb", MATMUL_CASES, ids=lambda s: "x".join(map(str, s)))
def test_matmul_ranks_against_torch_autograd(sa, sb):
    a, b = normal(sa, 1), normal(sb, 2)
    A, B = G.OTensor(a.copy(), True), G.OTensor(b.copy(), True)
    ta, tb = (torch.from_numpy(v.astype(np.float64)).requires_grad_(True) for v in (a, b))
    y = A.matmul(B)
    ty = torch.matmul(ta, tb)
    assert y.shape == tuple(ty.shape)
    assert np.max(np.abs(y.data - ty.detach().numpy())) <= 1e-6 * max(1.0, float(ty.abs().max()))
    go = np.array(normal(y.shape, 3), np.float32).reshape(y.shape)
    G.backward(y, go)
    ty.backward(torch.from_numpy(go.astype(np.float64)))
    for mine, theirs in ((A, ta), (B, tb)):
        g = mine.grad_by_value()
        assert g.shape == tuple(theirs.shape)  # operand-shaped gradients in every case
        assert np.max(np.abs(g - theirs.grad.numpy())) <= 1e-5 * max(1.0, float(theirs.grad.abs().max()))
    G.clear_gradients()


@pytest.mark.parametrize("sa,sb,msg", [((3,), (4,), "same length"), ((3,), (4, 2), "Vector length"),
                                       ((2, 3), (4,), "Matrix columns"), ((3,), (2, 3, 4), "at least 2D")])
def test_matmul_shape_errors(sa, sb, msg):
    with pytest.raises(ValueError, match=msg):
        G.OTensor(normal(sa, 1)).matmul(G.OTensor(normal(sb, 2)))


def _glibc_2_35():
    import platform
    return platform.libc_ver() == ("glibc", "2.35")


@pytest.mark.skipif(not _glibc_2_35(), reason="the restatement pins glibc 2.35, the image's libm")
@pytest.mark.parametrize("fn", ["exp", "log", "tanh", "cos", "expm1"])
def test_glibc_restatement_equals_the_host_libm(fn):
    # ts_oracle.c's restatement of glibc 2.35's expf / logf / tanhf / cosf
    # (below 120) / expm1f against the host libm on every 17th f32 bit
    # pattern from two offsets (about 5e8 inputs; every one of the 2^32 was
    # checked once, with 0 differences)
    for off in (0, 8):
        assert O.glibc_restated_diff(fn, 17, off) == 0, (fn, off)


@pytest.mark.skipif(not _glibc_2_35(), reason="the restatement pins glibc 2.35, the image's libm")
def test_glibc_restatement_through_the_ops_and_randn():
    # the modes end to end: unary ops, softmax and randn in the restated mode
    # equal the host-libm mode bit for bit, and the two differ from f64
    # rounded once (a mutation that made the restated mode call the f64
    # path would fail the last check)
    x = normal(1 << 18, 11, 8.0)
    for op in ("exp", "tanh", "sigmoid"):
        assert_bits_equal(O.unary(op, x, restated=True), O.unary(op, x), op)
    assert_bits_equal(O.unary("log", np.abs(x), restated=True), O.unary("log", np.abs(x)), "log")
    y = normal((64, 257), 12, 5.0)
    assert_bits_equal(O.softmax(y, 1, restated=True), O.softmax(y, 1), "softmax")
    r = O.randn(1 << 20, 77, restated=True)
    assert_bits_equal(r, O.randn(1 << 20, 77), "randn")
    assert np.any(r != O.randn(1 << 20, 77, correctly_rounded=True))
    assert np.any(O.unary("tanh", x, restated=True) != O.unary("tanh", x, correctly_rounded=True))
