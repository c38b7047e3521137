"""transpose / t() / contiguous() / fill on the device (transform/transpose.rs,
transform/contiguous.rs, init/basic.rs; Transpose and Contiguous GradFns),
against the oracle and the reference's own known answers.  Copies and fills
are bit-exact; products read through a transposed view are within the GEMM
bar (<= 1e-4 normwise) of the oracle, and a view given to matmul is never
copied (no transpose launch, forward or backward)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import assert_bits_equal, max_rel, normal
from gpu_util import Dev, hip, hip_check, sync

pytestmark = pytest.mark.gpu


@pytest.fixture()
def TS():
    import train_station_amd as TS

    TS.clear_gradients()
    yield TS
    TS.set_fusion(True)
    TS.clear_gradients()


@pytest.fixture()
def G(oracle):
    import oracle.gradtrack as G

    G.clear_gradients()
    yield G
    G.clear_gradients()


def _launches(TS, fn):
    """Elementwise-class launches (where the transpose kernel is charged)
    while fn() runs and the device finishes it."""
    TS.Profile.reset()
    TS.Profile.enable(True)
    try:
        out = fn()
        TS.synchronize()
    finally:
        TS.Profile.enable(False)
    return TS.Profile.read(TS.Profile.ELEMENTWISE)["launches"], out


@pytest.mark.parametrize("shape,d0,d1", [((1, 1), 0, 1), ((63, 65), 0, 1), ((1000, 3), 0, 1), ((3, 1000), 1, 0),
                                         ((4096, 4096), 0, 1), ((129, 4097), 0, 1),
                                         ((3, 70, 65), 0, 1), ((3, 70, 65), 0, 2), ((3, 70, 65), 1, 2),
                                         ((2, 3, 4, 5), 0, 2), ((2, 3, 4, 5), 1, 3), ((2, 3, 4, 5), 0, 3),
                                         ((5, 1, 7), 0, 2), ((0, 4), 0, 1)])
def test_transpose_kernel_bit_exact(shape, d0, d1):
    print(f"[transpose] shape={shape} axes=({d0},{d1})", flush=True)
    x = normal(shape, 7)
    n = x.size
    dx, do = Dev.of(x if n else np.zeros(1, np.float32)), Dev(max(n, 1))
    dims = (ctypes.c_size_t * len(shape))(*shape)
    hip_check(hip.ts_hip_transpose(dx.ptr, dims, len(shape), d0, d1, do.ptr, None), "ts_hip_transpose")
    sync()
    want = np.ascontiguousarray(np.swapaxes(x, d0, d1))
    if n:
        assert_bits_equal(do.get(want.shape), want, "transpose")


def test_transpose_kernel_rejects_bad_axes():
    d = Dev(8)
    dims = (ctypes.c_size_t * 2)(2, 4)
    assert hip.ts_hip_transpose(d.ptr, dims, 2, 0, 2, d.ptr, None) == 100001


def test_reference_known_answers_on_device(TS):
    t = TS.Tensor.from_slice(np.arange(1, 7, dtype=np.float32), [2, 3]).transpose(0, 1)
    assert tuple(t.shape) == (3, 2) and not t.is_contiguous()
    assert t.data().tolist() == [[1, 4], [2, 5], [3, 6]]                  # transpose.rs:454-470
    assert TS.Tensor.from_slice([1, 2, 3, 4], [2, 2]).t().data().tolist() == [[1, 3], [2, 4]]
    x = TS.Tensor.from_slice(np.arange(24, dtype=np.float32), [2, 3, 4]).transpose(0, 1)
    got = x.data()
    assert got.shape == (3, 2, 4)                                          # :556-578
    for idx, v in {(0, 0, 0): 0, (0, 1, 0): 12, (1, 0, 0): 4, (1, 1, 0): 16, (2, 0, 0): 8, (2, 1, 0): 20}.items():
        assert got[idx] == v
    s = TS.Tensor.from_slice([1, 2, 3, 4], [2, 2]).with_requires_grad()
    same = s.transpose(1, 1)                                               # :498-510: a clone
    assert same.data().tolist() == [[1, 2], [3, 4]] and same.id() != s.id() and not same.requires_grad()
    assert s.transpose(0, 1).requires_grad()                               # :513-520
    with pytest.raises(TS.TsError, match="dim1 3 out of bounds for tensor with rank 2"):
        TS.Tensor.zeros([2, 3]).transpose(0, 3)                            # :523-527
    with pytest.raises(TS.TsError, match="Matrix transpose requires at least 2 dimensions, got 1"):
        TS.Tensor.zeros([5]).t()                                           # :530-534
    c = TS.Tensor.from_slice(np.arange(1, 7, dtype=np.float32), [2, 3]).contiguous()
    assert c.is_contiguous() and c.data().tolist() == [[1, 2, 3], [4, 5, 6]]  # contiguous.rs:355-366
    # contiguous.rs:389-417: gradients flow through transpose + contiguous
    x = TS.Tensor.from_slice([1, 2, 3, 4], [2, 2]).with_requires_grad()
    xc = x.transpose(0, 1).contiguous()
    assert xc.is_contiguous() and xc.requires_grad()
    xc.sum().backward()
    assert x.grad_by_value().data().tolist() == [[1, 1], [1, 1]]


@pytest.mark.parametrize("shape", [(2, 3), (0,), (100, 100), (1 << 20) + 3])
def test_fill_bit_exact(TS, shape):
    t = TS.Tensor.zeros(list(shape) if isinstance(shape, tuple) else [shape])
    t.fill(np.pi)                                                          # basic.rs:460-495
    got = t.data()
    assert got.size == int(np.prod(shape))
    assert_bits_equal(got, np.full(got.shape, np.float32(np.pi)), "fill")
    t.fill(-0.0)
    assert_bits_equal(t.data(), np.full(got.shape, np.float32(-0.0)), "fill -0")


def test_fill_runs_pending_readers_first_and_writes_through_a_view(TS):
    a = TS.Tensor.from_slice(np.arange(6, dtype=np.float32), [2, 3])
    b = a.mul_scalar(2.0)          # deferred: reads a before the fill
    v = a.t()                      # a view: reads a as it is when read
    a.fill(1.0)
    assert b.data().tolist() == [[0, 2, 4], [6, 8, 10]]
    assert v.data().tolist() == [[1, 1], [1, 1], [1, 1]]
    w = TS.Tensor.from_slice(np.arange(6, dtype=np.float32), [2, 3])
    c = w.t().contiguous()         # a copy: keeps w's values at the call
    vw = w.t()
    vw.fill(5.0)                   # through the view into w (shared storage)
    assert c.data().tolist() == [[0, 3], [1, 4], [2, 5]]
    assert w.data().tolist() == [[5, 5, 5], [5, 5, 5]]


@pytest.mark.parametrize("shape,d0,d1", [((33, 70), 0, 1), ((3, 40, 50), 0, 2), ((4, 6, 8, 10), 1, 3)])
def test_transpose_gradient_bit_exact(TS, G, oracle, shape, d0, d1):
    # y = transpose(x) * c; loss = sum(y): the gradient of x is c transposed
    # back, bit for bit
    xv = normal(shape, 1)
    tshape = list(shape)
    tshape[d0], tshape[d1] = tshape[d1], tshape[d0]
    cv = normal(tshape, 2)
    x = TS.Tensor.from_slice(xv, list(shape)).with_requires_grad()
    y = x.transpose(d0, d1).mul_tensor(TS.Tensor.from_slice(cv, tshape))
    y.sum().backward()
    xo = G.OTensor(xv.copy()).with_requires_grad()
    yo = xo.transpose(d0, d1).mul_tensor(G.OTensor(cv))
    yo.sum().backward()
    assert_bits_equal(y.data(), yo.data, "forward")
    assert_bits_equal(x.grad_by_value().data(), xo.grad_by_value(), "gradient")


@pytest.mark.parametrize("fusion", [True, False])
@pytest.mark.parametrize("B,I,O", [(64, 48, 40), (300, 784, 130), (1024, 1024, 1024)])
def test_linear_idiom_x_matmul_w_t(TS, G, B, I, O, fusion):
    # y = relu(x . W^T + b), W[out, in]; loss = mean((y - t)^2): forward and
    # every gradient against the oracle, and the same launches as with a
    # W^T stored as a plain tensor (the view is read by the products)
    TS.set_fusion(fusion)
    rng = np.random.default_rng(B + I + O)
    xv = rng.standard_normal((B, I)).astype(np.float32)
    wv = (rng.standard_normal((O, I)) / np.sqrt(I)).astype(np.float32)
    bv = (0.1 * rng.standard_normal(O)).astype(np.float32)
    tv = rng.standard_normal((B, O)).astype(np.float32)

    def device(w_is_view):
        x = TS.Tensor.from_slice(xv, [B, I]).with_requires_grad()
        if w_is_view:
            w = TS.Tensor.from_slice(wv, [O, I]).with_requires_grad()
            wt = w.t()
        else:
            w = TS.Tensor.from_slice(np.ascontiguousarray(wv.T), [I, O]).with_requires_grad()
            wt = w
        b = TS.Tensor.from_slice(bv, [O]).with_requires_grad()

        def step():
            y = x.matmul(wt).add_tensor(b).relu()
            loss = y.sub_tensor(TS.Tensor.from_slice(tv, [B, O])).pow_scalar(2.0).mean()
            loss.backward()
            return y, loss, [x.grad_by_value().data(), w.grad_by_value().data(), b.grad_by_value().data()]

        launches, (y, loss, grads) = _launches(TS, step)
        out = y.data(), loss.value(), grads, launches
        TS.clear_gradients()
        return out

    y, loss, (gx, gw, gb), launches = device(True)
    _, _, (_, gw_plain, _), launches_plain = device(False)
    assert launches == launches_plain, (launches, launches_plain)
    xo = G.OTensor(xv.copy()).with_requires_grad()
    wo = G.OTensor(wv.copy()).with_requires_grad()
    bo = G.OTensor(bv.copy()).with_requires_grad()
    yo = xo.matmul(wo.t()).add_tensor(bo)
    zo = yo.data
    mism = (y > 0) != (zo > 0)
    assert np.all(np.abs(zo[mism]) <= 1e-5 * np.max(np.abs(zo))), "mask differs away from zero"
    yo = yo.relu(mask_source=y)
    lo = yo.sub_tensor(G.OTensor(tv)).pow_scalar(2.0).mean()
    lo.backward()
    assert max_rel(y, yo.data) <= 1e-4
    assert abs(loss - lo.value()) <= 1e-4 * abs(lo.value())
    for name, got, want in (("x", gx, xo.grad_by_value()), ("W", gw, wo.grad_by_value()),
                            ("b", gb, bo.grad_by_value())):
        assert got.shape == want.shape, name
        assert max_rel(got, want) <= 1e-4, name
    assert max_rel(gw, gw_plain.T) <= 1e-5


def test_transposed_product_and_view_of_view(TS, oracle):
    rng = np.random.default_rng(3)
    av = rng.standard_normal((200, 300)).astype(np.float32)
    bv = rng.standard_normal((300, 150)).astype(np.float32)
    a, b = TS.Tensor.from_slice(av, [200, 300]), TS.Tensor.from_slice(bv, [300, 150])
    # the transpose of a product not yet run is written by the product itself
    n, pt = _launches(TS, lambda: a.matmul(b).t().data())
    assert n == 0
    assert max_rel(pt, oracle.gemm_f64(av, bv).T) <= 1e-4
    # t() of t(): the source's values, a contiguous copy
    tt = a.t().t()
    assert tt.is_contiguous()
    assert_bits_equal(tt.data(), av, "t().t()")
    # both operands transposed views: A^T . B^T
    c = TS.Tensor.from_slice(np.ascontiguousarray(av.T), [300, 200]).t().matmul(
        TS.Tensor.from_slice(np.ascontiguousarray(bv.T), [150, 300]).t())
    assert max_rel(c.data(), oracle.gemm_f64(av, bv)) <= 1e-4
