"""Pins of the restated transpose / t() / contiguous() / fill
(oracle/gradtrack.py) against facts from outside it: the reference's own
tests of tensor/transform/{transpose,contiguous}.rs and init/basic.rs (their
known answers and panic messages), and torch float64 autograd for the
gradients through a transpose."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import normal

from oracle import gradtrack as G


@pytest.fixture(autouse=True)
def _clean():
    G.clear_gradients()
    yield
    G.clear_gradients()


def test_reference_transpose_known_answers():
    # transpose.rs:454-470 (test_transpose_2d_basic)
    t = G.OTensor.from_slice([1, 2, 3, 4, 5, 6], [2, 3]).transpose(0, 1)
    assert t.shape == (3, 2)
    assert t.data.tolist() == [[1, 4], [2, 5], [3, 6]]
    # :473-486 (test_matrix_transpose)
    assert G.OTensor.from_slice([1, 2, 3, 4], [2, 2]).t().data.tolist() == [[1, 3], [2, 4]]
    # :489-495, :536-552: shapes
    assert G.OTensor(np.zeros((2, 3, 4), np.float32)).transpose(0, 2).shape == (4, 3, 2)
    assert G.OTensor(np.zeros((3, 4), np.float32)).transpose(0, 1).shape == (4, 3)
    # :556-578 (test_transpose_first_dimensions_3d)
    x = G.OTensor.from_slice(np.arange(24), [2, 3, 4]).transpose(0, 1)
    assert x.shape == (3, 2, 4)
    for idx, v in {(0, 0, 0): 0, (0, 1, 0): 12, (1, 0, 0): 4, (1, 1, 0): 16, (2, 0, 0): 8, (2, 1, 0): 20}.items():
        assert x.data[idx] == v
    # :498-510: the same axis twice is the tensor unchanged (a clone)
    s = G.OTensor.from_slice([1, 2, 3, 4], [2, 2])
    r = s.transpose(1, 1)
    assert r.data.tolist() == s.data.tolist() and r.id != s.id


def test_reference_transpose_panics_and_grad_flag():
    with pytest.raises(ValueError, match="out of bounds"):          # :523-527
        G.OTensor(np.zeros((2, 3), np.float32)).transpose(0, 3)
    with pytest.raises(ValueError, match="Matrix transpose requires at least 2 dimensions"):  # :530-534
        G.OTensor(np.zeros(5, np.float32)).t()
    x = G.OTensor(np.zeros((2, 3), np.float32)).with_requires_grad()
    assert x.transpose(0, 1).requires_grad                          # :513-520
    assert not x.transpose(1, 1).requires_grad                      # a clone tracks nothing


def test_reference_contiguous_and_fill_known_answers():
    # contiguous.rs:355-366, :420-444
    c = G.OTensor.from_slice([1, 2, 3, 4, 5, 6], [2, 3]).contiguous()
    assert c.shape == (2, 3) and c.data[0, 0] == 1 and c.data[1, 2] == 6
    assert G.OTensor.from_slice([1, 2, 3], [3]).contiguous().data.tolist() == [1, 2, 3]
    # :389-417 (test_contiguous_gradient_flow): sum of x^T made contiguous -> ones
    x = G.OTensor.from_slice([1, 2, 3, 4], [2, 2]).with_requires_grad()
    xc = x.transpose(0, 1).contiguous()
    assert xc.requires_grad
    xc.sum().backward()
    assert x.grad_by_value().tolist() == [[1, 1], [1, 1]]
    # basic.rs:460-495 (fill)
    t = G.OTensor(np.zeros((2, 3), np.float32))
    t.fill(42.0)
    assert (t.data == 42.0).all()
    e = G.OTensor(np.zeros(0, np.float32))
    e.fill(42.0)
    assert e.size() == 0
    big = G.OTensor(np.zeros((100, 100), np.float32))
    big.fill(np.pi)
    assert np.all(np.abs(big.data - np.float32(np.pi)) < 1e-6)


@pytest.mark.parametrize("shape,d0,d1", [((5, 7), 0, 1), ((3, 4, 5), 0, 2), ((3, 4, 5), 1, 2), ((2, 3, 4, 5), 0, 2),
                                         ((2, 3, 4, 5), 1, 3)])
def test_transpose_gradients_against_torch_autograd(shape, d0, d1):
    # y = transpose(x) * c (c in the transposed shape), loss = sum(y); and the
    # Linear idiom x . w^T with the weight's gradient reaching w through the
    # transpose
    xv = normal(shape, 1)
    tshape = list(shape)
    tshape[d0], tshape[d1] = tshape[d1], tshape[d0]
    cv = normal(tshape, 2)
    x = G.OTensor(xv.copy()).with_requires_grad()
    x.transpose(d0, d1).mul_tensor(G.OTensor(cv)).sum().backward()
    xt = torch.tensor(xv, dtype=torch.float64, requires_grad=True)
    (xt.transpose(d0, d1) * torch.tensor(cv, dtype=torch.float64)).sum().backward()
    np.testing.assert_allclose(x.grad_by_value(), xt.grad.numpy(), rtol=1e-6, atol=1e-6)


def test_linear_idiom_against_torch_autograd():
    xv, wv, bv = normal((16, 12), 3), normal((8, 12), 4), normal(8, 5)
    x = G.OTensor(xv.copy()).with_requires_grad()
    w = G.OTensor(wv.copy()).with_requires_grad()
    b = G.OTensor(bv.copy()).with_requires_grad()
    x.matmul(w.t()).add_tensor(b).relu().sum().backward()
    xt, wt, bt = (torch.tensor(v, dtype=torch.float64, requires_grad=True) for v in (xv, wv, bv))
    torch.relu(xt @ wt.t() + bt).sum().backward()
    for o, t in ((x, xt), (w, wt), (b, bt)):
        np.testing.assert_allclose(o.grad_by_value(), t.grad.numpy(), rtol=1e-5, atol=1e-5)
