"""Pins the oracle's restatement of the gradtrack engine and Adam
(oracle/gradtrack.py) against the reference's own known answers, its LibTorch
Adam validation cases (torch.optim.Adam fixtures) and torch autograd in
float64.  CPU only."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import golden, max_rel, normal, uniform


@pytest.fixture()
def G(oracle):
    import oracle.gradtrack as G

    G.clear_gradients()
    yield G
    G.clear_gradients()


def test_matmul_2x2_known_answer(G):
    ka = golden("known_answers.json")["matmul_2x2"]
    a = G.OTensor.from_slice(ka["a"], [2, 2]).with_requires_grad()
    b = G.OTensor.from_slice(ka["b"], [2, 2]).with_requires_grad()
    r = a.matmul(b)
    assert r.data.reshape(-1).tolist() == ka["out"]
    r.backward(np.array(ka["grad_output"], np.float32).reshape(2, 2))
    assert a.grad_by_value().reshape(-1).tolist() == ka["grad_a"]
    assert b.grad_by_value().reshape(-1).tolist() == ka["grad_b"]


def test_linear_bias_grad_known_answer(G):
    ka = golden("known_answers.json")["linear_bias_grad"]
    x = G.OTensor.from_slice(ka["input"], ka["input_shape"]).with_requires_grad()
    w = G.OTensor.from_slice(ka["weight"], ka["weight_shape"]).with_requires_grad()
    b = G.OTensor.from_slice(ka["bias"], [4]).with_requires_grad()
    loss = x.matmul(w).add_tensor(b).sum()
    loss.backward()
    assert np.allclose(b.grad_by_value(), ka["bias_grad"], atol=ka["tol"])


def test_sum_and_mean_grad_known_answers(G):
    ka = golden("known_answers.json")
    c = ka["sum_all_ones_grad"]
    x = G.OTensor.from_slice(c["x"], c["shape"]).with_requires_grad()
    x.sum().backward()
    assert x.grad_by_value().reshape(-1).tolist() == c["grad"]
    G.clear_gradients()
    c = ka["sum_chain_grad"]
    x = G.OTensor.from_slice(c["x"], c["shape"]).with_requires_grad()
    x.mul_scalar(c["mul"]).add_scalar(c["add"]).sum().backward()
    assert x.grad_by_value().reshape(-1).tolist() == c["grad"]
    G.clear_gradients()
    c = ka["mean_grad"]
    x = G.OTensor.from_slice(c["x"], c["shape"]).with_requires_grad()
    x.mean().backward()
    assert x.grad_by_value().reshape(-1).tolist() == c["grad"]


def _loss_for(G, p, kind):
    if kind == "sum(2p+1)":
        return p.mul_scalar(2.0).add_scalar(1.0).sum()
    d = p.add_scalar(-0.5)                       # adam.rs:1112-1116
    return d.mul_tensor(d).sum()


@pytest.mark.parametrize("case", list(golden("adam_libtorch_cases.json")))
def test_adam_libtorch_validation_cases(G, case):
    c = golden("adam_libtorch_cases.json")[case]
    p = G.OTensor.from_slice(c["p0"], c["shape"]).with_requires_grad()
    opt = G.OAdam(weight_decay=c["config"].get("weight_decay", 0.0),
                  amsgrad=c["config"].get("amsgrad", False))
    opt.add_parameter(p)
    for step, want in enumerate(c["torch_trajectory"]):
        _loss_for(G, p, c["loss"]).backward()
        opt.step([p])
        opt.zero_grad([p])
        got = p.data.reshape(-1).astype(np.float64)
        want = np.array(want)
        ok = (np.abs(got - want) <= c["rtol"] * np.abs(want)) | (np.abs(got - want) <= c["atol"])
        assert ok.all(), (case, step, got, want)


def test_chain_gradients_against_torch_float64(G, oracle):
    # BASELINE config 2 graph at a small size with an 8-wide tail
    n = 1003
    a, b = normal(n, 1), normal(n, 2)
    c = uniform(n, 0.5, 2.0, 3)
    ta, tb, tc = (G.OTensor(v.copy()).with_requires_grad() for v in (a, b, c))
    t1 = ta.add_tensor(tb)
    y = t1.mul_tensor(tc).sub_tensor(ta.div_tensor(tc)).relu()
    loss = y.sum()
    loss.backward()
    A, B, C = (torch.tensor(v, dtype=torch.float64, requires_grad=True) for v in (a, b, c))
    L = torch.relu((A + B) * C - A / C).sum()
    L.backward()
    assert abs(loss.value() - L.item()) <= 1e-5 * abs(L.item())
    for t, T in ((ta, A), (tb, B), (tc, C)):
        assert max_rel(t.grad_by_value(), T.grad.numpy()) < 1e-5


def test_chain_backward_matches_closed_form_bits(G, oracle):
    # engine.rs LIFO order: t3 (div) before t2 (mul); derived formulas of the
    # C2 chain, evaluated with the same fp32 primitives, must match bit for bit.
    n = 77
    a, b = normal(n, 4), normal(n, 5)
    c = uniform(n, 0.5, 2.0, 6)
    ta, tb, tc = (G.OTensor(v.copy()).with_requires_grad() for v in (a, b, c))
    t1 = ta.add_tensor(tb)
    t4 = t1.mul_tensor(tc).sub_tensor(ta.div_tensor(tc))
    t4.relu().sum().backward()
    g4 = oracle.relu_bwd(t4.data, np.ones(n, np.float32))
    g3 = oracle.neg(g4)
    ga = oracle.add(oracle.div(g3, c), oracle.mul(g4, c))
    gb = oracle.mul(g4, c)
    gc = oracle.add(oracle.neg(oracle.div(oracle.mul(g3, a), oracle.mul(c, c))), oracle.mul(g4, t1.data))
    from conftest import assert_bits_equal
    assert_bits_equal(ta.grad_by_value(), ga, "ga")
    assert_bits_equal(tb.grad_by_value(), gb, "gb")
    assert_bits_equal(tc.grad_by_value(), gc, "gc")


def test_mlp_step_against_torch_float64(G):
    # BASELINE config 4 graph at a reduced size: relu(x W1 + b1) W2 + b2, MSE
    B, I, H, O = 64, 50, 32, 10
    x, t = normal((B, I), 7), normal((B, O), 8)
    w1 = uniform((I, H), -(6 / I) ** 0.5, (6 / I) ** 0.5, 9)
    w2 = uniform((H, O), -(6 / H) ** 0.5, (6 / H) ** 0.5, 10)
    b1, b2 = np.zeros(H, np.float32), np.zeros(O, np.float32)
    ps = [G.OTensor(v.copy()).with_requires_grad() for v in (w1, b1, w2, b2)]
    X, Tt = G.OTensor(x), G.OTensor(t)
    y = X.matmul(ps[0]).add_tensor(ps[1]).relu().matmul(ps[2]).add_tensor(ps[3])
    loss = y.sub_tensor(Tt).pow_scalar(2.0).mean()
    loss.backward()
    tp = [torch.tensor(v, dtype=torch.float64, requires_grad=True) for v in (w1, b1, w2, b2)]
    Y = torch.relu(torch.tensor(x, dtype=torch.float64) @ tp[0] + tp[1]) @ tp[2] + tp[3]
    L = ((Y - torch.tensor(t, dtype=torch.float64)) ** 2).mean()
    L.backward()
    assert abs(loss.value() - L.item()) <= 1e-5 * abs(L.item())
    for p, T in zip(ps, tp):
        assert max_rel(p.grad_by_value(), T.grad.numpy()) < 1e-4


def test_positional_gradient_mapping(G):
    # input_ids lists only operands that require grad while apply() returns
    # gradients by position (ops/sub.rs:149-156, grad_fn/ops/sub.rs:14-31):
    # in a - b with only b requiring grad, b receives +g.
    a = G.OTensor(np.ones(4, np.float32))
    b = G.OTensor(np.ones(4, np.float32)).with_requires_grad()
    a.sub_tensor(b).sum().backward()
    assert b.grad_by_value().tolist() == [1.0, 1.0, 1.0, 1.0]
