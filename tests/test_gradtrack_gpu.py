"""End-to-end parity of the training step on the GPU (libts_gradtrack.so over
libts_hip.so) against the oracle's restatement of the reference
(oracle/gradtrack.py), on the BASELINE configurations.

Bars: elementwise ops, ReLU masks and Adam arithmetic bit-exact; matmul-derived
gradients and reductions <= 1e-4 normwise relative error (max|d| / max|ref|);
parameters after 100 Adam steps <= 1e-4 relative (normwise).  Loss values are
compared with the f64 value (the reference's own sequential fp32 sum drifts,
see tests/test_oracle.py)."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_bits_equal, golden, max_rel, normal, uniform

pytestmark = pytest.mark.gpu


@pytest.fixture()
def TS():
    import train_station_amd as TS

    TS.clear_gradients()
    yield TS
    TS.clear_gradients()


@pytest.fixture()
def G(oracle):
    import oracle.gradtrack as G

    G.clear_gradients()
    yield G
    G.clear_gradients()


# ---- the reference's own known answers, through the device API --------------------------

def test_known_answers_on_device(TS):
    ka = golden("known_answers.json")
    c = ka["matmul_2x2"]
    a = TS.Tensor.from_slice(c["a"], [2, 2]).with_requires_grad()
    b = TS.Tensor.from_slice(c["b"], [2, 2]).with_requires_grad()
    r = a.matmul(b)
    assert r.data().reshape(-1).tolist() == c["out"]
    r.backward(TS.Tensor.from_slice(c["grad_output"], [2, 2]))
    assert a.grad_by_value().data().reshape(-1).tolist() == c["grad_a"]
    assert b.grad_by_value().data().reshape(-1).tolist() == c["grad_b"]
    TS.clear_gradients()

    c = ka["linear_bias_grad"]
    x = TS.Tensor.from_slice(c["input"], c["input_shape"]).with_requires_grad()
    w = TS.Tensor.from_slice(c["weight"], c["weight_shape"]).with_requires_grad()
    bias = TS.Tensor.from_slice(c["bias"], [4]).with_requires_grad()
    x.matmul(w).add_tensor(bias).sum().backward()
    assert np.allclose(bias.grad_by_value().data(), c["bias_grad"], atol=c["tol"])
    TS.clear_gradients()

    for key in ("sum_forward", "sum_21", "sum_276"):
        c = ka[key]
        assert abs(TS.Tensor.from_slice(c["x"], c["shape"]).sum().value() - c["sum"]) <= c.get("tol", 0)
    for key in ("mean_forward", "mean_3_5"):
        c = ka[key]
        assert abs(TS.Tensor.from_slice(c["x"], c["shape"]).mean().value() - c["mean"]) <= c["tol"]
    c = ka["sum_chain_grad"]
    x = TS.Tensor.from_slice(c["x"], c["shape"]).with_requires_grad()
    x.mul_scalar(c["mul"]).add_scalar(c["add"]).sum().backward()
    assert x.grad_by_value().data().reshape(-1).tolist() == c["grad"]
    TS.clear_gradients()
    c = ka["mean_grad"]
    x = TS.Tensor.from_slice(c["x"], c["shape"]).with_requires_grad()
    x.mean().backward()
    assert x.grad_by_value().data().reshape(-1).tolist() == c["grad"]
    c = ka["relu_forward"]
    assert TS.Tensor.from_slice(c["x"], [3]).relu().data().tolist() == c["out"]
    c = ka["pow_scalar_forward"]
    assert TS.Tensor.from_slice(c["x"], [4]).pow_scalar(2.0).data().tolist() == c["out"]


def _device_loss(TS, p, kind):
    if kind == "sum(2p+1)":
        return p.mul_scalar(2.0).add_scalar(1.0).sum()
    d = p.add_scalar(-0.5)
    return d.mul_tensor(d).sum()


@pytest.mark.parametrize("case", list(golden("adam_libtorch_cases.json")))
def test_adam_libtorch_cases_on_device(TS, G, case):
    c = golden("adam_libtorch_cases.json")[case]
    cfg = dict(weight_decay=c["config"].get("weight_decay", 0.0), amsgrad=c["config"].get("amsgrad", False))
    p = TS.Tensor.from_slice(c["p0"], c["shape"]).with_requires_grad()
    opt = TS.Adam.with_config(**cfg)
    opt.add_parameter(p)
    po = G.OTensor.from_slice(c["p0"], c["shape"]).with_requires_grad()
    oopt = G.OAdam(**cfg)
    oopt.add_parameter(po)
    for step, want in enumerate(c["torch_trajectory"]):
        _device_loss(TS, p, c["loss"]).backward()
        opt.step([p])
        opt.zero_grad([p])
        _device_loss(G, po, c["loss"]).backward()
        oopt.step([po])
        oopt.zero_grad([po])
        got = p.data()
        assert_bits_equal(got, po.data, f"{case} step {step} vs oracle")
        want = np.array(want).reshape(got.shape)
        d = np.abs(got.astype(np.float64) - want)
        assert ((d <= c["rtol"] * np.abs(want)) | (d <= c["atol"])).all(), (case, step)


# ---- config 1: README quick-start step ---------------------------------------------------------

def test_config1_readme_step(TS, G):
    x = normal((32, 784), 0)
    w = normal((784, 128), 1)
    b = np.zeros(128, np.float32)
    pd = [TS.Tensor.from_slice(w, w.shape).with_requires_grad(), TS.Tensor.from_slice(b, b.shape).with_requires_grad()]
    po = [G.OTensor(w.copy()).with_requires_grad(), G.OTensor(b.copy()).with_requires_grad()]
    opt, oopt = TS.Adam.with_learning_rate(1e-3), G.OAdam(1e-3)
    opt.add_parameters(pd)
    oopt.add_parameters(po)
    xd = TS.Tensor.from_slice(x, x.shape)
    for step in range(100):
        y = xd.matmul(pd[0]).add_tensor(pd[1]).relu()
        loss = y.sum()
        loss.backward()
        if step == 0:
            gw, gb = pd[0].grad_by_value().data(), pd[1].grad_by_value().data()
        opt.step(pd)
        opt.zero_grad(pd)
        yo = G.OTensor(x).matmul(po[0]).add_tensor(po[1]).relu()
        lo = yo.sum()
        lo.backward()
        if step == 0:
            assert max_rel(gw, po[0].grad_by_value()) <= 1e-4
            assert max_rel(gb, po[1].grad_by_value()) <= 1e-4
            assert abs(loss.value() - float(np.sum(yo.data, dtype=np.float64))) <= 1e-4 * abs(loss.value())
        oopt.step(po)
        oopt.zero_grad(po)
    for d, o in zip(pd, po):
        assert max_rel(d.data(), o.data) <= 1e-4


# ---- config 2: elementwise autograd chain ------------------------------------------------------

@pytest.mark.parametrize("n", [1003, (1 << 20) + 13, 1 << 26])
def test_config2_chain_bit_exact(TS, G, n):
    print(f"[chain] n={n}", flush=True)
    a, b = normal(n, 1), normal(n, 2)
    c = uniform(n, 0.5, 2.0, 3)
    ta, tb, tc = (TS.Tensor.from_slice(v, [n]).with_requires_grad() for v in (a, b, c))
    y = ta.add_tensor(tb).mul_tensor(tc).sub_tensor(ta.div_tensor(tc)).relu()
    loss = y.sum()
    loss.backward()
    oa, ob, oc = (G.OTensor(v.copy()).with_requires_grad() for v in (a, b, c))
    yo = oa.add_tensor(ob).mul_tensor(oc).sub_tensor(oa.div_tensor(oc)).relu()
    lo = yo.sum()
    lo.backward()
    assert_bits_equal(y.data(), yo.data, "forward y")
    for t, o, name in ((ta, oa, "ga"), (tb, ob, "gb"), (tc, oc, "gc")):
        assert_bits_equal(t.grad_by_value().data(), o.grad_by_value(), name)
    exact = float(np.sum(yo.data, dtype=np.float64))
    assert abs(loss.value() - exact) <= 1e-6 * abs(exact)


def test_division_by_zero_is_reported(TS):
    n = 40
    a = TS.Tensor.from_slice(np.ones(n, np.float32), [n])
    z = np.ones(n, np.float32)
    z[35] = 0.0
    q = a.div_tensor(TS.Tensor.from_slice(z, [n]))
    with pytest.raises(TS.TsError, match="Division by zero detected at index 35"):
        q.data()
    z[35] = 1.0
    z[3] = 0.0          # inside the unchecked body: no error, +inf as on the CPU
    q = a.div_tensor(TS.Tensor.from_slice(z, [n]))
    assert np.isinf(q.data()[3])
    with pytest.raises(TS.TsError, match="zero scalar"):
        a.div_scalar(0.0)


# ---- config 3: Adam alone -----------------------------------------------------------------------

def test_config3_adam_100_steps_via_api(TS, G):
    # p ~ N(0,1), g ~ N(0, 1e-2) set once with set_grad (utils.rs:766-770), m = v = 0
    n = 1 << 22
    p0, g = normal(n, 4), normal(n, 5, 0.1)
    p = TS.Tensor.from_slice(p0, [n]).with_requires_grad()
    p.set_grad(TS.Tensor.from_slice(g, [n]))
    opt = TS.Adam.new()
    opt.add_parameter(p)
    po = G.OTensor(p0.copy()).with_requires_grad()
    po.grad = g.copy()
    oopt = G.OAdam()
    oopt.add_parameter(po)
    for _ in range(100):
        opt.step([p])
        oopt.step([po])
    assert_bits_equal(p.data(), po.data, "params after 100 steps")


# ---- config 4 and a scaled config 5: MLP training steps ------------------------------------------

def _mlp(lib_tensor, x, t, params, relu_last=False):
    h = x
    n = len(params) // 2
    for i in range(n):
        h = h.matmul(params[2 * i]).add_tensor(params[2 * i + 1])
        if i < n - 1 or relu_last:
            h = h.relu()
    return h.sub_tensor(t).pow_scalar(2.0).mean()


def _mlp_parity(TS, G, dims, batch, steps, seed, init):
    rng = np.random.default_rng(seed)
    ws = []
    for i in range(len(dims) - 1):
        fan_in = dims[i]
        if init == "kaiming":
            bound = (6.0 / fan_in) ** 0.5
            w = rng.uniform(-bound, bound, (dims[i], dims[i + 1])).astype(np.float32)
        else:
            w = (rng.standard_normal((dims[i], dims[i + 1])) / np.sqrt(fan_in)).astype(np.float32)
        ws += [w, np.zeros(dims[i + 1], np.float32)]
    x = rng.standard_normal((batch, dims[0])).astype(np.float32)
    t = rng.standard_normal((batch, dims[-1])).astype(np.float32)
    pd = [TS.Tensor.from_slice(v, v.shape).with_requires_grad() for v in ws]
    po = [G.OTensor(v.copy()).with_requires_grad() for v in ws]
    opt, oopt = TS.Adam.new(), G.OAdam()
    opt.add_parameters(pd)
    oopt.add_parameters(po)
    xd, td = TS.Tensor.from_slice(x, x.shape), TS.Tensor.from_slice(t, t.shape)
    xo, to = G.OTensor(x), G.OTensor(t)
    worst = 0.0
    for step in range(steps):
        loss = _mlp(TS, xd, td, pd)
        loss.backward()
        lo = _mlp(G, xo, to, po)
        lo.backward()
        if step == 0:
            for d, o in zip(pd, po):
                assert max_rel(d.grad_by_value().data(), o.grad_by_value()) <= 1e-4
        assert abs(loss.value() - lo.value()) <= 1e-4 * abs(lo.value())
        opt.step(pd)
        opt.zero_grad(pd)
        oopt.step(po)
        oopt.zero_grad(po)
    for d, o in zip(pd, po):
        worst = max(worst, max_rel(d.data(), o.data))
    return worst


def test_config4_mlp(TS, G):
    # batch 1024, 784 -> 1024 -> 10, Kaiming-uniform, MSE; 10 steps against the oracle
    worst = _mlp_parity(TS, G, [784, 1024, 10], 1024, 10, seed=0, init="kaiming")
    assert worst <= 1e-4


def test_config5_scaled_mlp(TS, G):
    # config 5 structure (6 layers, N(0, 1/fan_in) weights, ReLU on layers 1-5, MSE) at width 256
    worst = _mlp_parity(TS, G, [256] * 7, 512, 5, seed=1, init="normal")
    assert worst <= 1e-4


def test_config5_full_size_step_runs(TS):
    # the bench workload itself: two steps at B = 8192, 6 x 4096^2; finite and
    # the loss moves (the contraction kernels at this shape are checked in
    # test_kernels_gpu.py::test_gemm_full_size_sampled_rows)
    rng = np.random.default_rng(2)
    D, B = 4096, 8192
    ps = []
    for _ in range(6):
        w = (rng.standard_normal((D, D), dtype=np.float32) / np.float32(64.0))
        ps += [TS.Tensor.from_slice(w, w.shape).with_requires_grad(),
               TS.Tensor.zeros([D]).with_requires_grad()]
    x = TS.Tensor.from_slice(rng.standard_normal((B, D), dtype=np.float32), [B, D])
    t = TS.Tensor.from_slice(rng.standard_normal((B, D), dtype=np.float32), [B, D])
    opt = TS.Adam.new()
    opt.add_parameters(ps)
    losses = []
    for _ in range(2):
        loss = _mlp(TS, x, t, ps)
        loss.backward()
        opt.step(ps)
        opt.zero_grad(ps)
        losses.append(loss.value())
    assert all(np.isfinite(losses)) and losses[1] < losses[0]
