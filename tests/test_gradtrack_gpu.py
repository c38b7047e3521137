"""End-to-end parity of the training step on the GPU (libts_gradtrack.so over
libts_hip.so) against the oracle's restatement of the reference
(oracle/gradtrack.py), on the BASELINE configurations.

Bars: elementwise ops, ReLU masks and Adam arithmetic bit-exact; matmul-derived
gradients and reductions <= 1e-4 normwise relative error (max|d| / max|ref|);
parameters after many Adam steps <= 1e-4 normwise L2 relative error (see
_train_both), with ReLU masks teacher-forced where a pre-activation is within
rounding of zero (see _relu_both).  Loss values are
compared with the f64 value (the reference's own sequential fp32 sum drifts,
see tests/test_oracle.py)."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_bits_equal, golden, max_rel, normal, rel_l2, uniform

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


# ---- teacher-forced ReLU masks -------------------------------------------------------------------
#
# Two correct fp32 GEMMs with different summation orders can put a
# pre-activation that lies within rounding of zero on opposite sides of it;
# the ReLU backward then routes an O(1) gradient differently.  The MLP tests
# therefore (1) assert that device and oracle masks differ only where
# |z| <= 1e-5 * max|z| and (2) hand the device's masks to the oracle's ReLU
# backward, so every remaining difference is arithmetic.

def _relu_both(z, zo, stats):
    zg = z.data()
    mism = (zg > 0) != (zo.data > 0)
    if mism.any():
        scale = float(np.max(np.abs(zo.data)))
        assert np.all(np.abs(zo.data[mism]) <= 1e-5 * scale), "mask differs away from zero"
        stats["flips"] = stats.get("flips", 0) + int(mism.sum())
    return z.relu(), zo.relu(mask_source=zg)


def _mlp_both(xd, td, pd, xo, to, po, stats, readme=False):
    h, ho = xd, xo
    n = len(pd) // 2
    for i in range(n):
        z = h.matmul(pd[2 * i]).add_tensor(pd[2 * i + 1])
        zo = ho.matmul(po[2 * i]).add_tensor(po[2 * i + 1])
        if i < n - 1 or readme:
            h, ho = _relu_both(z, zo, stats)
        else:
            h, ho = z, zo
    if readme:
        return h.sum(), ho.sum()
    return h.sub_tensor(td).pow_scalar(2.0).mean(), ho.sub_tensor(to).pow_scalar(2.0).mean()


def _train_both(TS, G, ws, x, t, steps, readme=False, lr=1e-3):
    pd = [TS.Tensor.from_slice(v, v.shape).with_requires_grad() for v in ws]
    po = [G.OTensor(v.copy()).with_requires_grad() for v in ws]
    opt, oopt = TS.Adam.with_learning_rate(lr), G.OAdam(lr)
    opt.add_parameters(pd)
    oopt.add_parameters(po)
    xd, xo = TS.Tensor.from_slice(x, x.shape), G.OTensor(x)
    td = TS.Tensor.from_slice(t, t.shape) if t is not None else None
    to = G.OTensor(t) if t is not None else None
    stats = {}
    for step in range(steps):
        loss, lo = _mlp_both(xd, td, pd, xo, to, po, stats, readme)
        loss.backward()
        lo.backward()
        if step == 0:
            for d, o in zip(pd, po):
                assert max_rel(d.grad_by_value().data(), o.grad_by_value()) <= 1e-4
        exact = lo.value()
        assert abs(loss.value() - exact) <= 1e-4 * abs(exact), (step, loss.value(), exact)
        opt.step(pd)
        opt.zero_grad(pd)
        oopt.step(po)
        oopt.zero_grad(po)
    # Parameters after several steps: normwise L2.  Adam's first steps move
    # each element by about lr * sign(g); an element whose gradient cancels to
    # the GEMM's rounding level has no fp32-determined sign, so a single
    # element may differ by up to ~lr per step between two correct GEMMs.
    worst = 0.0
    for d, o in zip(pd, po):
        got = d.data()
        print(f"[train {steps} steps] max_rel {max_rel(got, o.data):.2e} rel_l2 {rel_l2(got, o.data):.2e}")
        worst = max(worst, rel_l2(got, o.data))
    print(f"[train] mask flips conditioned on: {stats.get('flips', 0)}")
    return worst


# ---- config 1: README quick-start step ---------------------------------------------------------

def test_config1_readme_step(TS, G):
    # x[32,784] ~ N(0,1), W[784,128] ~ N(0,1), b = 0; y = relu(x.W + b); loss = sum(y); 100 Adam steps
    x = normal((32, 784), 0)
    ws = [normal((784, 128), 1), np.zeros(128, np.float32)]
    assert _train_both(TS, G, ws, x, None, 100, readme=True) <= 1e-4


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

def test_adam_step_with_a_parameter_listed_twice(TS, G):
    # adam/mod.rs:1036-1044 updates each listed parameter in turn, so a
    # parameter listed twice is stepped twice with the same step_count
    p0, g = normal(100, 6), normal(100, 7, 0.1)
    p = TS.Tensor.from_slice(p0, [100]).with_requires_grad()
    p.set_grad(TS.Tensor.from_slice(g, [100]))
    opt = TS.Adam.new()
    opt.add_parameter(p)
    po = G.OTensor(p0.copy()).with_requires_grad()
    po.grad = g.copy()
    oopt = G.OAdam()
    oopt.add_parameter(po)
    opt.step([p, p])
    oopt.step([po, po])
    assert_bits_equal(p.data(), po.data, "parameter stepped twice")


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

def _mlp_weights(dims, seed, init):
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
    return ws, rng


def test_config4_mlp(TS, G):
    # batch 1024, 784 -> 1024 -> 10, Kaiming-uniform, MSE; 10 steps against the oracle
    ws, rng = _mlp_weights([784, 1024, 10], 0, "kaiming")
    x = rng.standard_normal((1024, 784)).astype(np.float32)
    t = rng.standard_normal((1024, 10)).astype(np.float32)
    assert _train_both(TS, G, ws, x, t, 10) <= 1e-4


def test_config5_scaled_mlp(TS, G):
    # config 5 structure (6 layers, N(0, 1/fan_in) weights, ReLU on layers 1-5, MSE) at width 256
    ws, rng = _mlp_weights([256] * 7, 1, "normal")
    x = rng.standard_normal((512, 256)).astype(np.float32)
    t = rng.standard_normal((512, 256)).astype(np.float32)
    assert _train_both(TS, G, ws, x, t, 5) <= 1e-4


def _mlp(lib_tensor, x, t, params, relu_last=False):
    h = x
    n = len(params) // 2
    for i in range(n):
        h = h.matmul(params[2 * i]).add_tensor(params[2 * i + 1])
        if i < n - 1 or relu_last:
            h = h.relu()
    return h.sub_tensor(t).pow_scalar(2.0).mean()


def test_config5_full_size_step(TS, oracle):
    # The bench workload at its real size (B = 8192, 6 x 4096^2, ReLU on 1-5,
    # MSE), checked through size-independent properties: sampled output rows
    # against an f64 forward pass, the loss against f64 over the downloaded
    # output, the last bias gradient against 2/n * colsum(y - t) in f64, and
    # Adam's first step, which moves every weight by lr * |g| / (|g| + eps).
    rng = np.random.default_rng(2)
    D, B, L = 4096, 8192, 6
    ws = [rng.standard_normal((D, D), dtype=np.float32) * np.float32(1 / 64) for _ in range(L)]
    x = rng.standard_normal((B, D), dtype=np.float32)
    t = rng.standard_normal((B, D), dtype=np.float32)
    ps = []
    for w in ws:
        ps += [TS.Tensor.from_slice(w, w.shape).with_requires_grad(), TS.Tensor.zeros([D]).with_requires_grad()]
    xd, td = TS.Tensor.from_slice(x, [B, D]), TS.Tensor.from_slice(t, [B, D])
    opt = TS.Adam.new()
    opt.add_parameters(ps)
    h = xd
    for i in range(L):
        h = h.matmul(ps[2 * i]).add_tensor(ps[2 * i + 1])
        if i < L - 1:
            h = h.relu()
    y = h
    loss = y.sub_tensor(td).pow_scalar(2.0).mean()
    loss.backward()
    yg = y.data()
    rows = np.array([0, 1, 4095, 8191])
    hr = x[rows]
    for i, w in enumerate(ws):
        hr = oracle.gemm_f64(hr, w).astype(np.float32)
        if i < L - 1:
            hr = oracle.relu(hr)
    assert max_rel(yg[rows], hr) <= 1e-4
    d = yg.astype(np.float64) - t.astype(np.float64)
    want_loss = float(np.mean(d * d))
    assert abs(loss.value() - want_loss) <= 1e-5 * want_loss
    want_db = 2.0 / (B * D) * d.sum(axis=0)
    assert max_rel(ps[-1].grad_by_value().data(), want_db) <= 1e-4
    g1 = ps[0].grad_by_value().data().astype(np.float64)
    opt.step(ps)
    # first step: m_hat = g and v_hat = g^2 (to a few ulp), so each weight
    # moves by lr * |g| / (|g| + eps); the remaining error is the f32 rounding
    # of the updated weight (|w| < 0.1, ulp <= 7.5e-9)
    moved = np.abs(ps[0].data().astype(np.float64) - ws[0].astype(np.float64))
    expected = 1e-3 * np.abs(g1) / (np.abs(g1) + 1e-8)
    assert float(np.max(np.abs(moved - expected))) <= 2e-8
    opt.zero_grad(ps)


@pytest.mark.gpu
def test_sub_backward_skips_the_unconsumed_negation(TS):
    # gradients go to the recorded inputs by position; with constant targets only
    # the first is consumed, so y - t runs no negation pass, and the gradients
    # match the case where both inputs require them
    n = 4099
    yv, tv = normal(n, 31), normal(n, 32)

    def run(t_grad):
        y = TS.Tensor.from_slice(yv, [n]).with_requires_grad()
        t = TS.Tensor.from_slice(tv, [n])
        if t_grad:
            t = t.with_requires_grad()
        TS.Profile.reset()
        TS.Profile.enable(True)
        y.sub_tensor(t).pow_scalar(2.0).mean().backward()
        TS.Profile.enable(False)
        launches = TS.Profile.read(TS.Profile.ELEMENTWISE)["launches"]
        gy = y.grad_by_value().data()
        gt = t.grad_by_value().data() if t_grad else None
        TS.clear_gradients()
        return launches, gy, gt

    l1, gy1, _ = run(False)
    l2, gy2, gt2 = run(True)
    assert l2 == l1 + 1
    assert_bits_equal(gy1, gy2)
    assert_bits_equal(gt2, -gy2)
    np.testing.assert_allclose(gy1, 2.0 * (yv - tv) / n, rtol=1e-5, atol=1e-9)
