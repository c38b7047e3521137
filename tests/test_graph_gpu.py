"""Step graphs: one training step recorded as a HIP graph and replayed
(ts_step_graph_*).  N replays must give the bits of N eager steps of the same
loop: the same kernels in the same order, Adam's bias corrections following
the step count (adam/mod.rs:524-531 via the device table), and the
optimizer's counters advancing with the replays.  Also: the buffers a graph
uses stay reserved while other work allocates, errors inside a recording
leave the library usable, and AMSGrad's first step cannot be recorded.
"""
from __future__ import annotations

import gc

import numpy as np
import pytest

from conftest import assert_bits_equal

pytestmark = pytest.mark.gpu


@pytest.fixture
def T():
    import train_station_amd as T
    yield T
    if T.recording():
        T.native_gradtrack.ts_step_graph_abort()
    T.set_fusion(True)
    T.clear_gradients()


def _model(T, widths, batch, seed, readme=False):
    rng = np.random.default_rng(seed)
    ps = []
    for i in range(len(widths) - 1):
        w = (rng.standard_normal((widths[i], widths[i + 1])) / np.sqrt(widths[i])).astype(np.float32)
        b = (0.1 * rng.standard_normal(widths[i + 1])).astype(np.float32)
        ps += [T.Tensor.from_slice(w, w.shape).with_requires_grad(),
               T.Tensor.from_slice(b, b.shape).with_requires_grad()]
    x = T.Tensor.from_slice(rng.standard_normal((batch, widths[0])).astype(np.float32), [batch, widths[0]])
    t = T.Tensor.from_slice(rng.standard_normal((batch, widths[-1])).astype(np.float32), [batch, widths[-1]])
    return ps, x, t


def _step(ps, x, t, opt, readme):
    h = x
    n = len(ps) // 2
    for i in range(n):
        h = h.matmul(ps[2 * i]).add_tensor(ps[2 * i + 1])
        if i < n - 1 or readme:
            h = h.relu()
    loss = h.sum() if readme else h.sub_tensor(t).pow_scalar(2.0).mean()
    loss.backward()
    opt.step(ps)
    opt.zero_grad(ps)
    return loss


CASES = {  # name: widths, batch, readme
    "mlp_c4": ([784, 1024, 10], 1024, False),     # the 1024x10 products: the narrow kernel
    "readme_c1": ([784, 128], 32, True),          # forward and dW split K
    "deep": ([256, 512, 512, 128], 512, False),
}


def _eager(T, case, steps, amsgrad=False):
    widths, batch, readme = CASES[case]
    ps, x, t = _model(T, widths, batch, 11)
    opt = T.Adam.with_config(amsgrad=True) if amsgrad else T.Adam.with_learning_rate(1e-3)
    opt.add_parameters(ps)
    loss = None
    for _ in range(steps):
        loss = _step(ps, x, t, opt, readme)
    return [p.data() for p in ps], loss.value(), opt


@pytest.mark.parametrize("case", sorted(CASES))
@pytest.mark.parametrize("fusion", [True, False])
def test_replays_give_the_bits_of_eager_steps(T, case, fusion):
    T.set_fusion(fusion)
    widths, batch, readme = CASES[case]
    want, want_loss, _ = _eager(T, case, 7)
    print(f"[graph] {case} fusion={fusion}", flush=True)

    ps, x, t = _model(T, widths, batch, 11)
    opt = T.Adam.with_learning_rate(1e-3)
    opt.add_parameters(ps)
    _step(ps, x, t, opt, readme)                       # step 1 eagerly
    before = [p.data() for p in ps]
    with T.StepGraph.record() as g:                   # step 2, recorded, not run
        loss = _step(ps, x, t, opt, readme)
    for a, b in zip(before, [p.data() for p in ps]):  # nothing ran yet
        assert_bits_equal(a, b)
    g.replay(2)                                       # steps 2 and 3
    g.replay(4)                                       # steps 4 .. 7
    got = [p.data() for p in ps]
    for i, (a, b) in enumerate(zip(got, want)):
        assert_bits_equal(a, b, f"param {i} after 7 steps")
    assert loss.value() == want_loss                  # the loss of step 7
    assert opt.step_count() == 7
    for p in ps:
        assert opt.parameter_step(p) == 7
    g.free()


def _other_ops_step(T, leaves, opt):
    # the C2 chain (with division), 3-D broadcasting, a batched product, the
    # activations and axis reductions, all recorded
    a, b, c, w3, s = leaves
    chain = a.add_tensor(b).mul_tensor(c).sub_tensor(a.div_tensor(c)).relu().sum()
    y = w3.matmul(s).sigmoid().tanh()                       # [2,16,24] . [24,8] -> [2,16,8]
    z = y.add_tensor(y.mean_dims([2], True)).softmax(2).log().mean()
    loss = chain.mul_scalar(1e-6).add_tensor(z)
    loss.backward()
    opt.step(leaves)
    opt.zero_grad(leaves)
    return loss


def test_replays_of_other_ops(T):
    def make():
        rng = np.random.default_rng(8)
        n = 4099  # ragged: scalar tails
        vals = [rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32),
                rng.uniform(0.5, 2.0, n).astype(np.float32),
                (0.2 * rng.standard_normal((2, 16, 24))).astype(np.float32),
                (0.2 * rng.standard_normal((24, 8))).astype(np.float32)]
        leaves = [T.Tensor.from_slice(v, list(v.shape)).with_requires_grad() for v in vals]
        opt = T.Adam.with_learning_rate(1e-2)
        opt.add_parameters(leaves)
        return leaves, opt

    leaves, opt = make()
    for _ in range(5):
        want_loss = _other_ops_step(T, leaves, opt).value()
    want = [v.data() for v in leaves]

    leaves, opt = make()
    _other_ops_step(T, leaves, opt)
    with T.StepGraph.record() as g:
        loss = _other_ops_step(T, leaves, opt)
    g.replay(4)
    for i, (v, w) in enumerate(zip(leaves, want)):
        assert_bits_equal(v.data(), w, f"leaf {i}")
    assert loss.value() == want_loss
    assert opt.step_count() == 5
    g.free()


def test_counters_follow_the_replays(T):
    widths, batch, readme = CASES["deep"]
    ps, x, t = _model(T, widths, batch, 3)
    opt = T.Adam.with_learning_rate(1e-3)
    opt.add_parameters(ps)
    with T.StepGraph.record() as g:                   # the very first step, recorded
        _step(ps, x, t, opt, readme)
    assert opt.step_count() == 0                      # a recording runs nothing
    g.replay(1)
    assert opt.step_count() == 1
    g.replay(3)
    assert opt.step_count() == 4
    # an eager step after the replays continues the count
    _step(ps, x, t, opt, readme)
    assert opt.step_count() == 5
    for p in ps:
        assert opt.parameter_step(p) == 5
    g.free()


def test_replays_count_from_the_optimizer_at_replay_time(T):
    # record, 2 replays, 1 eager step, 2 replays: the bits of 5 eager steps
    # (each replay takes its bias corrections from the count the optimizer
    # has when it runs, eager steps in between included)
    widths, batch, readme = CASES["deep"]
    want, want_loss, _ = _eager(T, "deep", 6)
    ps, x, t = _model(T, widths, batch, 11)
    opt = T.Adam.with_learning_rate(1e-3)
    opt.add_parameters(ps)
    _step(ps, x, t, opt, readme)                      # step 1
    with T.StepGraph.record() as g:
        loss = _step(ps, x, t, opt, readme)
    assert opt.step_count() == 1
    g.replay(2)                                       # steps 2, 3
    _step(ps, x, t, opt, readme)                      # step 4, eager
    assert opt.step_count() == 4
    g.replay(2)                                       # steps 5, 6
    assert opt.step_count() == 6
    for p in ps:
        assert opt.parameter_step(p) == 6
    for i, (a, b) in enumerate(zip([p.data() for p in ps], want)):
        assert_bits_equal(a, b, f"param {i} after 6 steps")
    assert loss.value() == want_loss
    g.free()


def test_two_optimizer_steps_in_one_recording(T):
    # each replay runs both recorded steps, as steps 2k+1 and 2k+2
    widths, batch, readme = CASES["deep"]
    want, want_loss, _ = _eager(T, "deep", 6)
    ps, x, t = _model(T, widths, batch, 11)
    opt = T.Adam.with_learning_rate(1e-3)
    opt.add_parameters(ps)
    with T.StepGraph.record() as g:
        _step(ps, x, t, opt, readme)
        loss = _step(ps, x, t, opt, readme)
    assert opt.step_count() == 0
    g.replay(1)
    assert opt.step_count() == 2
    g.replay(2)
    assert opt.step_count() == 6
    for i, (a, b) in enumerate(zip([p.data() for p in ps], want)):
        assert_bits_equal(a, b, f"param {i} after 6 steps")
    assert loss.value() == want_loss
    g.free()


def test_two_graphs_on_one_optimizer(T):
    # a graph for the full batch and one for a short last batch, interleaved
    # with an eager step: the bits of the same steps run eagerly
    widths, batch, readme = CASES["deep"]
    rng = np.random.default_rng(21)
    xs = rng.standard_normal((batch, widths[0])).astype(np.float32)
    ts = rng.standard_normal((batch, widths[-1])).astype(np.float32)
    short = batch // 4
    order = ["full", "full", "short", "eager", "full", "short"]

    def run(recorded):
        ps, _, _ = _model(T, widths, batch, 11)
        x = T.Tensor.from_slice(xs, list(xs.shape))
        t = T.Tensor.from_slice(ts, list(ts.shape))
        xsh = T.Tensor.from_slice(xs[:short].copy(), [short, widths[0]])
        tsh = T.Tensor.from_slice(ts[:short].copy(), [short, widths[-1]])
        opt = T.Adam.with_learning_rate(1e-3)
        opt.add_parameters(ps)
        graphs = {}
        if recorded:
            with T.StepGraph.record() as gf:
                _step(ps, x, t, opt, readme)
            with T.StepGraph.record() as gs:
                _step(ps, xsh, tsh, opt, readme)
            graphs = {"full": gf, "short": gs}
        for kind in order:
            if recorded and kind in graphs:
                graphs[kind].replay(1)
            elif kind == "short":
                _step(ps, xsh, tsh, opt, readme)
            else:
                _step(ps, x, t, opt, readme)
        out = [p.data() for p in ps]
        assert opt.step_count() == len(order)
        for g in graphs.values():
            g.free()
        return out

    want = run(False)
    got = run(True)
    for i, (a, b) in enumerate(zip(got, want)):
        assert_bits_equal(a, b, f"param {i}")


def test_recording_with_gradients_held_is_refused(T):
    # a recorded accumulation would add the same stale gradient on every replay
    widths, batch, readme = CASES["deep"]
    ps, x, t = _model(T, widths, batch, 3)
    h = x
    for i in range(len(ps) // 2):
        h = h.matmul(ps[2 * i]).add_tensor(ps[2 * i + 1])
    h.sub_tensor(t).pow_scalar(2.0).mean().backward()
    with pytest.raises(T.TsError, match="no gradients are held"):
        T.StepGraph.record().__enter__()
    assert not T.recording()
    T.clear_gradients()
    opt = T.Adam.with_learning_rate(1e-3)
    opt.add_parameters(ps)
    with T.StepGraph.record() as g:
        _step(ps, x, t, opt, readme)
    g.replay(1)
    assert opt.step_count() == 1
    g.free()


def test_an_optimizer_step_that_fails_while_recording_takes_its_counts_back(T):
    # the step counts each parameter as it goes; an unlinked parameter late in
    # the list raises, the recording aborts, and every count is as before
    widths, batch, readme = CASES["deep"]
    ps, x, t = _model(T, widths, batch, 5)
    stray = T.Tensor.from_slice(np.ones(4, np.float32), [4]).with_requires_grad()
    opt = T.Adam.with_learning_rate(1e-3)
    opt.add_parameters(ps)
    _step(ps, x, t, opt, readme)
    with pytest.raises(T.TsError, match="linked to optimizer"):
        with T.StepGraph.record():
            h = x
            for i in range(len(ps) // 2):
                h = h.matmul(ps[2 * i]).add_tensor(ps[2 * i + 1])
            h.sub_tensor(t).pow_scalar(2.0).mean().backward()
            opt.step(ps + [stray])
    assert not T.recording()
    assert opt.step_count() == 1
    for p in ps:
        assert opt.parameter_step(p) == 1
    T.clear_gradients()
    # a recorded step whose parameters hold no gradient still counts once per replay
    with T.StepGraph.record() as g:
        opt.step(ps)
    assert opt.step_count() == 1
    g.replay(2)
    assert opt.step_count() == 3
    for p in ps:
        assert opt.parameter_step(p) == 1
    g.free()


def test_first_recorded_step_matches_eager(T):
    widths, batch, readme = CASES["deep"]
    want, want_loss, _ = _eager(T, "deep", 3)
    ps, x, t = _model(T, widths, batch, 11)
    opt = T.Adam.with_learning_rate(1e-3)
    opt.add_parameters(ps)
    with T.StepGraph.record() as g:
        loss = _step(ps, x, t, opt, readme)
    g.replay(3)
    for i, (a, b) in enumerate(zip([p.data() for p in ps], want)):
        assert_bits_equal(a, b, f"param {i}")
    assert loss.value() == want_loss
    g.free()


def test_graph_buffers_stay_reserved(T):
    widths, batch, readme = CASES["deep"]
    want, _, _ = _eager(T, "deep", 4)
    ps, x, t = _model(T, widths, batch, 11)
    opt = T.Adam.with_learning_rate(1e-3)
    opt.add_parameters(ps)
    _step(ps, x, t, opt, readme)
    with T.StepGraph.record() as g:
        _step(ps, x, t, opt, readme)
    T.clear_gradients()
    # eager work between replays allocates buffers of the recorded sizes
    rng = np.random.default_rng(5)
    keep = []
    for shape in ([batch, 512], [512, 512], [batch, 128], [512], [256, 512]):
        v = rng.standard_normal(shape).astype(np.float32)
        keep.append((T.Tensor.from_slice(v, shape).add_scalar(1.0), v + np.float32(1.0)))
    g.replay(1)
    extra = [T.Tensor.from_slice(v, v.shape).mul_scalar(2.0) for _, v in keep]
    g.replay(2)
    for (tt, v), e in zip(keep, extra):
        assert_bits_equal(tt.data(), v)
        assert_bits_equal(e.data(), v * np.float32(2.0))
    for i, (a, b) in enumerate(zip([p.data() for p in ps], want)):
        assert_bits_equal(a, b, f"param {i}")
    del keep, extra
    gc.collect()
    live = T.pool_stats()["live_bytes"]
    g.free()                                          # the recorded step's dropped temporaries were parked
    assert T.pool_stats()["live_bytes"] < live


def test_product_deferred_before_the_recording_stays_reserved(T):
    # a product deferred before the recording and run inside it because
    # Adam::step overwrites its operand (before_write) writes its output on
    # every replay: that block must not be handed to other work when its
    # tensor is dropped
    x = T.Tensor.from_slice(np.ones((256, 192), np.float32), [256, 192])
    w = T.Tensor.from_slice(np.full((192, 256), 0.5, np.float32), [192, 256]).with_requires_grad()
    gw = T.Tensor.from_slice(np.full((192, 256), 0.01, np.float32), [192, 256])
    opt = T.Adam.with_learning_rate(1e-3)
    opt.add_parameter(w)
    h = x.matmul(w)                                    # deferred, not run
    with T.StepGraph.record() as g:
        w.set_grad(gw)
        opt.step([w])                                  # runs h's product first, inside the recording
    del h
    gc.collect()
    other = [T.Tensor.from_slice(np.full((256, 256), 7.0, np.float32), [256, 256]) for _ in range(4)]
    g.replay(3)
    for o in other:
        assert_bits_equal(o.data(), np.full((256, 256), 7.0, np.float32))
    g.free()
    T.clear_gradients()


def test_reading_inside_a_recording_is_refused(T):
    widths, batch, readme = CASES["deep"]
    ps, x, t = _model(T, widths, batch, 2)
    opt = T.Adam.with_learning_rate(1e-3)
    opt.add_parameters(ps)
    with pytest.raises(T.TsError, match="recorded"):
        with T.StepGraph.record():
            loss = _step(ps, x, t, opt, readme)
            loss.value()
    assert not T.recording()
    assert opt.step_count() == 0                      # the aborted step never ran
    # the library works on afterwards, eagerly and recorded
    T.clear_gradients()
    _step(ps, x, t, opt, readme)
    with T.StepGraph.record() as g:
        _step(ps, x, t, opt, readme)
    g.replay(1)
    g.free()


def test_a_graph_freed_unreplayed_leaves_the_counters(T):
    # the recorded step never runs: the optimizer's count returns to its value
    # before the recording, and eager steps after it match an eager-only loop
    widths, batch, readme = CASES["deep"]
    ps, x, t = _model(T, widths, batch, 3)
    ps2, x2, t2 = _model(T, widths, batch, 3)
    opt = T.Adam.with_learning_rate(1e-3)
    opt.add_parameters(ps)
    opt2 = T.Adam.with_learning_rate(1e-3)
    opt2.add_parameters(ps2)
    _step(ps, x, t, opt, readme)
    _step(ps2, x2, t2, opt2, readme)
    with T.StepGraph.record() as g:
        _step(ps, x, t, opt, readme)
    assert opt.step_count() == 1                      # a recording runs nothing
    g.free()
    assert opt.step_count() == 1
    for _ in range(2):
        _step(ps, x, t, opt, readme)
        _step(ps2, x2, t2, opt2, readme)
    assert opt.step_count() == opt2.step_count() == 3
    for p, q in zip(ps, ps2):
        assert_bits_equal(p.data(), q.data())
    T.clear_gradients()


def test_linking_a_parameter_inside_a_recording_is_refused(T):
    # its state's zero fill would rerun on every replay
    widths, batch, readme = CASES["deep"]
    ps, x, t = _model(T, widths, batch, 4)
    opt = T.Adam.with_learning_rate(1e-3)
    opt.add_parameters(ps[:-1])
    with pytest.raises(T.TsError, match="before recording"):
        with T.StepGraph.record():
            opt.add_parameters(ps[-1:])
    assert not T.recording()
    opt.add_parameters(ps[-1:])                       # eagerly, it links
    _step(ps, x, t, opt, readme)
    assert opt.step_count() == 1
    T.clear_gradients()


def test_uploads_inside_a_recording_are_refused(T):
    widths, batch, readme = CASES["deep"]
    ps, x, t = _model(T, widths, batch, 6)
    opt = T.Adam.with_learning_rate(1e-3)
    opt.add_parameters(ps)
    with pytest.raises(T.TsError, match="cannot upload"):
        with T.StepGraph.record():
            T.Tensor.from_slice(np.ones(8, np.float32), [8])
    assert not T.recording()
    with pytest.raises(T.TsError, match="cannot upload"):
        with T.StepGraph.record():
            _step(ps, x, t, opt, readme).data()
    assert opt.step_count() == 0
    T.clear_gradients()


def test_amsgrad_first_step_is_not_recorded(T):
    widths, batch, readme = CASES["deep"]
    ps, x, t = _model(T, widths, batch, 4)
    opt = T.Adam.with_config(amsgrad=True)
    opt.add_parameters(ps)
    with pytest.raises(T.TsError, match="AMSGrad"):
        with T.StepGraph.record():
            _step(ps, x, t, opt, readme)
    assert opt.step_count() == 0
    T.clear_gradients()


def test_amsgrad_replays_after_the_first_step(T):
    widths, batch, readme = CASES["deep"]
    want, _, _ = _eager(T, "deep", 4, amsgrad=True)
    ps, x, t = _model(T, widths, batch, 11)
    opt = T.Adam.with_config(amsgrad=True)
    opt.add_parameters(ps)
    _step(ps, x, t, opt, readme)
    with T.StepGraph.record() as g:
        _step(ps, x, t, opt, readme)
    g.replay(3)
    for i, (a, b) in enumerate(zip([p.data() for p in ps], want)):
        assert_bits_equal(a, b, f"param {i}")
    g.free()
