"""Fused elementwise programs (ts_hip_map) and the host's deferred chains built
on them.  Every op of a program must give the bits of its separate kernel
(the reference's fp32 formula and order: ops/{add,sub,mul,div,relu,pow}.rs,
core/utils.rs:802-871, grad_fn/ops/relu.rs), a fused sum / mean the bits of
ts_hip_sum / ts_hip_mean over the same values, and a recorded chain the bits
of the op-by-op graph, with fusion on and off.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import assert_bits_equal, normal, sum_order_model, uniform

pytestmark = pytest.mark.gpu

SIZES = [1, 7, 1003, (1 << 20) + 5]


def _ffi():
    from train_station_amd import _ffi
    return _ffi


def _program(inputs, ops, outputs, scalar=0, reduce_reg=-1, consts=None):
    """inputs: device pointers; ops: (code name, a, b, imm, flags[, d]) with
    registers numbered as in include/ts_hip.h, op k writing register d
    (default R0 + k, one register per op); outputs: (pointer, register);
    consts: {input index: value} for constant inputs (their pointer unused)."""
    F = _ffi()
    p = F.MapProgram()
    p.n_inputs = len(inputs)
    for k, ptr in enumerate(inputs):
        p.inputs[k] = ptr
    p.scalar_inputs = scalar
    for k, v in (consts or {}).items():
        p.const_inputs |= 1 << k
        p.const_values[k] = v
    p.n_ops = len(ops)
    for k, op in enumerate(ops):
        code, a, b, imm, flags = op[:5]
        p.ops[k] = F.MapOp(F.MAP_CODES[code], a, b, flags, imm, op[5] if len(op) > 5 else R0 + k)
    p.n_outputs = len(outputs)
    for k, (ptr, reg) in enumerate(outputs):
        p.outputs[k] = ptr
        p.output_regs[k] = reg
    p.reduce_reg = reduce_reg
    return p


R0 = 5  # register of op 0 (TS_HIP_MAP_MAX_INPUTS)


def test_register_numbering_follows_the_header():
    assert _ffi().MAP_MAX_INPUTS == R0


@pytest.mark.parametrize("offset", [0, 1])
@pytest.mark.parametrize("n", SIZES)
def test_each_op_matches_its_kernel(n, offset):
    from gpu_util import Dev, ZeroIndex, hip, hip_check, sync
    print(f"[map ops] n={n} offset={offset}", flush=True)
    a = normal(n, 1)
    b = uniform(n, 0.5, 2.0, 2) * np.where(np.arange(n) % 3 == 0, -1, 1).astype(np.float32)
    a[: min(n, 4)] = np.array([0.0, -0.0, np.inf, -np.inf], np.float32)[: min(n, 4)]
    da, db = Dev.of(a, offset), Dev.of(b, offset)
    tail8, tail32 = 8 * (n // 8), 32 * (n // 32)
    zi = ZeroIndex()
    cases = [  # (op, imm, reference launcher)
        ("add", 0.0, lambda o: hip.ts_hip_add(da.ptr, db.ptr, o, n, None)),
        ("sub", 0.0, lambda o: hip.ts_hip_sub(da.ptr, db.ptr, o, n, None)),
        ("mul", 0.0, lambda o: hip.ts_hip_mul(da.ptr, db.ptr, o, n, None)),
        ("div", 0.0, lambda o: hip.ts_hip_div(da.ptr, db.ptr, o, n, tail32, zi.ptr, None)),
        ("neg", 0.0, lambda o: hip.ts_hip_neg(da.ptr, o, n, tail8, None)),
        ("relu", 0.0, lambda o: hip.ts_hip_relu(da.ptr, o, n, None)),
        ("relu_bwd", 0.0, lambda o: hip.ts_hip_relu_backward(da.ptr, db.ptr, o, n, None)),
        ("add_s", 0.37, lambda o: hip.ts_hip_add_scalar(da.ptr, ctypes.c_float(0.37), o, n, None)),
        ("sub_s", 0.37, lambda o: hip.ts_hip_sub_scalar(da.ptr, ctypes.c_float(0.37), o, n, None)),
        ("mul_s", -3.1, lambda o: hip.ts_hip_mul_scalar(da.ptr, ctypes.c_float(-3.1), o, n, None)),
        ("div_s", 7.0, lambda o: hip.ts_hip_div_scalar(da.ptr, ctypes.c_float(7.0), o, n, None)),
        ("square", 0.0, lambda o: hip.ts_hip_pow_scalar(da.ptr, ctypes.c_float(2.0), o, n, None)),
    ]
    for code, imm, ref in cases:
        got, want = Dev(n, offset), Dev(n, offset)
        flags = _ffi().MAP_CHECKED if code == "div" else 0
        prog = _program([da.ptr, db.ptr], [(code, 0, 1, imm, flags)], [(got.ptr, R0)])
        hip_check(hip.ts_hip_map(ctypes.byref(prog), n, tail8, tail32, zi.ptr, None, 0, None, 0, None), code)
        hip_check(ref(want.ptr), code)
        sync()
        assert_bits_equal(got.get(), want.get(), f"{code} n={n}")


def test_chain_multi_output_and_scalar_input():
    # the config-2 backward as one program over (y, go, c, a, t1), go one value
    # for every element: the three gradients equal the separate kernels' chain
    from gpu_util import Dev, hip, hip_check, sync
    n = 4099
    y, c, a, t1 = normal(n, 3), uniform(n, 0.5, 2.0, 4), normal(n, 5), normal(n, 6)
    go = np.array([1.0], np.float32)
    dy, dc, da, dt, dgo = (Dev.of(v) for v in (y, c, a, t1, go))
    tail8, tail32 = 8 * (n // 8), 32 * (n // 32)
    r = R0  # op k writes register r + k
    ops = [("relu_bwd", 0, 1, 0.0, 0),              # r+0  g4 = y > 0 ? go : 0
           ("neg", r, r, 0.0, 0),                   # r+1  g3
           ("div", r + 1, 2, 0.0, 1),               # r+2  g3 / c
           ("mul", r, 2, 0.0, 0),                   # r+3  g4 * c
           ("add", r + 2, r + 3, 0.0, 0),           # r+4  ga
           ("mul", r + 1, 3, 0.0, 0),               # r+5  g3 * a
           ("mul", 2, 2, 0.0, 0),                   # r+6  c * c
           ("div", r + 5, r + 6, 0.0, 1),           # r+7
           ("neg", r + 7, r + 7, 0.0, 0),           # r+8  gc_1
           ("mul", r, 4, 0.0, 0),                   # r+9  gc_2 = g4 * t1
           ("add", r + 8, r + 9, 0.0, 0)]           # r+10 gc
    ga, gb, gc = Dev(n), Dev(n), Dev(n)
    prog = _program([dy.ptr, dgo.ptr, dc.ptr, da.ptr, dt.ptr], ops,
                    [(ga.ptr, r + 4), (gb.ptr, r + 3), (gc.ptr, r + 10)], scalar=1 << 1)
    hip_check(hip.ts_hip_map(ctypes.byref(prog), n, tail8, tail32, None, None, 0, None, 0, None), "map")
    # the same through the separate kernels
    ones = Dev.of(np.ones(n, np.float32))
    g4, g3, q, qb, wa, wc = (Dev(n) for _ in range(6))
    hip_check(hip.ts_hip_relu_backward(dy.ptr, ones.ptr, g4.ptr, n, None))
    hip_check(hip.ts_hip_neg(g4.ptr, g3.ptr, n, tail8, None))
    hip_check(hip.ts_hip_div_backward(g3.ptr, da.ptr, dc.ptr, q.ptr, qb.ptr, n, tail8, tail32, None, None))
    hip_check(hip.ts_hip_mul_backward(g4.ptr, dt.ptr, dc.ptr, wa.ptr, wc.ptr, n, None))
    want_a, want_c = Dev(n), Dev(n)
    hip_check(hip.ts_hip_add(q.ptr, wa.ptr, want_a.ptr, n, None))
    hip_check(hip.ts_hip_add(qb.ptr, wc.ptr, want_c.ptr, n, None))
    sync()
    assert_bits_equal(ga.get(), want_a.get(), "ga")
    assert_bits_equal(gb.get(), wa.get(), "gb")
    assert_bits_equal(gc.get(), want_c.get(), "gc")


# up to 16 first-pass workgroups (n <= 16384) ts_hip_sum runs both passes in
# one workgroup; the fused sum always takes two: the same bits either way,
# the partition's order
@pytest.mark.parametrize("n", [1, 4, 5, 1024, 4096, 10240, 12288, 16384, 16385, 100003, 1 << 22, (1 << 22) + 13,
                               1 << 26])
@pytest.mark.parametrize("mean", [0, 1])
def test_fused_sum_has_the_bits_of_ts_hip_sum(n, mean):
    from gpu_util import Dev, hip, hip_check, sync
    y, t = normal(n, 7), normal(n, 8)
    dy, dt = Dev.of(y), Dev.of(t)
    d, out = Dev(n), Dev(1)
    ws = hip.ts_hip_map_workspace_floats(n)
    dws = Dev(ws + 2)
    # d = y - t stored; sum / mean of d * d without storing it
    prog = _program([dy.ptr, dt.ptr], [("sub", 0, 1, 0.0, 0), ("square", R0, R0, 0.0, 0)], [(d.ptr, R0)],
                    reduce_reg=R0 + 1)
    hip_check(hip.ts_hip_map(ctypes.byref(prog), n, 8 * (n // 8), 32 * (n // 32), None, out.ptr, mean, dws.ptr, ws,
                             None), "map")
    sq, want = Dev(n), Dev(1)
    hip_check(hip.ts_hip_sub(dy.ptr, dt.ptr, sq.ptr, n, None))
    hip_check(hip.ts_hip_pow_scalar(sq.ptr, ctypes.c_float(2.0), sq.ptr, n, None))
    sw = hip.ts_hip_sum_workspace_floats(n)
    dsw = Dev(sw + 2)
    fn = hip.ts_hip_mean if mean else hip.ts_hip_sum
    hip_check(fn(sq.ptr, n, want.ptr, dsw.ptr, sw, None))
    sync()
    assert_bits_equal(out.get(), want.get(), f"fused {'mean' if mean else 'sum'} n={n}")
    assert_bits_equal(d.get(), (y - t).astype(np.float32), "stored difference")
    # and both have the partition's bits
    dd = (y - t).astype(np.float32)
    model = sum_order_model((dd * dd).astype(np.float32), mean=bool(mean))
    assert_bits_equal(out.get(), np.array([model], np.float32), f"partition order n={n}")


def test_fused_sum_with_longer_runs():
    # past 2^28 elements a first-pass thread of the sum's partition takes five
    # float4 groups: the fused sum keeps ts_hip_sum's bits and the model's
    from gpu_util import Dev, hip, hip_check, sync
    n = (1 << 28) + 8
    print(f"[map fused sum] n={n}", flush=True)
    y = normal(n, 9)
    dy, d, out = Dev.of(y), Dev(n), Dev(1)
    ws = hip.ts_hip_map_workspace_floats(n)
    dws = Dev(ws + 2)
    # d = y * y stored; the sum of d
    prog = _program([dy.ptr], [("square", 0, 0, 0.0, 0)], [(d.ptr, R0)], reduce_reg=R0)
    hip_check(hip.ts_hip_map(ctypes.byref(prog), n, 8 * (n // 8), 32 * (n // 32), None, out.ptr, 0, dws.ptr, ws,
                             None), "map")
    want = Dev(1)
    sw = hip.ts_hip_sum_workspace_floats(n)
    dsw = Dev(sw + 2)
    hip_check(hip.ts_hip_sum(d.ptr, n, want.ptr, dsw.ptr, sw, None), "sum")
    sync()
    assert_bits_equal(out.get(), want.get(), "fused sum vs ts_hip_sum")
    assert_bits_equal(out.get(), np.array([sum_order_model((y * y).astype(np.float32))], np.float32), "model")


@pytest.mark.parametrize("n", [7, 4099])
def test_constant_inputs_match_a_filled_buffer(n):
    # a constant input is the value ts_hip_fill writes: every op reading it,
    # on either side, has the bits of its separate kernel reading a buffer
    # filled with it (NEG's body / tail rule included)
    from gpu_util import Dev, hip, hip_check, sync
    print(f"[map constant inputs] n={n}", flush=True)
    a = normal(n, 11)
    a[: 3] = np.array([0.0, -0.0, np.inf], np.float32)
    da = Dev.of(a)
    tail8, tail32 = 8 * (n // 8), 32 * (n // 32)
    binary = {"add": hip.ts_hip_add, "sub": hip.ts_hip_sub, "mul": hip.ts_hip_mul,
              "div": lambda x, y, o, m, s: hip.ts_hip_div(x, y, o, m, tail32, None, s),
              "relu_bwd": hip.ts_hip_relu_backward}
    for v in (1.0, -0.0, 0.0, 0.625, -3.0):
        filled = Dev(n)
        hip_check(hip.ts_hip_fill(filled.ptr, ctypes.c_float(v), n, None))
        for code, ref in binary.items():
            for side in (0, 1):  # the constant as operand a (side 0) or b
                got, want = Dev(n), Dev(n)
                ins = [None, da.ptr] if side == 0 else [da.ptr, None]
                k = side  # the constant's register
                prog = _program(ins, [(code, 0, 1, 0.0, 0)], [(got.ptr, R0)], consts={k: v})
                hip_check(hip.ts_hip_map(ctypes.byref(prog), n, tail8, tail32, None, None, 0, None, 0, None), code)
                x, y = (filled, da) if side == 0 else (da, filled)
                hip_check(ref(x.ptr, y.ptr, want.ptr, n, None))
                sync()
                assert_bits_equal(got.get(), want.get(), f"{code} constant {v} as operand {'ab'[side]}")
        got, want = Dev(n), Dev(n)
        prog = _program([None], [("neg", 0, 0, 0.0, 0)], [(got.ptr, R0)], consts={0: v})
        hip_check(hip.ts_hip_map(ctypes.byref(prog), n, tail8, tail32, None, None, 0, None, 0, None), "neg")
        hip_check(hip.ts_hip_neg(filled.ptr, want.ptr, n, tail8, None))
        sync()
        assert_bits_equal(got.get(), want.get(), f"neg of constant {v}")


@pytest.mark.parametrize("n", [1, 4096, 4099, 100003])
def test_program_of_a_constant_input(n):
    # a constant input (the deferred gradient seed), stored as it is and
    # scaled, the scaled value summed: no input buffer at all
    from gpu_util import Dev, hip, hip_check, sync
    print(f"[map const] n={n}", flush=True)
    stored, both, out = Dev(n), Dev(n), Dev(1)
    ws = hip.ts_hip_map_workspace_floats(n)
    dws = Dev(ws + 2)
    prog = _program([None], [("mul_s", 0, 0, 0.25, 0)], [(stored.ptr, R0), (both.ptr, 0)], reduce_reg=R0,
                    consts={0: 1.5})
    hip_check(hip.ts_hip_map(ctypes.byref(prog), n, 8 * (n // 8), 32 * (n // 32), None, out.ptr, 0, dws.ptr, ws,
                             None), "map")
    filled, want = Dev(n), Dev(1)
    hip_check(hip.ts_hip_fill(filled.ptr, ctypes.c_float(0.375), n, None))
    sw = hip.ts_hip_sum_workspace_floats(n)
    dsw = Dev(sw + 2)
    hip_check(hip.ts_hip_sum(filled.ptr, n, want.ptr, dsw.ptr, sw, None))
    sync()
    assert_bits_equal(stored.get(), np.full(n, 0.375, np.float32), "stored")
    assert_bits_equal(both.get(), np.full(n, 1.5, np.float32), "the constant itself")
    assert_bits_equal(out.get(), want.get(), "sum")


def test_division_by_zero_index_is_reported_as_by_ts_hip_div():
    from gpu_util import Dev, ZeroIndex, hip, hip_check, sync
    n = 100
    a = np.ones(n, np.float32)
    b = np.ones(n, np.float32)
    b[5] = 0.0   # inside the unchecked body (< 96)
    b[97] = 0.0  # checked tail
    da, db, out = Dev.of(a), Dev.of(b), Dev(n)
    zi = ZeroIndex()
    prog = _program([da.ptr, db.ptr], [("div", 0, 1, 0.0, 1)], [(out.ptr, R0)])
    hip_check(hip.ts_hip_map(ctypes.byref(prog), n, 96, 96, zi.ptr, None, 0, None, 0, None))
    sync()
    assert zi.value() == 97
    zi.reset()
    prog = _program([da.ptr, db.ptr], [("div", 0, 1, 0.0, 0)], [(out.ptr, R0)])  # unchecked
    hip_check(hip.ts_hip_map(ctypes.byref(prog), n, 96, 96, zi.ptr, None, 0, None, 0, None))
    sync()
    assert zi.value() is None
    assert np.isinf(out.get()[5]) and np.isinf(out.get()[97])


def test_bad_programs_are_refused():
    from gpu_util import Dev, hip
    d = Dev(16)
    bad = [
        _program([d.ptr], [("add", 0, R0 + 1, 0.0, 0)], [(d.ptr, R0)]),    # reads a later register
        _program([], [], [(d.ptr, 0)]),                                     # stores an absent input
        _program([None], [("neg", 0, 0, 0.0, 0)], [(d.ptr, R0)]),          # no buffer, not constant
        _program([d.ptr], [("add", 0, 3, 0.0, 0)], [(d.ptr, R0)]),         # input register past n_inputs
        _program([d.ptr], [("add", 0, 0, 0.0, 0)], [(d.ptr, R0 + 1)]),     # output of no op
        _program([d.ptr], [("add", 0, 0, 0.0, 0)], []),                    # nothing stored, no sum
        _program([d.ptr], [("add", 0, 0, 0.0, 0, 16)], [(d.ptr, 0)]),      # writes past the register file
        _program([d.ptr], [("add", 0, 0, 0.0, 0, 7), ("neg", R0, R0, 0.0, 0, 8)], [(d.ptr, 8)]),  # reads an unwritten register
    ]
    for p in bad:
        assert hip.ts_hip_map(ctypes.byref(p), 16, 16, 0, None, None, 0, None, 0, None) == 100001
    p = _program([d.ptr], [("add", 0, 0, 0.0, 0)], [(d.ptr, R0)])
    p.ops[0].code = 12                                                   # no such op
    assert hip.ts_hip_map(ctypes.byref(p), 16, 16, 0, None, None, 0, None, 0, None) == 100001
    p = _program([d.ptr], [("add", 0, 0, 0.0, 0)], [(d.ptr, R0)], reduce_reg=2)  # sums an absent input
    out = Dev(1)
    assert hip.ts_hip_map(ctypes.byref(p), 16, 16, 0, None, out.ptr, 0, d.ptr, 16, None) == 100001
    p = _program([d.ptr], [("add", 0, 0, 0.0, 0)], [(d.ptr, R0)], reduce_reg=R0)
    out = Dev(1)
    assert hip.ts_hip_map(ctypes.byref(p), 16, 16, 0, None, out.ptr, 0, None, 0, None) == 100003  # no workspace


# ---- deferred chains through the handle API ------------------------------------------------------

@pytest.fixture
def T():
    import train_station_amd as T
    yield T
    T.set_fusion(True)
    T.clear_gradients()


def _chain(T, a, b, c, n):
    ta, tb, tc = (T.Tensor.from_slice(v, [n]).with_requires_grad() for v in (a, b, c))
    y = ta.add_tensor(tb).mul_tensor(tc).sub_tensor(ta.div_tensor(tc)).relu()
    loss = y.sum()
    loss.backward()
    out = (loss.value(), y.data(), ta.grad_by_value().data(), tb.grad_by_value().data(),
           tc.grad_by_value().data())
    T.clear_gradients()
    return out


@pytest.mark.parametrize("n", [1003, (1 << 20) + 13])
def test_chain_bits_with_fusion_on_and_off(T, oracle, n):
    a, b = normal(n, 11), normal(n, 12)
    c = uniform(n, 0.5, 2.0, 13)
    T.set_fusion(True)
    on = _chain(T, a, b, c, n)
    T.set_fusion(False)
    off = _chain(T, a, b, c, n)
    assert on[0] == off[0], "loss"
    for name, u, v in zip(("y", "ga", "gb", "gc"), on[1:], off[1:]):
        assert_bits_equal(u, v, name)


def _chain_profiled(T, ta, tb, tc, read_loss_first):
    T.synchronize()
    T.Profile.reset()
    T.Profile.enable(True)
    y = ta.add_tensor(tb).mul_tensor(tc).sub_tensor(ta.div_tensor(tc)).relu()
    loss = y.sum()
    first = loss.value() if read_loss_first else None
    loss.backward()
    T.synchronize()
    T.Profile.enable(False)
    ew = T.Profile.read(T.Profile.ELEMENTWISE)
    red = T.Profile.read(T.Profile.REDUCTION)
    out = (loss.value(), y.data(), ta.grad_by_value().data(), tb.grad_by_value().data(),
           tc.grad_by_value().data())
    assert first is None or first == out[0]
    assert_bits_equal(loss.grad().data(), np.ones(1, np.float32), "seed")  # still ones when read
    T.clear_gradients()
    return ew, red, out


def test_chain_runs_as_one_fused_pass(T, oracle):
    # the loss not read before backward: one pass reads a, b, c, recomputes the
    # forward values, writes the three gradients and adds y up into the loss
    # (the seed, ones, a constant of it): 12 B read + 12 B written per element,
    # the fused floor.  Read before backward: a forward pass with the sum
    # (storing y and a + b, held for the backward) and a backward pass, 20 + 28
    # B.  Both give every value the bits of the op-by-op run.
    n = 1 << 20
    a, b = normal(n, 21), normal(n, 22)
    c = uniform(n, 0.5, 2.0, 23)
    T.set_fusion(True)
    ta, tb, tc = (T.Tensor.from_slice(v, [n]).with_requires_grad() for v in (a, b, c))
    ew, red, one = _chain_profiled(T, ta, tb, tc, False)
    assert red["launches"] == 0
    assert ew["launches"] == 1, ew                      # the fused pass (y is recomputed when read after)
    assert ew["work"] / n == 24.0
    ew, red, two = _chain_profiled(T, ta, tb, tc, True)
    assert red["launches"] == 0
    assert ew["launches"] == 2, ew                      # forward pass, backward pass
    assert ew["work"] / n == 20.0 + 28.0
    for name, u, v in zip(("loss", "y", "ga", "gb", "gc"), one, two):
        assert_bits_equal(u, v, name)
    T.set_fusion(False)
    _, _, off = _chain_profiled(T, ta, tb, tc, False)
    for name, u, v in zip(("loss", "y", "ga", "gb", "gc"), one, off):
        assert_bits_equal(u, v, name + " (fusion off)")


def test_chain_pass_moves_the_fused_floor(T):
    n = 1 << 20
    a, b = normal(n, 24), normal(n, 25)
    c = uniform(n, 0.5, 2.0, 26)
    T.set_fusion(True)
    ta, tb, tc = (T.Tensor.from_slice(v, [n]).with_requires_grad() for v in (a, b, c))
    T.synchronize()
    T.Profile.reset()
    T.Profile.enable(True)
    loss = ta.add_tensor(tb).mul_tensor(tc).sub_tensor(ta.div_tensor(tc)).relu().sum()
    loss.backward()
    T.synchronize()
    T.Profile.enable(False)
    ew = T.Profile.read(T.Profile.ELEMENTWISE)
    assert ew["launches"] == 1, ew
    assert ew["work"] / n == 24.0
    exact = float(np.sum(oracle_chain_y(a, b, c), dtype=np.float64))
    assert abs(loss.value() - exact) <= 1e-6 * abs(exact)
    T.clear_gradients()


def oracle_chain_y(a, b, c):
    import oracle as O
    return O.relu(O.sub(O.mul(O.add(a, b), c), O.div(a, c)))


@pytest.mark.parametrize("op", ["add", "sub", "mul", "div"])
@pytest.mark.parametrize("loss", ["sum", "mean"])
@pytest.mark.parametrize("relu", [False, True])
def test_seeded_gradients_equal_the_unfused_ones(T, op, loss, relu):
    # backward(None) seeds a deferred constant, an input of the backward
    # formulas' pass with no buffer: the gradients have the bits of the
    # op-by-op sequence with a stored seed (fusion off)
    n = 4099
    av, bv = normal(n, 31), uniform(n, 0.5, 2.0, 32)

    def run(fused):
        T.set_fusion(fused)
        a, b = (T.Tensor.from_slice(v, [n]).with_requires_grad() for v in (av, bv))
        y = getattr(a, f"{op}_tensor")(b)
        if relu:
            y = y.relu()
        getattr(y, loss)().backward()
        out = [a.grad_by_value().data(), b.grad_by_value().data()]
        T.clear_gradients()
        return out

    off = run(False)
    on = run(True)
    for name, u, v in zip(("ga", "gb"), on, off):
        assert_bits_equal(u, v, f"{op} {loss} relu={relu} {name}")
