"""Compiled elementwise programs (ts_hip_map_jit_mode): a program run as its
kernel compiled at run time gives the interpreter's bits -- stored values,
the fused sum and the division-by-zero index -- for every op code, with
registers reused, scalar and constant inputs, several outputs and a sum;
and the training-step chains give the same bits compiled or interpreted."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import assert_bits_equal, normal, uniform
from test_map_gpu import R0, _program

pytestmark = pytest.mark.gpu


@pytest.fixture()
def jit():
    from gpu_util import hip
    old = hip.ts_hip_map_jit_mode(1)
    yield hip
    hip.ts_hip_map_jit_mode(old)


def _stats(hip):
    c, f = ctypes.c_size_t(), ctypes.c_size_t()
    hip.ts_hip_map_jit_stats(ctypes.byref(c), ctypes.byref(f))
    return c.value, f.value


def _run(hip, prog_fn, n, outs, reduce):
    """Run the program from prog_fn() (fresh output buffers each time) and
    return the stored values, the sum and the zero index."""
    from gpu_util import Dev, ZeroIndex, hip_check, sync
    bufs = [Dev(n) for _ in range(outs)]
    prog = prog_fn([b.ptr for b in bufs])
    zi = ZeroIndex()
    tail8, tail32 = 8 * (n // 8), 32 * (n // 32)
    if reduce:
        out = Dev(1)
        ws = Dev(hip.ts_hip_map_workspace_floats(n))
        hip_check(hip.ts_hip_map(ctypes.byref(prog), n, tail8, tail32, zi.ptr, out.ptr, 0, ws.ptr, ws.n, None), "map")
    else:
        out = None
        hip_check(hip.ts_hip_map(ctypes.byref(prog), n, tail8, tail32, zi.ptr, None, 0, None, 0, None), "map")
    sync()
    return [b.get() for b in bufs], (out.get()[0] if out else None), zi.value()


CODES = ["add", "sub", "mul", "div", "neg", "relu", "relu_bwd", "add_s", "sub_s", "mul_s", "div_s", "square"]


@pytest.mark.parametrize("n", [4, 1000, 4099 * 4, (1 << 20) + 12])
@pytest.mark.parametrize("reduce", [False, True])
def test_every_op_compiled_equals_interpreted(jit, n, reduce):
    from gpu_util import Dev
    print(f"[jit ops] n={n} reduce={reduce}", flush=True)
    a = normal(n, 1)
    b = uniform(n, 0.5, 2.0, 2) * np.where(np.arange(n) % 3 == 0, -1, 1).astype(np.float32)
    a[:4] = np.array([0.0, -0.0, np.inf, -np.inf], np.float32)
    b[n - 1] = 0.0                                    # a zero divisor in the checked tail
    da, db = Dev.of(a), Dev.of(b)
    s = Dev.of(np.array([1.5], np.float32))
    # every op once, registers reused past their values' last use (dst 5..9
    # in turn), inputs a, b, a scalar s and the constant 2: 12 ops
    ops = []
    for k, code in enumerate(CODES):
        src = (0, 1) if k % 3 == 0 else (R0 + (k - 1) % 5, 1) if k % 3 == 1 else (R0 + (k - 1) % 5, 2)
        flags = 1 if code == "div" else 0
        ops.append((code, src[0], src[1] if code not in ("div_s",) else 0, 0.25 * (k + 1), flags, R0 + k % 5))
    ops.append(("mul", R0 + 1, 3, 0.0, 0, 12))       # times the constant input
    ops.append(("add", 12, R0 + 4, 0.0, 0, 13))

    def prog(ptrs):
        p = _program([da.ptr, db.ptr, s.ptr, None], ops, [(ptrs[0], 12), (ptrs[1], 13), (ptrs[2], R0 + 2)],
                     scalar=1 << 2, reduce_reg=13 if reduce else -1, consts={3: 2.0})
        return p

    jit.ts_hip_map_jit_mode(0)
    want = _run(jit, prog, n, 3, reduce)
    before = _stats(jit)
    jit.ts_hip_map_jit_mode(2)
    got = _run(jit, prog, n, 3, reduce)
    after = _stats(jit)
    assert after[1] == before[1], jit.ts_hip_map_jit_log()
    for i, (u, v) in enumerate(zip(got[0], want[0])):
        assert_bits_equal(u, v, f"output {i}")
    if reduce:
        assert_bits_equal(np.float32(got[1]), np.float32(want[1]), "sum")
    assert got[2] == want[2] == n - 1


def test_shapes_compile_on_their_second_use(jit):
    from gpu_util import Dev, hip_check, sync
    n = 1 << 16
    x = Dev.of(normal(n, 3))
    out = Dev(n)
    # a shape no other test uses: x * 0.375 + 0.625, squared, then negated
    p = _program([x.ptr], [("mul_s", 0, 0, 0.375, 0, 7), ("add_s", 7, 7, 0.625, 0, 9), ("square", 9, 9, 0.0, 0, 3),
                           ("neg", 3, 3, 0.0, 0, 11)], [(out.ptr, 11)])
    jit.ts_hip_map_jit_mode(1)
    c0, f0 = _stats(jit)
    for use in range(3):
        hip_check(jit.ts_hip_map(ctypes.byref(p), n, n, n, None, None, 0, None, 0, None), "map")
        sync()
        c, f = _stats(jit)
        assert f == f0
        assert c == c0 + (0 if use == 0 else 1), use
    v = x.get()
    t = (v * np.float32(0.375)) + np.float32(0.625)
    want = np.float32(0.0) - t * t                    # neg before tail_start: 0 - x
    assert_bits_equal(out.get(), want.astype(np.float32), "compiled")


@pytest.mark.parametrize("n", [1 << 20, (1 << 20) + 13])
def test_training_chain_compiled_equals_interpreted(jit, oracle, n):
    import train_station_amd as T
    a, b = normal(n, 41), normal(n, 42)
    c = uniform(n, 0.5, 2.0, 43)

    def run():
        ta, tb, tc = (T.Tensor.from_slice(v, [n]).with_requires_grad() for v in (a, b, c))
        y = ta.add_tensor(tb).mul_tensor(tc).sub_tensor(ta.div_tensor(tc)).relu()
        loss = y.sum()
        loss.backward()
        out = [np.array([loss.value()], np.float32), y.data(), ta.grad_by_value().data(),
               tb.grad_by_value().data(), tc.grad_by_value().data()]
        T.clear_gradients()
        return out

    jit.ts_hip_map_jit_mode(0)
    want = run()
    jit.ts_hip_map_jit_mode(2)
    got = run()
    for name, u, v in zip(("loss", "y", "ga", "gb", "gc"), got, want):
        assert_bits_equal(u, v, name)
    assert _stats(jit)[1] == 0, jit.ts_hip_map_jit_log()


def test_a_training_loop_compiles_nothing_after_its_warm_up(jit):
    # the step builds the same programs every time (the leaf gradients merge
    # in a fixed order), so a loop with no synchronisation between steps
    # compiles nothing after the warm-up
    import train_station_amd as T
    n = (1 << 20) + 64
    a = T.Tensor.from_slice(normal(n, 51), [n]).with_requires_grad()
    b = T.Tensor.from_slice(normal(n, 52), [n]).with_requires_grad()
    c = T.Tensor.from_slice(uniform(n, 0.5, 2.0, 53), [n]).with_requires_grad()

    def step():
        loss = a.add_tensor(b).mul_tensor(c).sub_tensor(a.div_tensor(c)).relu().sum()
        loss.backward()
        T.clear_gradients()

    jit.ts_hip_map_jit_mode(1)
    for _ in range(3):
        step()
    T.synchronize()
    before = _stats(jit)
    for _ in range(60):
        step()
    T.synchronize()
    assert _stats(jit) == before
