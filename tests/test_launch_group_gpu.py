"""Launch groups (ts_hip_launch_group_begin / _end): products held between
the two calls run after them with the bits of the same calls made one by one.
Config 4's last matmul backward (grad_fn/ops/matmul.rs:68-80: dW = H1^T . dY
and dX = dY . W2^T, here with the MSE's 2 * d * (1/n) applied to d as it is
loaded, the bias gradient's column sums and the loss in dW's launch, and
relu's backward mask in dX's store) runs as ONE launch of the pair kernel;
other sets of products run as issued, and any other work on the stream runs
what is held first.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import assert_bits_equal, normal, uniform

pytestmark = pytest.mark.gpu

XF_MUL_S, XF_SQUARE = 2, 8
MSE_XF = ((XF_MUL_S, 2.0), (XF_MUL_S, 1.0 / 10240))


def _xf(*ops):
    from train_station_amd._ffi import OperandXf
    x = OperandXf()
    x.n_ops = len(ops)
    for i, (code, imm) in enumerate(ops):
        x.code[i] = code
        x.imm[i] = imm
    return x


def _launches(fn):
    """Runs fn inside a kernel timing window: the number of kernels it launched."""
    from train_station_amd._ffi import hip, hip_check
    start, stop = ctypes.c_void_p(), ctypes.c_void_p()
    hip_check(hip.ts_hip_event_create(ctypes.byref(start)))
    hip_check(hip.ts_hip_event_create(ctypes.byref(stop)))
    hip_check(hip.ts_hip_timing_begin(start, stop))
    fn()
    kernels = ctypes.c_int()
    hip_check(hip.ts_hip_timing_end(ctypes.byref(kernels)))
    hip_check(hip.ts_hip_device_synchronize())
    hip_check(hip.ts_hip_event_destroy(start))
    hip_check(hip.ts_hip_event_destroy(stop))
    return kernels.value


class _Layer:
    """Config 4's second layer: H1 [1024, 1024] (relu output, the mask), d =
    y - t [1024, 10], W2 [1024, 10]; dW2 = H1^T . xf(d) with db2 and the loss,
    dX2 = xf(d) . W2^T masked by H1 > 0."""

    def __init__(self, seed, transforms):
        from gpu_util import Dev
        self.B, self.I, self.O = 1024, 1024, 10
        h = np.maximum(normal((self.B, self.I), seed), 0.0)
        self.h, self.d, self.w = Dev.of(h), Dev.of(normal((self.B, self.O), seed + 1)), \
            Dev.of(uniform((self.I, self.O), -0.1, 0.1, seed + 2))
        self.xd = _xf(*MSE_XF) if transforms else None
        self.xs = _xf((XF_SQUARE, 0.0)) if transforms else None

    def outputs(self):
        from gpu_util import Dev
        return Dev(self.I * self.O), Dev(self.O), Dev(1), Dev(self.B * self.I)

    def dw(self, out):
        from train_station_amd._ffi import hip
        dw, db, loss, _ = out
        return hip.ts_hip_gemm_colsum_bsum(1, self.I, self.O, self.B, self.h.ptr, self.I, None, self.d.ptr,
                                           ctypes.byref(self.xd) if self.xd else None, dw.ptr, self.O, db.ptr,
                                           ctypes.byref(self.xs) if self.xs else None, loss.ptr, 1, None)

    def dx(self, out):
        from train_station_amd._ffi import hip
        dx = out[3]
        return hip.ts_hip_gemm_fused_xf(0, 1, self.B, self.I, self.O, self.d.ptr, self.O,
                                        ctypes.byref(self.xd) if self.xd else None, self.w.ptr, self.O, None, None,
                                        0, self.h.ptr, dx.ptr, self.I, None, 0, None)


def _same(got, want, what):
    for g, w, name in zip(got, want, ("dW", "db", "loss", "dX")):
        assert_bits_equal(g.get(), w.get(), f"{what}: {name}")


@pytest.mark.parametrize("transforms", [True, False])
def test_config4_backward_pair_runs_as_one_launch(transforms):
    from train_station_amd._ffi import hip, hip_check
    print(f"[group] config-4 pair, transforms={transforms}", flush=True)
    for call, seed in enumerate((5, 41)):  # two groups in a row
        layer = _Layer(seed, transforms)
        want = layer.outputs()
        hip_check(layer.dw(want))
        hip_check(layer.dx(want))
        got = layer.outputs()

        def grouped():
            hip_check(hip.ts_hip_launch_group_begin(None))
            hip_check(layer.dx(got))
            hip_check(layer.dw(got))
            hip_check(hip.ts_hip_launch_group_end(None))

        assert _launches(grouped) == 1
        _same(got, want, f"group {call}")
        # and one by one (no group) they are two launches
        again = layer.outputs()
        assert _launches(lambda: (hip_check(layer.dw(again)), hip_check(layer.dx(again)))) == 2
        _same(again, want, f"ungrouped {call}")


def test_work_between_begin_and_end_runs_the_held_products_first():
    from gpu_util import Dev
    from train_station_amd._ffi import hip, hip_check
    layer = _Layer(7, True)
    want = layer.outputs()
    hip_check(layer.dw(want))
    hip_check(layer.dx(want))
    got = layer.outputs()
    copy = Dev(layer.I * layer.O)

    def grouped():
        hip_check(hip.ts_hip_launch_group_begin(None))
        hip_check(layer.dw(got))
        # the copy reads dW: the held product runs before it
        hip_check(hip.ts_hip_copy(got[0].ptr, copy.ptr, layer.I * layer.O, None))
        hip_check(layer.dx(got))
        hip_check(hip.ts_hip_launch_group_end(None))

    assert _launches(grouped) == 2  # dW (run by the copy, which launches no kernel), then dX
    _same(got, want, "with a copy inside")
    assert_bits_equal(copy.get(), want[0].get(), "copy of the held product")


def test_three_products_and_pairs_the_library_does_not_build_run_as_issued():
    from gpu_util import Dev
    from train_station_amd._ffi import hip, hip_check
    layer = _Layer(9, True)
    want = layer.outputs()
    hip_check(layer.dw(want))
    hip_check(layer.dx(want))
    # a third product (the first layer's narrow forward of another width): launched after the two held
    M, N, K = 512, 12, 300
    a, b = Dev.of(normal((M, K), 3)), Dev.of(normal((K, N), 4))
    c_want, c_got = Dev(M * N), Dev(M * N)
    n3 = _launches(lambda: hip_check(hip.ts_hip_gemm(0, 0, M, N, K, a.ptr, K, b.ptr, N, c_want.ptr, N, None)))
    got = layer.outputs()

    def three():
        hip_check(hip.ts_hip_launch_group_begin(None))
        hip_check(layer.dw(got))
        hip_check(layer.dx(got))
        hip_check(hip.ts_hip_gemm(0, 0, M, N, K, a.ptr, K, b.ptr, N, c_got.ptr, N, None))
        hip_check(hip.ts_hip_launch_group_end(None))

    assert _launches(three) == 2 + n3
    _same(got, want, "three products")
    assert_bits_equal(c_got.get(), c_want.get(), "third product")
    # a narrow product and another: no pair kernel for them, launched as issued
    got2 = layer.outputs()
    c2 = Dev(M * N)

    def two_narrow():
        hip_check(hip.ts_hip_launch_group_begin(None))
        hip_check(layer.dw(got2))
        hip_check(hip.ts_hip_gemm(0, 0, M, N, K, a.ptr, K, b.ptr, N, c2.ptr, N, None))
        hip_check(hip.ts_hip_launch_group_end(None))

    assert _launches(two_narrow) == 1 + n3
    for g, w, name in zip(got2[:3], want[:3], ("dW", "db", "loss")):
        assert_bits_equal(g.get(), w.get(), f"two narrow: {name}")
    assert_bits_equal(c2.get(), c_want.get(), "two narrow: second")


def test_group_calls_out_of_order_are_refused():
    from train_station_amd._ffi import hip, hip_check
    from gpu_util import init
    init()
    s = ctypes.c_void_p()
    hip_check(hip.ts_hip_stream_create(ctypes.byref(s)))
    try:
        assert hip.ts_hip_launch_group_end(None) != 0  # no group open
        hip_check(hip.ts_hip_launch_group_begin(None))
        assert hip.ts_hip_launch_group_begin(None) != 0  # one at a time
        assert hip.ts_hip_launch_group_end(s) != 0  # another stream
        hip_check(hip.ts_hip_launch_group_end(None))
        assert hip.ts_hip_launch_group_end(None) != 0  # already closed
    finally:
        hip_check(hip.ts_hip_stream_synchronize(s))
        hip_check(hip.ts_hip_stream_destroy(s))


@pytest.fixture
def T():
    import train_station_amd as T
    yield T
    T.set_fusion(True)
    T.clear_gradients()


def _narrow_mlp(T, seed, frozen_first):
    """784 -> 1024 -> 10 at batch 1024 with an MSE: the second layer's dW and
    dX are held for one launch.  frozen_first: W1 and b1 constant and x
    requiring a gradient instead, so nothing reads dX2 before x.grad does."""
    rng = np.random.default_rng(seed)
    ps = []
    for fi, fo in ((784, 1024), (1024, 10)):
        bound = np.float32(np.sqrt(6.0 / fi))
        w = T.Tensor.from_slice(rng.uniform(-bound, bound, (fi, fo)).astype(np.float32), [fi, fo])
        b = T.Tensor.from_slice((0.1 * rng.standard_normal(fo)).astype(np.float32), [fo])
        if not (frozen_first and fi == 784):
            w, b = w.with_requires_grad(), b.with_requires_grad()
        ps += [w, b]
    x = T.Tensor.from_slice(rng.standard_normal((1024, 784)).astype(np.float32), [1024, 784])
    if frozen_first:
        x = x.with_requires_grad()
    t = T.Tensor.from_slice(rng.standard_normal((1024, 10)).astype(np.float32), [1024, 10])
    return ps, x, t


@pytest.mark.parametrize("order", ["dw_first", "dx_first", "loss_first"])
def test_held_weight_gradient_read_before_its_pair_runs_by_itself(T, order):
    # W1 constant, x requiring a gradient: after backward dX2 is still
    # deferred (only x.grad reads it), so reading W2's gradient, b2's or the
    # loss first runs the held dW2 by itself; x.grad then runs dX2 alone.
    # Every value equals the unfused run's.
    got = {}
    for on in (True, False):
        T.set_fusion(on)
        ps, x, t = _narrow_mlp(T, 23, True)
        h = x.matmul(ps[0]).add_tensor(ps[1]).relu()
        loss = h.matmul(ps[2]).add_tensor(ps[3]).sub_tensor(t).pow_scalar(2.0).mean()
        loss.backward()
        vals = {}
        reads = {"dw_first": ("w2", "b2", "loss", "x"), "dx_first": ("x", "w2", "b2", "loss"),
                 "loss_first": ("loss", "x", "b2", "w2")}[order]
        for r in reads:
            if r == "w2":
                vals[r] = ps[2].grad_by_value().data()
            elif r == "b2":
                vals[r] = ps[3].grad_by_value().data()
            elif r == "x":
                vals[r] = x.grad_by_value().data()
            else:
                vals[r] = np.array([loss.value()], dtype=np.float32)
        got[on] = vals
        T.clear_gradients()
    for k in got[True]:
        assert_bits_equal(got[True][k], got[False][k], f"{order}: {k}")


def test_held_weight_gradient_runs_before_its_input_is_written_in_place(T):
    # the held dW2 reads relu's output h; writing h in place (fill) before
    # anything reads dW2 runs the held product first, with the old h
    got = {}
    for on in (True, False):
        T.set_fusion(on)
        ps, x, t = _narrow_mlp(T, 29, True)
        h = x.matmul(ps[0]).add_tensor(ps[1]).relu()
        loss = h.matmul(ps[2]).add_tensor(ps[3]).sub_tensor(t).pow_scalar(2.0).mean()
        loss.backward()
        h.fill(0.5)
        got[on] = (ps[2].grad_by_value().data(), ps[3].grad_by_value().data(), x.grad_by_value().data(),
                   loss.value())
        T.clear_gradients()
    for name, a, b in zip(("w2", "b2", "x"), got[True][:3], got[False][:3]):
        assert_bits_equal(a, b, name)
    assert got[True][3] == got[False][3]
