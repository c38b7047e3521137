"""A sum formed in a weight-gradient product's launch
(ts_hip_gemm_colsum_bsum) and a subtraction in a product's store
(ts_hip_gemm_fused_sub).  The product and its column sums have the bits of
ts_hip_gemm_colsum_xf, and B's sum (or mean) as stored -- before B's
transform, after the sum's own transform -- has the bits of ts_hip_sum /
ts_hip_mean over those values; the subtraction has the bits of the product
followed by ts_hip_sub.  In the engine the README step's loss,
sum(relu(x W + b)) (README.md:71-79), is formed by the weight-gradient
product, which reads relu's output through relu's backward anyway: the step
runs in three launches -- forward product, weight gradient with the bias
gradient and the loss, Adam.  Config 4's MSE, mean((x W2 + b2 - t)^2)
(feedforward_network.rs:478-479), runs as the last forward product with the
subtraction in its store and the loss in the last weight gradient: six
launches, no elementwise pass.  Every result has the bits of the op-by-op
run.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import assert_bits_equal, normal

pytestmark = pytest.mark.gpu

XF_MUL_S, XF_RELU_BWD_S = 2, 7


def _hip():
    from train_station_amd._ffi import hip, hip_check
    return hip, hip_check


XF_SQUARE = 8


def _xf(*ops):
    """ops: (code, imm) pairs, applied in order"""
    from train_station_amd._ffi import OperandXf
    x = OperandXf()
    x.n_ops = len(ops)
    for i, (code, imm) in enumerate(ops):
        x.code[i] = code
        x.imm[i] = imm
    return x


# (M, N, K, xa, xb, xs, mean) of dW[M,N] = A[K,M]^T . B[K,N], xs the sum's
# transform: the README step's weight gradient (784x128 from 32 rows, relu's
# backward of a constant applied to B as loaded), other 64x64-tile grids, an
# odd N (element loads, a B whose values end past the float4 groups), a
# transformed A, the largest B one workgroup's sum covers (16384 values),
# 128x128 tiles; and the narrow kernel (N <= 16, K >= 1024): config 4's last
# weight gradient (1024x10 from 1024 rows, the MSE's 2 * d * (1/n) applied
# to B as loaded, the loss d * d summed), 16 columns at 16384 values, and a
# ragged K
MSE_XB = ((XF_MUL_S, 2.0), (XF_MUL_S, 1.0 / 10240))
CASES = [
    (784, 128, 32, None, ((XF_RELU_BWD_S, 1.0),), None, False),
    (784, 128, 32, None, ((XF_RELU_BWD_S, 1.0),), None, True),
    (300, 260, 40, None, None, ((XF_SQUARE, 0.0),), False),
    (1024, 130, 31, None, ((XF_MUL_S, 0.5),), None, True),
    (400, 96, 77, ((XF_MUL_S, 2.0),), None, None, False),
    (256, 128, 128, None, ((XF_RELU_BWD_S, 0.25),), None, False),
    (2048, 1024, 16, None, None, None, False),
    (1024, 10, 1024, None, MSE_XB, ((XF_SQUARE, 0.0),), True),
    (1024, 10, 1024, None, None, None, False),
    (512, 16, 1024, None, ((XF_MUL_S, 3.0),), ((XF_SQUARE, 0.0),), False),
    (300, 7, 2000, ((XF_MUL_S, 0.5),), None, ((XF_SQUARE, 0.0),), True),
]


@pytest.mark.parametrize("M,N,K,xa,xb,xs,mean", CASES)
def test_sum_of_b_in_the_product_launch(M, N, K, xa, xb, xs, mean):
    from gpu_util import Dev, sync
    hip, check = _hip()
    print(f"[bsum] {M}x{N}x{K} xa={xa} xb={xb} xs={xs} mean={mean}", flush=True)
    assert hip.ts_hip_gemm_takes_bsum(1, M, N, K) == 1
    pxa = ctypes.byref(_xf(*xa)) if xa else None
    pxb = ctypes.byref(_xf(*xb)) if xb else None
    pxs = ctypes.byref(_xf(*xs)) if xs else None
    for call, seed in enumerate((3, 23)):  # two calls in a row
        a, b = normal((K, M), seed), normal((K, N), seed + 1)
        da, db = Dev.of(a), Dev.of(b)
        c, cs, s = Dev(M * N), Dev(N), Dev(1)
        rc, rcs, want = Dev(M * N), Dev(N), Dev(1)
        check(hip.ts_hip_gemm_colsum_bsum(1, M, N, K, da.ptr, M, pxa, db.ptr, pxb, c.ptr, N, cs.ptr, pxs, s.ptr,
                                          int(mean), None))
        ws_floats = hip.ts_hip_gemm_colsum_workspace_floats(1, M, N, K)
        ws = Dev(max(ws_floats, 2))
        check(hip.ts_hip_gemm_colsum_xf(1, M, N, K, da.ptr, M, pxa, db.ptr, N, pxb, rc.ptr, N, rcs.ptr, ws.ptr,
                                        ws.n, None))
        # the summed values: B, or B * B (pow_scalar(2)'s bits) for the square
        summed = db
        if xs:
            summed = Dev(K * N)
            check(hip.ts_hip_mul(db.ptr, db.ptr, summed.ptr, K * N, None))
        sws = Dev(max(hip.ts_hip_sum_workspace_floats(K * N), 2))
        check((hip.ts_hip_mean if mean else hip.ts_hip_sum)(summed.ptr, K * N, want.ptr, sws.ptr, sws.n, None))
        sync()
        assert_bits_equal(c.get(), rc.get(), f"dW, call {call}")
        assert_bits_equal(cs.get(), rcs.get(), f"column sums, call {call}")
        assert_bits_equal(s.get(), want.get(), f"sum of B, call {call}")
        # and the sum is the sum: f64 over the uploaded values (squared in f64 for xs)
        b64 = b.astype(np.float64)
        vals = b64 * b64 if xs else b64
        exact = np.sum(vals) / (K * N if mean else 1)
        scale = np.sum(np.abs(vals)) / (K * N if mean else 1)
        assert abs(float(s.get()[0]) - exact) <= 1e-6 * scale


def test_products_the_sum_does_not_ride_on_are_refused():
    from gpu_util import Dev
    hip, _ = _hip()
    # not trans_a; the LDS-DMA grid; B past one workgroup's sum; the narrow
    # kernel below its widest workgroups (K < 1024) or past one workgroup's
    # sum
    assert hip.ts_hip_gemm_takes_bsum(0, 784, 128, 32) == 0
    for shape in [(4096, 4096, 8192), (784, 1024, 1024), (784, 128, 200), (32, 128, 784), (1024, 10, 64),
                  (1024, 10, 512), (784, 0, 32), (1024, 16, 2048)]:
        assert hip.ts_hip_gemm_takes_bsum(1, *shape) == 0, shape
    M, N, K = 784, 128, 32
    a, b = Dev.of(normal((K, M), 1)), Dev.of(normal((K, N), 2))
    bu = Dev.of(normal((K, N), 2), 1)  # B not 16-byte aligned
    c, cs, s = Dev(M * N), Dev(N), Dev(1)
    assert hip.ts_hip_gemm_colsum_bsum(1, M, N, K, a.ptr, M, None, bu.ptr, None, c.ptr, N, cs.ptr, None, s.ptr,
                                       0, None) != 0
    assert hip.ts_hip_gemm_colsum_bsum(1, M, N, K, a.ptr, M, None, b.ptr, None, c.ptr, N, cs.ptr, None, None, 0,
                                       None) != 0
    assert hip.ts_hip_gemm_colsum_bsum(1, M, N, K, a.ptr, M, None, b.ptr, None, c.ptr, N, None, None, s.ptr, 0,
                                       None) != 0
    assert hip.ts_hip_gemm_colsum_bsum(0, M, N, K, a.ptr, K, None, b.ptr, None, c.ptr, N, cs.ptr, None, s.ptr,
                                       0, None) != 0


# (ta, tb, M, N, K, A offset, bias, relu, mask): config 4's last forward
# product, unaligned A, transposed operands, few tiles with a long K
SUB_CASES = [
    (0, 0, 1024, 10, 1024, 0, True, False, False),
    (0, 0, 100, 7, 333, 1, False, True, False),
    (0, 1, 33, 5, 70, 0, True, False, True),
    (1, 0, 64, 12, 600, 0, True, True, False),
    (0, 0, 32, 128, 784, 0, True, False, False),
]


@pytest.mark.parametrize("ta,tb,M,N,K,off,bias,relu,mask", SUB_CASES)
def test_subtraction_in_the_product_store(ta, tb, M, N, K, off, bias, relu, mask):
    from gpu_util import Dev, sync
    hip, check = _hip()
    print(f"[sub] ta={ta} tb={tb} {M}x{N}x{K} off={off} bias={bias} relu={relu} mask={mask}", flush=True)
    assert hip.ts_hip_gemm_takes_sub(ta, tb, M, N, K) == 1
    a = normal((K, M) if ta else (M, K), 1)
    b = normal((N, K) if tb else (K, N), 2)
    da, db = Dev.of(a, off), Dev.of(b)
    dbias, dt, dmask = Dev.of(normal(N, 3)), Dev.of(normal((M, N), 4)), Dev.of(normal((M, N), 5))
    lda, ldb = (M if ta else K), (K if tb else N)
    got, ref = Dev(M * N), Dev(M * N)
    check(hip.ts_hip_gemm_fused_sub(ta, tb, M, N, K, da.ptr, lda, db.ptr, ldb, dbias.ptr if bias else None, dt.ptr,
                                    int(relu), dmask.ptr if mask else None, got.ptr, N, None))
    check(hip.ts_hip_gemm_fused(ta, tb, M, N, K, da.ptr, lda, db.ptr, ldb, dbias.ptr if bias else None, 0, None,
                                ref.ptr, N, None, 0, None))
    check(hip.ts_hip_sub(ref.ptr, dt.ptr, ref.ptr, M * N, None))
    if relu:
        check(hip.ts_hip_relu(ref.ptr, ref.ptr, M * N, None))
    if mask:
        check(hip.ts_hip_relu_backward(dmask.ptr, ref.ptr, ref.ptr, M * N, None))
    sync()
    assert_bits_equal(got.get(), ref.get(), "product minus t")


def test_subtraction_is_refused_off_the_narrow_kernel():
    from gpu_util import Dev
    hip, _ = _hip()
    for shape in [(1024, 1024, 784), (8192, 4096, 4096), (32, 128, 256), (0, 10, 100)]:
        assert hip.ts_hip_gemm_takes_sub(0, 0, *shape) == 0, shape
    a, b, t, c = Dev.of(normal((64, 64), 1)), Dev.of(normal((64, 64), 2)), Dev(64 * 64), Dev(64 * 64)
    assert hip.ts_hip_gemm_fused_sub(0, 0, 64, 64, 64, a.ptr, 64, b.ptr, 64, None, t.ptr, 0, None, c.ptr, 64,
                                     None) != 0
    assert hip.ts_hip_gemm_fused_sub(0, 0, 64, 10, 1024, a.ptr, 1024, b.ptr, 10, None, None, 0, None, c.ptr, 10,
                                     None) != 0


@pytest.fixture
def T():
    import train_station_amd as T
    yield T
    T.set_fusion(True)
    T.clear_gradients()


def _readme_params(T, seed):
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((784, 128)).astype(np.float32)
    b = (0.1 * rng.standard_normal(128)).astype(np.float32)
    x = rng.standard_normal((32, 784)).astype(np.float32)
    return (T.Tensor.from_slice(w, [784, 128]).with_requires_grad(),
            T.Tensor.from_slice(b, [128]).with_requires_grad(), T.Tensor.from_slice(x, [32, 784]))


@pytest.mark.parametrize("kind", ["sum", "mean"])
@pytest.mark.parametrize("read_first", [False, True])
def test_readme_step_launches(T, kind, read_first):
    # the loss read only after backward: three launches; read before
    # backward: its own sum pass as well.  The same bits every way.
    out, counts = {}, {}
    for on in (True, False):
        T.set_fusion(on)
        w, b, x = _readme_params(T, 5)
        opt = T.Adam.with_learning_rate(1e-3)
        opt.add_parameters([w, b])
        losses = []
        for step in range(3):
            T.synchronize()
            T.Profile.reset()
            T.Profile.enable(True)
            loss = getattr(x.matmul(w).add_tensor(b).relu(), kind)()
            if read_first:
                losses.append(loss.value())
            loss.backward()
            opt.step([w, b])
            opt.zero_grad([w, b])
            T.synchronize()
            T.Profile.enable(False)
            if step == 2:
                counts[on] = {k: T.Profile.read(getattr(T.Profile, k))["launches"]
                              for k in ("GEMM", "ELEMENTWISE", "REDUCTION", "ADAM")}
            if not read_first:
                losses.append(loss.value())
        out[on] = (losses, w.data(), b.data())
    want = {"GEMM": 2, "ELEMENTWISE": 0, "REDUCTION": 1 if read_first else 0, "ADAM": 1}
    assert counts[True] == want, counts
    (l1, w1, b1), (l0, w0, b0) = out[True], out[False]
    assert l1 == l0
    assert_bits_equal(w1, w0, "W after 3 steps")
    assert_bits_equal(b1, b0, "b after 3 steps")


def test_sum_of_a_product_with_other_consumers(T):
    # the product is also read by a second chain: it runs bare once, each
    # chain as its epilogue, and the sum as a pass of its own -- the same bits
    vals = {}
    for on in (True, False):
        T.set_fusion(on)
        w, b, x = _readme_params(T, 9)
        b2 = T.Tensor.from_slice(normal(128, 4), [128])
        z = x.matmul(w)
        h = z.add_tensor(b).relu()
        other = z.add_tensor(b2)
        loss = h.sum()
        vals[on] = (loss.value(), other.data(), h.data())
    assert vals[True][0] == vals[False][0]
    assert_bits_equal(vals[True][1], vals[False][1], "other consumer")
    assert_bits_equal(vals[True][2], vals[False][2], "summed value")


def test_sum_before_an_inplace_update_of_the_weight(T):
    # Adam writes W in place before the loss is read: the product runs first
    # and the loss, formed later, still sees the old W
    T.set_fusion(True)
    w, b, x = _readme_params(T, 13)
    wv, xv = w.data().copy(), x.data().copy()
    loss = x.matmul(w).add_tensor(b).relu().sum()
    w.set_grad(T.Tensor.from_slice(normal((784, 128), 6), [784, 128]))
    opt = T.Adam.with_learning_rate(0.5)
    opt.add_parameter(w)
    opt.step([w])
    got = loss.value()
    T.set_fusion(False)
    want = T.Tensor.from_slice(xv.reshape(32, 784), [32, 784]).matmul(
        T.Tensor.from_slice(wv.reshape(784, 128), [784, 128])).add_tensor(b).relu().sum().value()
    assert got == want
    assert not np.array_equal(w.data(), wv)


def _config4(T, seed):
    rng = np.random.default_rng(seed)
    ws = []
    for fi, fo in ((784, 1024), (1024, 10)):
        bound = np.float32(np.sqrt(6.0 / fi))
        w = rng.uniform(-bound, bound, (fi, fo)).astype(np.float32)
        b = (0.1 * rng.standard_normal(fo)).astype(np.float32)
        ws += [T.Tensor.from_slice(w, [fi, fo]).with_requires_grad(), T.Tensor.from_slice(b, [fo]).with_requires_grad()]
    x = T.Tensor.from_slice(rng.standard_normal((1024, 784)).astype(np.float32), [1024, 784])
    t = T.Tensor.from_slice(rng.standard_normal((1024, 10)).astype(np.float32), [1024, 10])
    return ws, x, t


def _mse_loss(x, t, ps):
    h = x.matmul(ps[0]).add_tensor(ps[1]).relu()
    y = h.matmul(ps[2]).add_tensor(ps[3])
    return y.sub_tensor(t).pow_scalar(2.0).mean()


@pytest.mark.parametrize("read_first", [False, True])
def test_config4_step_launches(T, read_first):
    # the loss read after backward: five launches (two forward products, the
    # last with the MSE's subtraction; dX2 and dW2 with db2 and the loss as
    # one launch of a launch group; dW1 with db1; Adam), no elementwise pass;
    # read before backward: its own pass.  The same bits as the op-by-op run
    # either way.
    out, counts = {}, {}
    for on in (True, False):
        T.set_fusion(on)
        ps, x, t = _config4(T, 17)
        opt = T.Adam.with_learning_rate(1e-3)
        opt.add_parameters(ps)
        losses = []
        for step in range(3):
            T.synchronize()
            T.Profile.reset()
            T.Profile.enable(True)
            loss = _mse_loss(x, t, ps)  # the prediction is not held: the loss is its only consumer
            if read_first:
                losses.append(loss.value())
            loss.backward()
            opt.step(ps)
            opt.zero_grad(ps)
            T.synchronize()
            T.Profile.enable(False)
            if step == 2:
                counts[on] = {k: T.Profile.read(getattr(T.Profile, k))["launches"]
                              for k in ("GEMM", "ELEMENTWISE", "REDUCTION", "ADAM")}
            if not read_first:
                losses.append(loss.value())
        out[on] = (losses, [p.data() for p in ps])
    if read_first:
        assert counts[True]["GEMM"] == 4 and counts[True]["ADAM"] == 1, counts
    else:
        assert counts[True] == {"GEMM": 4, "ELEMENTWISE": 0, "REDUCTION": 0, "ADAM": 1}, counts
    assert out[True][0] == out[False][0]
    for i, (a, b) in enumerate(zip(out[True][1], out[False][1])):
        assert_bits_equal(a, b, f"param {i} after 3 steps")


def test_prediction_and_loss_of_a_fused_subtraction(T):
    # the prediction y is read as well as y - t: the product runs once, bare,
    # and both keep the bits of the op-by-op run
    vals = {}
    for on in (True, False):
        T.set_fusion(on)
        ps, x, t = _config4(T, 23)
        h = x.matmul(ps[0]).add_tensor(ps[1]).relu()
        y = h.matmul(ps[2]).add_tensor(ps[3])
        d = y.sub_tensor(t)
        loss = d.pow_scalar(2.0).mean()
        vals[on] = (loss.value(), y.data(), d.data())
    assert vals[True][0] == vals[False][0]
    assert_bits_equal(vals[True][1], vals[False][1], "prediction")
    assert_bits_equal(vals[True][2], vals[False][2], "difference")
