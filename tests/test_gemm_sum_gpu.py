"""A sum formed in a weight-gradient product's launch
(ts_hip_gemm_colsum_bsum): the product and its column sums have the bits of
ts_hip_gemm_colsum_xf, and B's sum (or mean) as stored -- before B's
transform -- has the bits of ts_hip_sum / ts_hip_mean over B.  In the engine
the README step's loss, sum(relu(x W + b)) (README.md:71-79), is formed by
the weight-gradient product, which reads relu's output through relu's
backward anyway: the step runs in three launches -- forward product, weight
gradient with the bias gradient and the loss, Adam -- with the bits of the
op-by-op run.
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


def _xf(code, imm):
    from train_station_amd._ffi import OperandXf
    x = OperandXf()
    x.n_ops = 1
    x.code[0] = code
    x.imm[0] = imm
    return x


# (M, N, K, xa, xb, mean) of dW[M,N] = A[K,M]^T . B[K,N]: the README step's
# weight gradient (784x128 from 32 rows, relu's backward of a constant applied
# to B as loaded), other 64x64-tile grids, an odd N (element loads, a B whose
# values end past the float4 groups), a transformed A, the largest B one
# workgroup's sum covers (16384 values), and 128x128 tiles
CASES = [
    (784, 128, 32, None, (XF_RELU_BWD_S, 1.0), False),
    (784, 128, 32, None, (XF_RELU_BWD_S, 1.0), True),
    (300, 260, 40, None, None, False),
    (1024, 130, 31, None, (XF_MUL_S, 0.5), True),
    (400, 96, 77, (XF_MUL_S, 2.0), None, False),
    (256, 128, 128, None, (XF_RELU_BWD_S, 0.25), False),
    (2048, 1024, 16, None, None, False),
]


@pytest.mark.parametrize("M,N,K,xa,xb,mean", CASES)
def test_sum_of_b_in_the_product_launch(M, N, K, xa, xb, mean):
    from gpu_util import Dev, sync
    hip, check = _hip()
    print(f"[bsum] {M}x{N}x{K} xa={xa} xb={xb} mean={mean}", flush=True)
    assert hip.ts_hip_gemm_takes_bsum(1, M, N, K) == 1
    pxa = ctypes.byref(_xf(*xa)) if xa else None
    pxb = ctypes.byref(_xf(*xb)) if xb else None
    for call, seed in enumerate((3, 23)):  # two calls in a row
        a, b = normal((K, M), seed), normal((K, N), seed + 1)
        da, db = Dev.of(a), Dev.of(b)
        c, cs, s = Dev(M * N), Dev(N), Dev(1)
        rc, rcs, want = Dev(M * N), Dev(N), Dev(1)
        check(hip.ts_hip_gemm_colsum_bsum(1, M, N, K, da.ptr, M, pxa, db.ptr, pxb, c.ptr, N, cs.ptr, s.ptr,
                                          int(mean), None))
        ws_floats = hip.ts_hip_gemm_colsum_workspace_floats(1, M, N, K)
        ws = Dev(max(ws_floats, 2))
        check(hip.ts_hip_gemm_colsum_xf(1, M, N, K, da.ptr, M, pxa, db.ptr, N, pxb, rc.ptr, N, rcs.ptr, ws.ptr,
                                        ws.n, None))
        sws = Dev(max(hip.ts_hip_sum_workspace_floats(K * N), 2))
        check((hip.ts_hip_mean if mean else hip.ts_hip_sum)(db.ptr, K * N, want.ptr, sws.ptr, sws.n, None))
        sync()
        assert_bits_equal(c.get(), rc.get(), f"dW, call {call}")
        assert_bits_equal(cs.get(), rcs.get(), f"column sums, call {call}")
        assert_bits_equal(s.get(), want.get(), f"sum of B, call {call}")
        # the sum is B's, untransformed: f64 over the uploaded values
        exact = np.sum(b.astype(np.float64)) / (K * N if mean else 1)
        scale = np.sum(np.abs(b.astype(np.float64))) / (K * N if mean else 1)
        assert abs(float(s.get()[0]) - exact) <= 1e-6 * scale


def test_products_the_sum_does_not_ride_on_are_refused():
    from gpu_util import Dev
    hip, _ = _hip()
    # not trans_a; the LDS-DMA grid; B past one workgroup's sum; the narrow
    # kernel (few tiles, long K) and few columns (N <= 16)
    assert hip.ts_hip_gemm_takes_bsum(0, 784, 128, 32) == 0
    for shape in [(4096, 4096, 8192), (784, 1024, 1024), (784, 128, 200), (32, 128, 784), (1024, 10, 64),
                  (784, 0, 32)]:
        assert hip.ts_hip_gemm_takes_bsum(1, *shape) == 0, shape
    M, N, K = 784, 128, 32
    a, b = Dev.of(normal((K, M), 1)), Dev.of(normal((K, N), 2))
    bu = Dev.of(normal((K, N), 2), 1)  # B not 16-byte aligned
    c, cs, s = Dev(M * N), Dev(N), Dev(1)
    assert hip.ts_hip_gemm_colsum_bsum(1, M, N, K, a.ptr, M, None, bu.ptr, None, c.ptr, N, cs.ptr, s.ptr, 0,
                                       None) != 0
    assert hip.ts_hip_gemm_colsum_bsum(1, M, N, K, a.ptr, M, None, b.ptr, None, c.ptr, N, cs.ptr, None, 0,
                                       None) != 0
    assert hip.ts_hip_gemm_colsum_bsum(1, M, N, K, a.ptr, M, None, b.ptr, None, c.ptr, N, None, s.ptr, 0,
                                       None) != 0
    assert hip.ts_hip_gemm_colsum_bsum(0, M, N, K, a.ptr, K, None, b.ptr, None, c.ptr, N, cs.ptr, s.ptr, 0,
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
