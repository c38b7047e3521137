"""Batched / N-D and vector matmul on the device (matmul/mod.rs:263-760,
grad_fn/ops/matmul.rs:4-219), through the C-ABI and the handle API, against
float64 references (the oracle's textbook product rounded once).

Bars: products and gradients within 1e-4 normwise relative error of f64
(observed ~1e-6); the outer product and the dot-product gradient, which are
elementwise in the reference, bit-exact.
"""
from __future__ import annotations

import ctypes
import time

import numpy as np
import pytest

from conftest import assert_bits_equal, max_rel, normal

from oracle import gradtrack as G

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _hip():
    from train_station_amd._ffi import SZ, hip, hip_check
    return hip, hip_check, SZ


def _T():
    import train_station_amd as T
    return T


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
@pytest.mark.parametrize("bshape_a,bshape_b,M,N,K", [
    ((3,), (3,), 64, 48, 40), ((2, 1), (1, 5), 33, 17, 9), ((4,), (1,), 130, 257, 129),
    ((2, 3), (2, 3), 256, 256, 64), ((1,), (6,), 7, 300, 513), ((4, 1), (1, 4), 1024, 1000, 72)])
def test_gemm_batched_against_f64(ta, tb, bshape_a, bshape_b, M, N, K):
    from gpu_util import Dev, sync
    hip, check, SZ = _hip()
    ob = tuple(np.broadcast_shapes(bshape_a, bshape_b))
    a_mat = (K, M) if ta else (M, K)
    b_mat = (N, K) if tb else (K, N)
    A = normal(bshape_a + a_mat, 1)
    B = normal(bshape_b + b_mat, 2)
    want = np.matmul(np.swapaxes(A, -1, -2) if ta else A, np.swapaxes(B, -1, -2) if tb else B,
                     dtype=np.float64).reshape(ob + (M, N))

    def strides(bs, mat):
        st, s = [0] * len(ob), mat[0] * mat[1]
        for j in range(len(bs) - 1, -1, -1):
            st[j + len(ob) - len(bs)] = 0 if bs[j] == 1 else s
            s *= bs[j]
        return st

    dA, dB, dC = Dev.of(A), Dev.of(B), Dev(int(np.prod(ob)) * M * N)
    c = lambda v: (SZ * max(len(v), 1))(*v)
    check(hip.ts_hip_gemm_batched(ta, tb, M, N, K, dA.ptr, a_mat[1], dB.ptr, b_mat[1], dC.ptr, N, len(ob), c(ob),
                                  c(strides(bshape_a, a_mat)), c(strides(bshape_b, b_mat)), M * N, None))
    sync()
    got = dC.get(ob + (M, N))
    assert max_rel(got, want) < TOL


@pytest.mark.parametrize("rows,cols", [(1, 1), (7, 5), (4096, 4096), (33, 1000), (1000, 3), (8192, 1024)])
def test_gemv_both_orientations(rows, cols):
    from gpu_util import Dev, sync
    hip, check, SZ = _hip()
    A = normal((rows, cols), 3)
    for trans in (0, 1):
        x = normal(rows if trans else cols, 4)
        want = (A.T.astype(np.float64) @ x) if trans else (A.astype(np.float64) @ x)
        ws = hip.ts_hip_gemv_workspace_floats(trans, rows, cols)
        dA, dx, dy = Dev.of(A), Dev.of(x), Dev(want.size)
        dw = Dev(max(ws, 1))
        check(hip.ts_hip_gemv(trans, rows, cols, dA.ptr, cols, dx.ptr, dy.ptr, dw.ptr, ws, None))
        sync()
        assert max_rel(dy.get(), want) < 1e-6, (trans, rows, cols)
        if trans:  # the weighted column sum: the fixed chunk order, bit for bit
            import oracle
            assert_bits_equal(dy.get(), oracle.sum_dim0_chunked(A, x), f"gemv^T {rows}x{cols}")


def test_dot_and_outer():
    from gpu_util import Dev, sync
    hip, check, SZ = _hip()
    for n in (1, 7, 4096 + 3, 1 << 22):
        a, b = normal(n, 5), normal(n, 6)
        ws = hip.ts_hip_sum_workspace_floats(n)
        da, db, dout, dw = Dev.of(a), Dev.of(b), Dev(1), Dev(ws)
        check(hip.ts_hip_dot(da.ptr, db.ptr, n, dout.ptr, dw.ptr, ws, None))
        sync()
        want = float(np.dot(a.astype(np.float64), b))
        assert abs(dout.get()[0] - want) <= 1e-6 * np.sum(np.abs(a.astype(np.float64) * b))
    a, b = normal(300, 7), normal(257, 8)
    da, db, do = Dev.of(a), Dev.of(b), Dev(300 * 257)
    check(hip.ts_hip_outer(da.ptr, 300, db.ptr, 257, do.ptr, None))
    sync()
    assert_bits_equal(do.get((300, 257)), a[:, None] * b[None, :])


CASES = [((7,), (7,)), ((7,), (7, 5)), ((6, 7), (7,)), ((6, 7), (7, 5)), ((3, 6, 7), (3, 7, 5)),
         ((2, 1, 6, 7), (4, 7, 5)), ((6, 7), (4, 7, 5)), ((2, 3, 6, 7), (7, 5)), ((1, 6, 7), (7, 5)),
         ((6, 7), (1, 7, 5)), ((4, 2, 300, 130), (4, 2, 130, 257)), ((1000,), (1000, 4096)),
         ((4096, 1000), (1000,))]


@pytest.mark.parametrize("sa,sb", CASES, ids=lambda s: "x".join(map(str, s)))
def test_matmul_ranks_and_gradients(sa, sb):
    T = _T()
    a, b = normal(sa, 1), normal(sb, 2)
    ta = T.Tensor.from_slice(a, sa).with_requires_grad()
    tb = T.Tensor.from_slice(b, sb).with_requires_grad()
    oa, ob = G.OTensor(a.copy(), True), G.OTensor(b.copy(), True)
    y, oy = ta.matmul(tb), oa.matmul(ob)
    assert tuple(y.shape) == oy.shape
    assert max_rel(y.data().reshape(oy.shape), oy.data) < TOL
    go = np.array(normal(oy.shape, 3), np.float32).reshape(oy.shape)
    y.backward(T.Tensor.from_slice(go.reshape(-1), list(oy.shape)))
    G.backward(oy, go)
    for mine, theirs in ((ta, oa), (tb, ob)):
        g, w = mine.grad_by_value().data(), theirs.grad_by_value()
        assert g.shape == w.shape == theirs.shape  # operand-shaped in every case
        if len(sa) == 1 and len(sb) == 1:
            assert_bits_equal(g, w)  # go * b, go * a elementwise
        else:
            assert max_rel(g, w) < TOL, (sa, sb)
    T.clear_gradients()
    G.clear_gradients()


def test_matmul_errors():
    T = _T()
    z = lambda *s: T.Tensor.zeros(list(s))
    with pytest.raises(T.TsError, match="same length for dot product"):
        z(3).matmul(z(4))
    with pytest.raises(T.TsError, match="Vector length must match matrix rows"):
        z(3).matmul(z(4, 2))
    with pytest.raises(T.TsError, match="Matrix columns must match vector length"):
        z(2, 3).matmul(z(4))
    with pytest.raises(T.TsError, match="Batched matmul requires at least 2D tensors"):
        z(3).matmul(z(2, 3, 4))
    with pytest.raises(T.TsError, match="Inner dimensions must match for batched matmul"):
        z(2, 3, 4).matmul(z(2, 5, 6))
    with pytest.raises(T.TsError, match="Cannot broadcast dimensions 2 and 3"):
        z(2, 3, 4).matmul(z(3, 4, 6))


def test_batched_throughput():
    # attention-shaped batch: 64 independent 1024x1024x128 products on the MFMA tiles
    T = _T()
    a = T.Tensor.randn([8, 8, 1024, 128], seed=1)
    b = T.Tensor.randn([8, 8, 128, 1024], seed=2)
    y = a.matmul(b)
    T.synchronize()
    t0 = time.perf_counter()
    for _ in range(10):
        y = a.matmul(b)
    T.synchronize()
    dt = (time.perf_counter() - t0) / 10
    flop = 2.0 * 64 * 1024 * 1024 * 128
    print(f"batched 64 x (1024x128 . 128x1024): {dt * 1e3:.3f} ms, {flop / dt / 1e12:.1f} TFLOP/s", flush=True)
    got = y.data()[3, 5]
    A, B = a.data()[3, 5].astype(np.float64), b.data()[3, 5].astype(np.float64)
    assert max_rel(got, A @ B) < TOL
