"""Fusion of recorded ops into the producing product: a 2-D matmul deferred
until its result is read, a following row-bias add and relu applied in its
store, and relu's backward applied in the store of the dX product
(ts_hip_gemm_fused).  The fused results must be the bits of the separate
kernels (the reference's op sequence: matmul/mod.rs:572-611, ops/add.rs,
ops/relu.rs, grad_fn/ops/relu.rs), for every GEMM path: LDS-DMA tiles,
register-staged tiles (unaligned operands), 64x64 tiles and split-K.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_bits_equal, normal

pytestmark = pytest.mark.gpu


def _T():
    import train_station_amd as T
    return T


def _hip():
    from train_station_amd._ffi import hip, hip_check
    return hip, hip_check


@pytest.fixture
def fusion():
    T = _T()
    yield T
    T.set_fusion(True)
    T.clear_gradients()


# (M, N, K, offset): offset 1 shifts A by one float so the operands are not
# 16-byte aligned (register-staged kernel); N <= 16 and few tiles with a long
# K (32x128x784) take the narrow kernel, a K past it split-K (32x128x16384);
# 784 rows leave an edge tile (clamped loads)
SHAPES = [(8192, 4096, 512, 0), (1024, 1024, 784, 0), (32, 128, 784, 0), (300, 260, 77, 0), (1024, 512, 256, 1),
          (1024, 10, 1024, 0), (1000, 7, 333, 1), (784, 1024, 1024, 0), (32, 128, 16384, 0)]


@pytest.mark.parametrize("M,N,K,off", SHAPES)
@pytest.mark.parametrize("mode", ["bias", "relu", "bias_relu", "mask", "mask_nn", "all"])
def test_fused_entry_point_matches_separate_kernels(M, N, K, off, mode):
    from gpu_util import Dev, sync
    hip, check = _hip()
    print(f"[fused] {mode} M={M} N={N} K={K} off={off}", flush=True)
    # the dX product (mask) is NT, the forward one NN; mask_nn and all cover
    # the mask on the NN kernels too
    tb = 1 if mode == "mask" else 0
    a = normal((M, K), 1)
    b = normal((N, K) if tb else (K, N), 2)
    bias = normal(N, 3)
    mask = normal((M, N), 4)
    da, db, dbias, dmask = Dev.of(a, off), Dev.of(b), Dev.of(bias), Dev.of(mask)
    ldb = K if tb else N
    use_bias = mode in ("bias", "bias_relu", "all")
    use_relu = mode in ("relu", "bias_relu", "all")
    use_mask = mode in ("mask", "mask_nn", "all")
    fused, ref = Dev(M * N), Dev(M * N)
    # a split product takes its temporary from the workspace (the host's way)
    ws_floats = hip.ts_hip_gemm_workspace_floats(M, N, K)
    dws = Dev(max(ws_floats, 1))
    check(hip.ts_hip_gemm_fused(0, tb, M, N, K, da.ptr, K, db.ptr, ldb, dbias.ptr if use_bias else None,
                                int(use_relu), dmask.ptr if use_mask else None, fused.ptr, N,
                                dws.ptr if ws_floats else None, ws_floats, None))
    check(hip.ts_hip_gemm(0, tb, M, N, K, da.ptr, K, db.ptr, ldb, ref.ptr, N, None))
    if use_bias:
        check(hip.ts_hip_bias_add(ref.ptr, dbias.ptr, ref.ptr, M, N, 0, None))
    if use_relu:
        check(hip.ts_hip_relu(ref.ptr, ref.ptr, M * N, None))
    if use_mask:
        check(hip.ts_hip_relu_backward(dmask.ptr, ref.ptr, ref.ptr, M * N, None))
    sync()
    assert_bits_equal(fused.get(), ref.get(), f"{mode} {M}x{N}x{K}")


def _mlp(T, widths, batch, seed):
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


def _step(T, ps, x, t, bias_first=False):
    h = x
    n = len(ps) // 2
    for i in range(n):
        m = h.matmul(ps[2 * i])
        h = ps[2 * i + 1].add_tensor(m) if bias_first else m.add_tensor(ps[2 * i + 1])
        if i < n - 1:
            h = h.relu()
    loss = h.sub_tensor(t).pow_scalar(2.0).mean()
    loss.backward()
    return loss, h


@pytest.mark.parametrize("widths,batch", [([512, 1024, 1024, 256], 2048), ([784, 1024, 10], 1024),
                                          ([64, 96, 48], 33)])
@pytest.mark.parametrize("bias_first", [False, True])
def test_training_step_is_bit_identical_with_and_without_fusion(fusion, widths, batch, bias_first):
    T = fusion
    out = {}
    for on in (True, False):
        T.set_fusion(on)
        ps, x, t = _mlp(T, widths, batch, 7)
        opt = T.Adam.with_learning_rate(1e-3)
        opt.add_parameters(ps)
        losses = []
        for _ in range(3):
            loss, y = _step(T, ps, x, t, bias_first)
            losses.append(loss.value())
            grads = [p.grad_by_value().data() for p in ps]
            opt.step(ps)
            opt.zero_grad(ps)
        out[on] = (losses, y.data(), grads, [p.data() for p in ps])
    (l1, y1, g1, p1), (l0, y0, g0, p0) = out[True], out[False]
    assert l1 == l0
    assert_bits_equal(y1, y0, "output")
    for i, (a, b) in enumerate(zip(g1, g0)):
        assert_bits_equal(a, b, f"grad {i}")
    for i, (a, b) in enumerate(zip(p1, p0)):
        assert_bits_equal(a, b, f"param {i} after 3 steps")


def test_intermediates_stay_readable(fusion):
    # the deferred product and the pre-activation are never written when the
    # fused chain runs; reading them later computes them then
    T = fusion
    x = T.Tensor.from_slice(normal((512, 384), 1), [512, 384])
    w = T.Tensor.from_slice(normal((384, 640), 2), [384, 640])
    b = T.Tensor.from_slice(normal(640, 3), [640])
    vals = {}
    for on in (True, False):
        T.set_fusion(on)
        h = x.matmul(w)
        z = h.add_tensor(b)
        y = z.relu()
        vals[on] = (y.data(), z.data(), h.data())  # y first: the fused kernel runs, then z and h on demand
    for name, a, c in zip("yzh", vals[True], vals[False]):
        assert_bits_equal(a, c, name)


def test_deferred_product_sees_the_operand_before_an_inplace_update(fusion):
    # Adam updates W in place; a product of W deferred before the step must
    # still give the pre-step value
    T = fusion
    T.set_fusion(True)
    xv, wv = normal((256, 128), 4), normal((128, 192), 5)
    x = T.Tensor.from_slice(xv, [256, 128])
    w = T.Tensor.from_slice(wv, [128, 192]).with_requires_grad()
    h = x.matmul(w)                                       # deferred
    w.set_grad(T.Tensor.from_slice(normal((128, 192), 6), [128, 192]))
    opt = T.Adam.with_learning_rate(0.5)
    opt.add_parameter(w)
    opt.step([w])                                         # runs h's product first
    T.set_fusion(False)
    want = T.Tensor.from_slice(xv, [256, 128]).matmul(T.Tensor.from_slice(wv, [128, 192])).data()
    assert_bits_equal(h.data(), want)
    assert not np.array_equal(w.data(), wv)               # the step did update W


def test_deferred_product_sees_the_operand_before_fill_randn(fusion):
    T = fusion
    T.set_fusion(True)
    xv, wv = normal((64, 96), 7), normal((96, 80), 8)
    x = T.Tensor.from_slice(xv, [64, 96])
    w = T.Tensor.from_slice(wv, [96, 80])
    h = x.matmul(w)
    w.fill_randn(seed=3)
    T.set_fusion(False)
    want = T.Tensor.from_slice(xv, [64, 96]).matmul(T.Tensor.from_slice(wv, [96, 80])).data()
    assert_bits_equal(h.data(), want)


def test_profiler_charges_fused_products_to_the_gemm_class(fusion):
    # a deferred product runs inside the window of the launch that first reads
    # it; the profiler splits that window, so the GEMM class sees every product
    T = fusion
    T.set_fusion(True)
    ps, x, t = _mlp(T, [256, 512, 512, 128], 1024, 9)
    T.Profile.reset()
    T.Profile.enable(True)
    _step(T, ps, x, t)
    T.synchronize()
    T.Profile.enable(False)
    g = T.Profile.read(T.Profile.GEMM)
    # 3 forward + 2 dX (the first layer's input has no gradient) + 3 dW
    assert g["launches"] == 8
    flops = 2.0 * 1024 * (256 * 512 + 512 * 512 + 512 * 128)
    assert abs(g["work"] - flops * (1 + 1) - 2.0 * 1024 * (512 * 512 + 512 * 128)) < 1.0


def test_product_with_several_consumers(fusion):
    # a deferred product read by the fused bias + relu chain and, separately,
    # by other ops (a scalar multiply, a second bias add): every branch and
    # every gradient equals the unfused graph's, and the product runs once
    # (the chain already deferred on it becomes its epilogue alone)
    T = fusion
    out = {}
    for on in (True, False):
        T.set_fusion(on)
        x = T.Tensor.from_slice(normal((300, 260), 1), [300, 260])
        w = T.Tensor.from_slice((normal((260, 130), 2) / 16).astype(np.float32), [260, 130]).with_requires_grad()
        b = T.Tensor.from_slice(normal(130, 3), [130]).with_requires_grad()
        b2 = T.Tensor.from_slice(normal(130, 4), [130]).with_requires_grad()
        T.Profile.reset()
        T.Profile.enable(True)
        h = x.matmul(w)
        a = h.add_tensor(b).relu()          # fused into the product's store
        c = h.mul_scalar(2.0)               # reads the bare product
        d = b2.add_tensor(h).relu()         # a second fused chain on the same product
        loss = a.add_tensor(c).mul_tensor(d).sum()
        loss.value()                        # the sum is deferred until read (or until backward's pass)
        T.Profile.enable(False)
        assert T.Profile.read(T.Profile.GEMM)["launches"] == 1, on   # the forward product, once
        T.Profile.reset()
        T.Profile.enable(True)
        loss.backward()
        T.synchronize()
        T.Profile.enable(False)
        # the LIFO engine applies the product's node once per gradient path
        # that reaches it (engine.rs:962-1047): three dW products, x needs none
        assert T.Profile.read(T.Profile.GEMM)["launches"] == 3, on
        out[on] = (loss.value(), a.data(), c.data(), d.data(),
                   [p.grad_by_value().data() for p in (w, b, b2)])
        T.clear_gradients()
    (l1, a1, c1, d1, g1), (l0, a0, c0, d0, g0) = out[True], out[False]
    assert l1 == l0
    for name, u, v in (("a", a1, a0), ("c", c1, c0), ("d", d1, d0)):
        assert_bits_equal(u, v, name)
    for i, (u, v) in enumerate(zip(g1, g0)):
        assert_bits_equal(u, v, f"grad {i}")


def test_two_fused_chains_on_one_product_run_it_once(fusion):
    # both consumers extend the deferred product before anything reads it:
    # the second one runs the product (bare) and turns the first chain into
    # its epilogue alone; a chain forked from a chain follows
    T = fusion
    out = {}
    for on in (True, False):
        T.set_fusion(on)
        x = T.Tensor.from_slice(normal((512, 384), 5), [512, 384])
        w = T.Tensor.from_slice((normal((384, 256), 6) / 20).astype(np.float32), [384, 256])
        b1 = T.Tensor.from_slice(normal(256, 7), [256])
        b2 = T.Tensor.from_slice(normal(256, 8), [256])
        T.Profile.reset()
        T.Profile.enable(True)
        h = x.matmul(w)
        z1 = h.add_tensor(b1)               # fork of the product
        r1 = z1.relu()                      # fork of the fork
        r2 = h.add_tensor(b2).relu()        # second consumer: the product runs here, once
        z1_read = z1.data()                 # the first fork, as its epilogue alone
        vals = (r1.data(), r2.data(), z1_read, h.data())
        T.Profile.enable(False)
        assert T.Profile.read(T.Profile.GEMM)["launches"] == 1, on
        out[on] = vals
    for name, u, v in zip(("relu(h+b1)", "relu(h+b2)", "h+b1", "h"), out[True], out[False]):
        assert_bits_equal(u, v, name)


@pytest.mark.parametrize("widths,batch", [([784, 1024, 10], 1024), ([256, 512, 512, 128], 1024), ([64, 96, 48], 33)])
def test_bias_gradients_come_out_of_the_weight_products(fusion, widths, batch):
    """With fusion on, each bias gradient (the column sum of the layer's
    output gradient, grad_fn/utils.rs:23-60) is written by the dW product that
    reads the same rows: no reduction launches in backward, and the bits of the
    separate column sum.  The GEMM launches are the same, except that a layer
    with at most 16 outputs whose dX is needed runs its dX and dW (with the
    bias gradient) as one launch (a launch group)."""
    T = fusion
    grads, counts = {}, {}
    for on in (True, False):
        T.set_fusion(on)
        ps, x, t = _mlp(T, widths, batch, 11)
        h = x
        n = len(ps) // 2
        for i in range(n):
            h = h.matmul(ps[2 * i]).add_tensor(ps[2 * i + 1])
            if i < n - 1:
                h = h.relu()
        loss = h.sub_tensor(t).pow_scalar(2.0).mean()
        loss.value()
        T.synchronize()
        T.Profile.reset()
        T.Profile.enable(True)
        loss.backward()
        T.synchronize()
        T.Profile.enable(False)
        counts[on] = (T.Profile.read(T.Profile.GEMM)["launches"], T.Profile.read(T.Profile.REDUCTION)["launches"])
        grads[on] = [p.grad_by_value().data() for p in ps]
        T.clear_gradients()
    for i, (a, b) in enumerate(zip(grads[True], grads[False])):
        assert_bits_equal(a, b, f"grad {i}")
    n = len(widths) - 1
    pairs = sum(1 for i in range(1, n) if widths[i + 1] <= 16)  # the first layer's dX is not computed
    assert counts[True] == (counts[False][0] - pairs, 0), counts
    assert counts[False][1] == n, counts


def test_bias_gradient_without_a_weight_product_runs_on_its_own(fusion):
    # W is constant: no dW product reads the rows, so the deferred column sum
    # runs by itself at the end of backward, with the same bits
    T = fusion
    vals = {}
    for on in (True, False):
        T.set_fusion(on)
        x = T.Tensor.from_slice(normal((300, 70), 12), [300, 70])
        w = T.Tensor.from_slice(normal((70, 40), 13), [70, 40])
        b = T.Tensor.from_slice(normal(40, 14), [40]).with_requires_grad()
        loss = x.matmul(w).add_tensor(b).relu().sum()
        loss.backward()
        vals[on] = b.grad_by_value().data()
        T.clear_gradients()
    assert_bits_equal(vals[True], vals[False], "bias grad")


@pytest.mark.parametrize("readme", [True, False])
def test_gradient_chains_are_applied_in_the_products(fusion, readme):
    """With fusion on, an output gradient that is a chain of elementwise ops
    over one buffer -- relu's backward of the seed in the README step
    (README.md:71-79), the MSE's gradient 2 * d * (1/n) of config 4 -- is
    applied by the products that read it, as an operand transform of that
    buffer (ts_hip_gemm_*_xf): the backward launches no elementwise pass, and
    every gradient has the bits of the op-by-op run."""
    T = fusion
    widths, batch = ([784, 128], 32) if readme else ([784, 1024, 10], 1024)
    grads, counts = {}, {}
    for on in (True, False):
        T.set_fusion(on)
        ps, x, t = _mlp(T, widths, batch, 13)
        h = x
        n = len(ps) // 2
        for i in range(n):
            h = h.matmul(ps[2 * i]).add_tensor(ps[2 * i + 1])
            if readme or i < n - 1:
                h = h.relu()
        loss = h.sum() if readme else h.sub_tensor(t).pow_scalar(2.0).mean()
        loss.value()
        T.synchronize()
        T.Profile.reset()
        T.Profile.enable(True)
        loss.backward()
        T.synchronize()
        T.Profile.enable(False)
        counts[on] = (T.Profile.read(T.Profile.GEMM)["launches"], T.Profile.read(T.Profile.ELEMENTWISE)["launches"])
        grads[on] = [p.grad_by_value().data() for p in ps]
        T.clear_gradients()
    for i, (a, b) in enumerate(zip(grads[True], grads[False])):
        assert_bits_equal(a, b, f"grad {i}")
    assert counts[True][1] == 0, counts
    # dW (+db) per layer; config 4's dX2 runs with dW2 (+db2) as one launch (a launch group)
    assert counts[True][0] == (1 if readme else 2), counts


@pytest.mark.parametrize("op", ["mul", "div"])
@pytest.mark.parametrize("loss", ["sum", "mean"])
def test_product_gradient_times_a_constant_buffer(fusion, op, loss):
    """y = (x . W) op B with B a buffer that needs no gradient: W's gradient
    reads go * B (or go / B) with go the seed's constant, a chain over B that
    the dW product applies to B as it loads it when the division is not
    checked for zeros (mul; a checked division runs its pass); the gradients
    have the bits of the op-by-op run either way."""
    T = fusion
    rng = np.random.default_rng(17)
    M, K, N = 96, 784, 128
    xv = rng.standard_normal((M, K)).astype(np.float32)
    wv = (rng.standard_normal((K, N)) / np.sqrt(K)).astype(np.float32)
    bv = rng.uniform(0.5, 2.0, (M, N)).astype(np.float32)
    grads, ew = {}, {}
    for on in (True, False):
        T.set_fusion(on)
        x = T.Tensor.from_slice(xv, [M, K])
        w = T.Tensor.from_slice(wv, [K, N]).with_requires_grad()
        b = T.Tensor.from_slice(bv, [M, N])
        y = getattr(x.matmul(w), f"{op}_tensor")(b)
        lv = getattr(y, loss)()
        lv.value()
        T.synchronize()
        T.Profile.reset()
        T.Profile.enable(True)
        lv.backward()
        T.synchronize()
        T.Profile.enable(False)
        ew[on] = T.Profile.read(T.Profile.ELEMENTWISE)["launches"]
        grads[on] = w.grad_by_value().data()
        T.clear_gradients()
    assert_bits_equal(grads[True], grads[False], f"{op} {loss} dW")
    if op == "mul":
        assert ew[True] == 0, ew
