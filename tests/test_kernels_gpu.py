"""Kernel-level parity of libts_hip.so against the CPU oracle, through the
C-ABI of include/ts_hip.h.  Bit-exact for elementwise ops, ReLU masks and
Adam; <= 1e-4 normwise relative error (max|d| / max|ref|) for GEMMs and
reductions, as the parity bar for this path states."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_bits_equal, max_rel, normal, sum_order_model, uniform
from gpu_util import Dev, ZeroIndex, hip, hip_check, sync

pytestmark = pytest.mark.gpu

SIZES = [1, 3, 7, 8, 31, 32, 33, 1000, (1 << 20) + 5]
SPECIAL = np.array([0.0, -0.0, 1.0, -1.0, 1e-45, -1e-45, 1e-38, 3.4e38, -3.4e38, np.inf,
                    -np.inf, np.nan, 0.5, 2.0, 1e30, -1e-30], dtype=np.float32)


def _with_special(x):
    x = x.copy()
    k = min(x.size, SPECIAL.size)
    x.reshape(-1)[:k] = SPECIAL[:k]
    return x


def _run(name, *args):
    hip_check(getattr(hip, name)(*args), name)
    sync()


@pytest.mark.parametrize("offset", [0, 1])
@pytest.mark.parametrize("n", SIZES)
def test_binary_elementwise_bit_exact(oracle, n, offset):
    print(f"[binary] n={n} offset={offset}", flush=True)
    a = _with_special(normal(n, 1))
    b = _with_special(normal(n, 2))[::-1].copy()
    da, db, do = Dev.of(a, offset), Dev.of(b, offset), Dev(n, offset)
    for name, ref in (("ts_hip_add", oracle.add), ("ts_hip_sub", oracle.sub), ("ts_hip_mul", oracle.mul)):
        _run(name, da.ptr, db.ptr, do.ptr, n, None)
        assert_bits_equal(do.get(), ref(a, b), name)
    bz = b.copy()
    bz[bz == 0] = 1.5
    dbz = Dev.of(bz, offset)
    _run("ts_hip_div", da.ptr, dbz.ptr, do.ptr, n, (n // 32) * 32, None, None)
    assert_bits_equal(do.get(), oracle.div(a, bz), "ts_hip_div")


@pytest.mark.parametrize("n", [1, 9, 1000, (1 << 20) + 3])
def test_unary_and_scalar_bit_exact(oracle, n):
    print(f"[unary] n={n}", flush=True)
    x = _with_special(normal(n, 3))
    dx, do = Dev.of(x), Dev(n)
    _run("ts_hip_relu", dx.ptr, do.ptr, n, None)
    assert_bits_equal(do.get(), oracle.relu(x), "relu")
    _run("ts_hip_neg", dx.ptr, do.ptr, n, (n // 8) * 8, None)
    assert_bits_equal(do.get(), oracle.neg(x), "neg")
    _run("ts_hip_pow_scalar", dx.ptr, 2.0, do.ptr, n, None)
    assert_bits_equal(do.get(), oracle.pow2(x), "pow2")
    ax = np.abs(x)
    dax = Dev.of(ax)
    _run("ts_hip_pow_scalar", dax.ptr, 0.5, do.ptr, n, None)
    assert_bits_equal(do.get(), np.sqrt(ax), "pow 0.5 (IEEE sqrt)")
    for s in (2.0, -0.5, 1e-3):
        for name, ref in (("ts_hip_add_scalar", oracle.add_scalar), ("ts_hip_sub_scalar", oracle.sub_scalar),
                          ("ts_hip_mul_scalar", oracle.mul_scalar), ("ts_hip_div_scalar", oracle.div_scalar)):
            _run(name, dx.ptr, s, do.ptr, n, None)
            assert_bits_equal(do.get(), ref(x, s), f"{name}({s})")
    _run("ts_hip_fill", do.ptr, -2.5, n, None)
    assert np.all(do.get() == np.float32(-2.5))
    _run("ts_hip_copy", dx.ptr, do.ptr, n, None)
    assert_bits_equal(do.get(), x, "copy")
    src = Dev.of(np.array([0.75], np.float32))
    _run("ts_hip_fill_from_device", do.ptr, src.ptr, 0.0, 0, n, None)
    assert np.all(do.get() == np.float32(0.75))
    base = np.float32(1.0) / np.float32(n)
    _run("ts_hip_fill_from_device", do.ptr, src.ptr, float(base), 1, n, None)
    assert np.all(do.get() == np.float32(base * np.float32(0.75)))


def test_negate_tail_zero_sign():
    z = np.zeros(13, np.float32)
    dz, do = Dev.of(z), Dev(13)
    _run("ts_hip_neg", dz.ptr, do.ptr, 13, 8, None)
    out = do.get()
    assert not np.any(np.signbit(out[:8])) and np.all(np.signbit(out[8:]))


@pytest.mark.parametrize("n", [5, 64, 1000, (1 << 20) + 7])
def test_backward_elementwise_bit_exact(oracle, n):
    print(f"[backward] n={n}", flush=True)
    x = _with_special(normal(n, 4))
    go = normal(n, 5)
    a = normal(n, 6)
    b = uniform(n, 0.5, 2.0, 7) * np.where(np.arange(n) % 3 == 0, -1, 1).astype(np.float32)
    dx, dgo, da, db = Dev.of(x), Dev.of(go), Dev.of(a), Dev.of(b)
    o1, o2 = Dev(n), Dev(n)
    _run("ts_hip_relu_backward", dx.ptr, dgo.ptr, o1.ptr, n, None)
    assert_bits_equal(o1.get(), oracle.relu_bwd(x, go), "relu_backward")
    # a saved relu OUTPUT gives the same mask as its input
    dy = Dev.of(oracle.relu(x))
    _run("ts_hip_relu_backward", dy.ptr, dgo.ptr, o1.ptr, n, None)
    assert_bits_equal(o1.get(), oracle.relu_bwd(x, go), "relu_backward from output")
    _run("ts_hip_pow_backward", dx.ptr, dgo.ptr, o1.ptr, n, 2.0, None)
    assert_bits_equal(o1.get(), oracle.pow_bwd(x, go, 2.0), "pow_backward")
    _run("ts_hip_mul_backward", dgo.ptr, da.ptr, db.ptr, o1.ptr, o2.ptr, n, None)
    assert_bits_equal(o1.get(), oracle.mul(go, b), "mul_backward ga")
    assert_bits_equal(o2.get(), oracle.mul(go, a), "mul_backward gb")
    _run("ts_hip_div_backward", dgo.ptr, da.ptr, db.ptr, o1.ptr, o2.ptr, n, (n // 8) * 8,
         (n // 32) * 32, None, None)
    assert_bits_equal(o1.get(), oracle.div(go, b), "div_backward ga")
    want_gb = oracle.neg(oracle.div(oracle.mul(go, a), oracle.mul(b, b)))
    assert_bits_equal(o2.get(), want_gb, "div_backward gb")


@pytest.mark.parametrize("rows,cols", [(1, 1), (32, 128), (1024, 10), (33, 7), (8192, 4096)])
def test_row_broadcast_bit_exact(oracle, rows, cols):
    print(f"[row_broadcast] {rows}x{cols}", flush=True)
    x = normal((rows, cols), 8)
    v = uniform(cols, 0.5, 2.0, 9)
    dx, dv, do = Dev.of(x), Dev.of(v), Dev(rows * cols)
    _run("ts_hip_bias_add", dx.ptr, dv.ptr, do.ptr, rows, cols, 0, None)
    assert_bits_equal(do.get((rows, cols)), oracle.bias_add(x, v), "bias_add")
    vb = np.broadcast_to(v, x.shape)
    refs = {0: oracle.add, 1: oracle.sub, 2: oracle.mul, 3: oracle.div}
    for op, ref in refs.items():
        for vec_first in (0, 1):
            _run("ts_hip_row_broadcast", op, dx.ptr, dv.ptr, do.ptr, rows, cols, vec_first, 0, None, None)
            want = ref(vb, x) if vec_first else ref(x, vb)
            assert_bits_equal(do.get((rows, cols)), want, f"row_broadcast op={op} vec_first={vec_first}")


def test_division_zero_index_reports_tail_only():
    n = 40
    a = np.ones(n, np.float32)
    b = np.ones(n, np.float32)
    b[3] = 0.0      # inside the reference's unchecked 32-wide body
    da, db, do = Dev.of(a), Dev.of(b), Dev(n)
    zi = ZeroIndex()
    _run("ts_hip_div", da.ptr, db.ptr, do.ptr, n, 32, zi.ptr, None)
    assert zi.value() is None
    b[37] = 0.0
    b[35] = 0.0
    db.put(b)
    _run("ts_hip_div", da.ptr, db.ptr, do.ptr, n, 32, zi.ptr, None)
    assert zi.value() == 35


@pytest.mark.parametrize("n", [0, 1, 5, 4096, 100003, 1 << 26])
def test_sum_and_mean(oracle, n):
    print(f"[sum] n={n}", flush=True)
    x = normal(n, 10)
    dx = Dev.of(x)
    ws = hip.ts_hip_sum_workspace_floats(n)
    dws, dout = Dev(ws), Dev(1)
    _run("ts_hip_sum", dx.ptr if n else None, n, dout.ptr, dws.ptr, ws, None)
    exact = oracle.sum_f64(x)
    scale = max(float(np.sum(np.abs(x), dtype=np.float64)), 1e-30)
    assert abs(float(dout.get()[0]) - exact) <= 1e-6 * scale + 1e-30
    _run("ts_hip_mean", dx.ptr if n else None, n, dout.ptr, dws.ptr, ws, None)
    if n:
        assert abs(float(dout.get()[0]) - exact / n) <= 1e-6 * scale / n
    else:
        assert float(dout.get()[0]) == 0.0
    if n:  # too small a workspace is refused, not overrun
        assert hip.ts_hip_sum(dx.ptr, n, dout.ptr, dws.ptr, ws - 1, None) == 100003


# the one-workgroup form (up to 16 first-pass workgroups, aligned) and the two
# passes give the partition's bits, aligned or not
@pytest.mark.parametrize("offset", [0, 1])
@pytest.mark.parametrize("n", [1, 3, 4, 5, 1024, 1027, 4096, 10240, 15361, 16384, 16385, 100003, 1 << 21,
                               (1 << 21) + 4, 1 << 22, (1 << 22) + 5, 1 << 26])
def test_sum_bits_follow_the_partition(n, offset):
    print(f"[sum bits] n={n} offset={offset}", flush=True)
    x = normal(n, 12)
    dx = Dev.of(x, offset)
    ws = hip.ts_hip_sum_workspace_floats(n)
    dws, dout = Dev(ws), Dev(1)
    for name, mean in (("ts_hip_sum", False), ("ts_hip_mean", True)):
        _run(name, dx.ptr, n, dout.ptr, dws.ptr, ws, None)
        want = sum_order_model(x, mean=mean, aligned=offset == 0)
        assert_bits_equal(dout.get(), np.array([want], np.float32), f"{name} n={n} offset={offset}")


def test_sum_bits_with_longer_runs():
    # past 2^28 inputs a first-pass thread takes more than four groups (five here)
    n = (1 << 28) + 12
    print(f"[sum bits] n={n}", flush=True)
    x = normal(n, 15)
    dx = Dev.of(x)
    ws = hip.ts_hip_sum_workspace_floats(n)
    dws, dout = Dev(ws), Dev(1)
    want = sum_order_model(x)
    _run("ts_hip_sum", dx.ptr, n, dout.ptr, dws.ptr, ws, None)
    assert_bits_equal(dout.get(), np.array([want], np.float32), f"sum n={n}")
    _run("ts_hip_mean", dx.ptr, n, dout.ptr, dws.ptr, ws, None)
    assert_bits_equal(dout.get(), np.array([want / np.float32(n)], np.float32), f"mean n={n}")


@pytest.mark.parametrize("offset", [0, 1])
@pytest.mark.parametrize("n", [1, 5, 1024, 4096, 8192, 8193, 16384, 100003, (1 << 22) + 3])
def test_dot_bits_follow_the_partition(n, offset):
    print(f"[dot bits] n={n} offset={offset}", flush=True)
    a, b = normal(n, 13), normal(n, 14)
    da, db = Dev.of(a, offset), Dev.of(b, offset)
    ws = hip.ts_hip_sum_workspace_floats(n)
    dws, dout = Dev(ws), Dev(1)
    _run("ts_hip_dot", da.ptr, db.ptr, n, dout.ptr, dws.ptr, ws, None)
    want = sum_order_model(a, aligned=offset == 0, times=b)
    assert_bits_equal(dout.get(), np.array([want], np.float32), f"dot n={n} offset={offset}")


def test_sum_known_answers():
    for xs, want in (([i * 0.5 for i in range(6)], 7.5), ([1, 2, 3, 4, 5, 6], 21.0),
                     (list(range(24)), 276.0)):
        x = np.array(xs, np.float32)
        dx, dws, dout = Dev.of(x), Dev(hip.ts_hip_sum_workspace_floats(x.size)), Dev(1)
        _run("ts_hip_sum", dx.ptr, x.size, dout.ptr, dws.ptr, dws.n, None)
        assert float(dout.get()[0]) == want


@pytest.mark.parametrize("rows,cols", [(1, 1), (2, 4), (32, 128), (1024, 10), (33, 7), (1024, 1024),
                                       (8192, 4096), (5000, 1001), (300, 4100), (8193, 260), (17, 70000)])
def test_sum_dim0(oracle, rows, cols):
    print(f"[sum_dim0] {rows}x{cols}", flush=True)
    x = normal((rows, cols), 11)
    ws = hip.ts_hip_sum_dim0_workspace_floats(rows, cols)
    dx, dws, do = Dev.of(x), Dev(ws), Dev(cols)
    _run("ts_hip_sum_dim0", dx.ptr, rows, cols, do.ptr, dws.ptr, ws, None)
    want = oracle.sum_dim0_f64(x)
    got = do.get()
    assert max_rel(got, want) <= 1e-6
    assert_bits_equal(got, oracle.sum_dim0_chunked(x), f"sum_dim0 {rows}x{cols}")   # the fixed order
    if rows * cols <= 1 << 16:
        assert max_rel(got, oracle.sum_dim0(x)) <= 1e-4   # the reference's fp32 row order


GEMM_SHAPES = [(1, 1, 1), (2, 2, 2), (32, 128, 784), (784, 128, 32), (129, 127, 33), (1024, 10, 1024),
               (1024, 1024, 10), (1024, 1024, 784), (784, 1024, 1024), (300, 200, 4096),
               # N <= 16 (the narrow kernel): ragged rows, K not a multiple of 4, ragged wave ranges
               (1000, 16, 777), (63, 1, 4096), (5000, 13, 65), (70, 9, 3),
               # N <= 16 over few rows with a long K: the sliced skinny kernel and its slice sum
               (64, 10, 16384),
               # K <= 16 (one k tile, operands straight to registers): ragged edges, K = 16 and 1
               (129, 127, 16), (100, 33, 1),
               # few output tiles and a long K: the narrow kernel's column blocks (ragged N), and
               # split-K past its K
               (40, 200, 1000), (32, 128, 16384)]


def _gemm_case(oracle, ta, tb, M, N, K, seed, check_rows=None):
    a = normal((K, M) if ta else (M, K), seed)
    b = normal((N, K) if tb else (K, N), seed + 1)
    da, db, dc = Dev.of(a), Dev.of(b), Dev(M * N)
    lda = M if ta else K
    ldb = K if tb else N
    _run("ts_hip_gemm", int(ta), int(tb), M, N, K, da.ptr, lda, db.ptr, ldb, dc.ptr, N, None)
    got = dc.get((M, N))
    if check_rows is None:
        want = oracle.gemm_f64(a, b, ta=ta, tb=tb)
        return got, want
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(seed).integers(0, M, check_rows)]))
    a_rows = (a[:, rows].T if ta else a[rows, :]).copy()
    want = oracle.gemm_f64(a_rows, b, ta=False, tb=tb)
    return got[rows], want


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_gemm_layouts(oracle, ta, tb, M, N, K):
    print(f"[gemm] ta={ta} tb={tb} M={M} N={N} K={K}", flush=True)
    got, want = _gemm_case(oracle, ta, tb, M, N, K, seed=M + N + K)
    assert max_rel(got, want) <= 1e-4, (M, N, K, ta, tb)


def test_gemm_known_answer():
    a = np.array([[1, 2], [3, 4]], np.float32)
    b = np.array([[5, 6], [7, 8]], np.float32)
    da, db, dc = Dev.of(a), Dev.of(b), Dev(4)
    _run("ts_hip_matmul", da.ptr, db.ptr, dc.ptr, 2, 2, 2, None)
    assert dc.get().tolist() == [19.0, 22.0, 43.0, 50.0]


@pytest.mark.parametrize("ta,tb,M,N,K", [(0, 0, 8192, 4096, 4096), (0, 1, 8192, 4096, 4096),
                                         (1, 0, 4096, 4096, 8192)])
def test_gemm_full_size_every_element(oracle, ta, tb, M, N, K):
    # BASELINE config 5 contractions at their real shape: forward X.W, dX = dY.W^T,
    # dW = X^T.dY, each on the LDS-DMA kernel with its XCD-renumbered grid;
    # every element of C against f64, so an unwritten or mis-placed tile fails
    print(f"[gemm full] ta={ta} tb={tb} M={M} N={N} K={K}", flush=True)
    got, want = _gemm_case(oracle, bool(ta), bool(tb), M, N, K, seed=5)
    assert got.shape == want.shape == (M, N)
    assert max_rel(got, want) <= 1e-4
    # per element, against the RMS of C for entries smaller than it
    tol = 1e-4 * np.maximum(np.abs(want), np.sqrt(np.mean(want * want)))
    assert np.all(np.abs(got.astype(np.float64) - want) <= tol)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(4100, 4100, 100), (4100, 4097, 103), (4096, 4096, 9), (100, 65536, 64),
                                   (65536, 100, 40)])
def test_gemm_large_grid_edges(oracle, ta, tb, M, N, K):
    # enough 256x256 tiles to fill the chip: aligned layouts take the LDS-DMA
    # kernel (clamped edge rows, a partial last k tile), the others the
    # register-staged one, K <= 16 the one-tile kernel; f64 check on sampled
    # rows, always including the last
    print(f"[gemm grid] ta={ta} tb={tb} M={M} N={N} K={K}", flush=True)
    got, want = _gemm_case(oracle, bool(ta), bool(tb), M, N, K, seed=11, check_rows=16)
    assert max_rel(got, want) <= 1e-4


def test_gemm_rejects_bad_leading_dimension():
    d = Dev(64)
    assert hip.ts_hip_gemm(0, 0, 8, 8, 8, d.ptr, 4, d.ptr, 8, d.ptr, 8, None) == 100001


@pytest.mark.parametrize("n", [1, 7, 8, 9, 1000, (1 << 20) + 3])
@pytest.mark.parametrize("mode", ["plain", "weight_decay", "amsgrad"])
def test_adam_bit_exact(oracle, n, mode):
    print(f"[adam] n={n} mode={mode}", flush=True)
    p = normal(n, 12)
    g = normal(n, 13, 0.1)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    wd = 0.01 if mode == "weight_decay" else 0.0
    vm = np.zeros(n, np.float32) if mode == "amsgrad" else None
    dp, dg, dm, dv = Dev.of(p), Dev.of(g), Dev.of(m), Dev.of(v)
    dvm = Dev.of(vm) if vm is not None else None
    for step in range(1, 11):
        g = normal(n, 100 + step, 0.1)
        dg.put(g)
        _run("ts_hip_adam_step", dp.ptr, dg.ptr, dm.ptr, dv.ptr, dvm.ptr if dvm else None, n, 1e-3,
             0.9, 0.999, 1e-8, wd, step, (n // 8) * 8, int(step == 1), None)
        oracle.adam_step(p, g, m, v, step, weight_decay=wd, vmax=vm, amsgrad_first=(step == 1))
    assert_bits_equal(dp.get(), p, "p")
    assert_bits_equal(dm.get(), m, "m")
    assert_bits_equal(dv.get(), v, "v")
    if vm is not None:
        assert_bits_equal(dvm.get(), vm, "v_hat_max")


def test_adam_100_steps_bit_exact(oracle):
    # BASELINE config 3 (Adam alone, constant gradient set once, m = v = 0) at 2^22 params
    n = 1 << 22
    p = normal(n, 14)
    g = normal(n, 15, 0.1)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    dp, dg, dm, dv = Dev.of(p), Dev.of(g), Dev.of(m), Dev.of(v)
    for step in range(1, 101):
        hip_check(hip.ts_hip_adam_step(dp.ptr, dg.ptr, dm.ptr, dv.ptr, None, n, 1e-3, 0.9, 0.999, 1e-8,
                                       0.0, step, n, 0, None), "adam")
        oracle.adam_step(p, g, m, v, step)
    sync()
    assert_bits_equal(dp.get(), p, "p after 100 steps")
    assert_bits_equal(dv.get(), v, "v after 100 steps")


def test_adam_large_tensors_bit_exact(oracle):
    # tensors of 2^26 parameters and more take the non-temporal load / store
    # path (one tensor alone, then in one launch beside a small tensor, which
    # keeps the ordinary path); AMSGrad and weight decay on, odd size for the tail
    from train_station_amd._ffi import AdamParam
    import ctypes
    n = (1 << 26) + 5
    print(f"[adam] large n={n}", flush=True)
    p = normal(n, 16)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    vm = np.zeros(n, np.float32)
    small = [normal(1000, 17), np.zeros(1000, np.float32), np.zeros(1000, np.float32)]
    dp, dm, dv, dvm = Dev.of(p), Dev.of(m), Dev.of(v), Dev.of(vm)
    ds = [Dev.of(a) for a in small]
    for step in range(1, 4):
        g = normal(n, 400 + step, 0.1)
        dg = Dev.of(g)
        if step < 3:
            _run("ts_hip_adam_step", dp.ptr, dg.ptr, dm.ptr, dv.ptr, dvm.ptr, n, 1e-3, 0.9, 0.999, 1e-8, 0.01,
                 step, (n // 8) * 8, int(step == 1), None)
        else:
            gs = normal(1000, 500, 0.1)
            dgs = Dev.of(gs)
            arr = (AdamParam * 2)()
            arr[0] = AdamParam(dp.ptr, dg.ptr, dm.ptr, dv.ptr, dvm.ptr, n, 0)
            arr[1] = AdamParam(ds[0].ptr, dgs.ptr, ds[1].ptr, ds[2].ptr, None, 1000, 0)
            _run("ts_hip_adam_step_multi", ctypes.cast(arr, ctypes.c_void_p), 2, 1e-3, 0.9, 0.999, 1e-8, 0.01,
                 step, None)
        oracle.adam_step(p, g, m, v, step, weight_decay=0.01, vmax=vm, amsgrad_first=(step == 1))
    # the small tensor stepped once (its first step, without AMSGrad)
    oracle.adam_step(small[0], gs, small[1], small[2], 3, weight_decay=0.01)
    assert_bits_equal(dp.get(), p, "p")
    assert_bits_equal(dm.get(), m, "m")
    assert_bits_equal(dv.get(), v, "v")
    assert_bits_equal(dvm.get(), vm, "v_hat_max")
    assert_bits_equal(ds[0].get(), small[0], "small p")
    assert_bits_equal(ds[2].get(), small[2], "small v")


def test_adam_multi_matches_per_parameter(oracle):
    # one launch over several parameters (different sizes, tails, AMSGrad
    # first/later steps, weight decay) gives the per-parameter bits
    from train_station_amd._ffi import AdamParam
    import ctypes
    # an empty tensor in the middle and one with unaligned buffers (scalar path)
    # check the flat grid's tensor lookup
    sizes = [1, 7, 9, 4096, 0, 1000, (1 << 18) + 3, 4099]
    offs = [0, 0, 0, 0, 0, 0, 0, 1]
    for wd, ams in ((0.0, False), (0.01, True)):
        host = []
        for i, n in enumerate(sizes):
            p = normal(n, 200 + i)
            m = np.zeros(n, np.float32)
            v = np.zeros(n, np.float32)
            vm = np.zeros(n, np.float32) if ams else None
            host.append([p, m, v, vm])
        dev = [[Dev.of(h[0], offs[i]), Dev.of(h[1], offs[i]), Dev.of(h[2], offs[i]),
                Dev.of(h[3], offs[i]) if ams else None] for i, h in enumerate(host)]
        for step in range(1, 4):
            grads = [normal(n, 300 + 10 * step + i, 0.1) for i, n in enumerate(sizes)]
            dg = [Dev.of(g, offs[i]) for i, g in enumerate(grads)]
            arr = (AdamParam * len(sizes))()
            for i, n in enumerate(sizes):
                d = dev[i]
                arr[i] = AdamParam(d[0].ptr, dg[i].ptr, d[1].ptr, d[2].ptr, d[3].ptr if ams else None, n,
                                   int(step == 1))
            _run("ts_hip_adam_step_multi", ctypes.cast(arr, ctypes.c_void_p), len(sizes), 1e-3, 0.9, 0.999,
                 1e-8, wd, step, None)
            for i, n in enumerate(sizes):
                h = host[i]
                oracle.adam_step(h[0], grads[i], h[1], h[2], step, weight_decay=wd, vmax=h[3],
                                 amsgrad_first=(step == 1))
        for i in range(len(sizes)):
            assert_bits_equal(dev[i][0].get(), host[i][0], f"p[{i}] wd={wd} ams={ams}")
            assert_bits_equal(dev[i][2].get(), host[i][2], f"v[{i}] wd={wd} ams={ams}")
    assert hip.ts_hip_adam_step_multi(None, 17, 1e-3, 0.9, 0.999, 1e-8, 0.0, 1, None) == 100001


def test_adam_ticket_launches_read_their_own_table_entries():
    # five launches on one set of tickets read table entries 0..4: the bits
    # of eager steps 3..7
    import ctypes
    from train_station_amd._ffi import AdamParam
    sizes = [4099, 10, (1 << 17) + 5]
    first = 3
    table = np.zeros(2 * 5, np.float32)
    table_c = table.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    hip_check(hip.ts_hip_adam_bias_corrections(ctypes.c_float(0.9), ctypes.c_float(0.999), first, 5, table_c))
    dtable = Dev.of(table)
    res = {}
    for mode in ("eager", "ticket"):
        ps = [Dev.of(normal(n, 400 + i)) for i, n in enumerate(sizes)]
        ms = [Dev.of(np.zeros(n, np.float32)) for n in sizes]
        vs = [Dev.of(np.zeros(n, np.float32)) for n in sizes]
        for k in range(5):
            gs = [Dev.of(normal(n, 500 + 10 * k + i, 0.1)) for i, n in enumerate(sizes)]
            arr = (AdamParam * len(sizes))()
            for i, n in enumerate(sizes):
                arr[i] = AdamParam(ps[i].ptr, gs[i].ptr, ms[i].ptr, vs[i].ptr, None, n, 0)
            if k == 0:
                nw = hip.ts_hip_adam_multi_waves(ctypes.cast(arr, ctypes.c_void_p), len(sizes))
                ticket = Dev.of(np.zeros(nw, np.float32))
            if mode == "eager":
                _run("ts_hip_adam_step_multi", ctypes.cast(arr, ctypes.c_void_p), len(sizes), 1e-3, 0.9, 0.999,
                     1e-8, 0.0, first + k, None)
            else:
                _run("ts_hip_adam_step_multi_ticket", ctypes.cast(arr, ctypes.c_void_p), len(sizes), 1e-3, 0.9,
                     0.999, 1e-8, 0.0, dtable.ptr, ticket.ptr, None)
            sync()
        res[mode] = [p.get() for p in ps] + [v.get() for v in vs]
    for i, (a, b) in enumerate(zip(res["ticket"], res["eager"])):
        assert_bits_equal(a, b, f"array {i}")
    # every wave counted the 5 launches in its own word
    counts = np.frombuffer(ticket.get().tobytes(), np.uint32)
    assert counts.size >= len(sizes) * 4 and np.all(counts == 5)
    assert hip.ts_hip_adam_step_multi_ticket(None, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, dtable.ptr, None, None) != 0
