"""Pins the CPU oracle (oracle/ts_oracle.c) against checks that do not restate it:
the reference's own known answers, torch CPU (an independent IEEE fp32 /
float64 implementation), closed forms and brute force.  CPU only."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import assert_bits_equal, bits, golden, max_rel, normal, uniform

SPECIAL = np.array([0.0, -0.0, 1.0, -1.0, 1e-45, -1e-45, 1e-38, 3.4e38, -3.4e38, np.inf, -np.inf,
                    0.5, 2.0, 1e30, -1e-30, 7.0], dtype=np.float32)


def _inputs(n, seed):
    a = normal(n, seed)
    b = normal(n, seed + 1)
    a[: SPECIAL.size] = SPECIAL
    b[: SPECIAL.size] = SPECIAL[::-1]
    return a, b


@pytest.mark.parametrize("n", [1, 7, 8, 33, 1000])
def test_binary_ops_match_torch_bits(oracle, n):
    a, b = _inputs(max(n, 16), 3)
    a, b = a[:n], b[:n]
    ta, tb = torch.from_numpy(a), torch.from_numpy(b)
    assert_bits_equal(oracle.add(a, b), (ta + tb).numpy(), "add")
    assert_bits_equal(oracle.sub(a, b), (ta - tb).numpy(), "sub")
    assert_bits_equal(oracle.mul(a, b), (ta * tb).numpy(), "mul")
    nz = b.copy()
    nz[nz == 0] = 3.0
    assert_bits_equal(oracle.div(a, nz), (ta / torch.from_numpy(nz)).numpy(), "div")


def test_scalar_ops_match_torch_bits(oracle):
    x = normal(257, 5)
    tx = torch.from_numpy(x)
    for s in (2.0, -0.5, 1e-3, 3.0):
        sf = torch.tensor(s, dtype=torch.float32)
        assert_bits_equal(oracle.add_scalar(x, s), (tx + sf).numpy(), "add_scalar")
        assert_bits_equal(oracle.sub_scalar(x, s), (tx - sf).numpy(), "sub_scalar")
        assert_bits_equal(oracle.mul_scalar(x, s), (tx * sf).numpy(), "mul_scalar")
        assert_bits_equal(oracle.div_scalar(x, s), (tx / sf).numpy(), "div_scalar")


def test_pow2_and_bias_add_match_torch_bits(oracle):
    x = normal((37, 41), 7)
    x.reshape(-1)[:SPECIAL.size] = SPECIAL
    assert_bits_equal(oracle.pow2(x), (torch.from_numpy(x) * torch.from_numpy(x)).numpy(), "pow2")
    bias = normal(41, 8)
    want = (torch.from_numpy(x) + torch.from_numpy(bias)).numpy()
    assert_bits_equal(oracle.bias_add(x, bias), want, "bias_add")
    assert_bits_equal(oracle.bias_add(x, bias, bias_first=True), want, "bias_add (bias first)")


def test_relu_known_answers_and_ieee_cases(oracle):
    ka = golden("known_answers.json")["relu_forward"]          # relu.rs:280-291
    assert_bits_equal(oracle.relu(np.array(ka["x"], np.float32)), np.array(ka["out"], np.float32))
    lt = golden("ltv_patterns.json")["relu"]                   # LibTorch pattern, x[5] == 0
    x = np.array(lt["x"], np.float32)
    assert x[5] == 0.0
    assert_bits_equal(oracle.relu(x), np.array(lt["out"], np.float32), "relu pattern")
    # `if v > 0.0 { v } else { 0.0 }`: -0 and NaN give +0 (both fail the comparison)
    out = oracle.relu(np.array([-0.0, np.nan, -np.inf, np.inf, 1e-45], np.float32))
    assert_bits_equal(out, np.array([0.0, 0.0, 0.0, np.inf, 1e-45], np.float32), "relu ieee")


def test_negate_zero_sign_rule(oracle):
    # utils.rs:847-870: 0.0 - x on the 8-wide body gives +0 for +/-0; -x on the tail flips the sign
    z = np.zeros(11, np.float32)
    out = oracle.neg(z)
    assert np.all(np.signbit(out[8:])) and not np.any(np.signbit(out[:8]))
    nz = -np.zeros(11, np.float32)
    out = oracle.neg(nz)
    assert not np.any(np.signbit(out))
    x = normal(1003, 9)
    assert_bits_equal(oracle.neg(x), (-torch.from_numpy(x)).numpy(), "neg of nonzero values")


def test_division_by_zero_only_outside_unrolled_body(oracle):
    # ops/div.rs:378-417: the 32-wide unrolled body divides without checking
    a = np.ones(40, np.float32)
    b = np.ones(40, np.float32)
    b[3] = 0.0
    out = oracle.div(a, b)
    assert np.isinf(out[3])
    b[35] = 0.0
    with pytest.raises(oracle.DivisionByZero, match="index 35"):
        oracle.div(a, b)
    with pytest.raises(oracle.DivisionByZero):
        oracle.div_scalar(a, 0.0)


def test_backward_elementwise_match_torch_autograd(oracle):
    x = normal(513, 11)
    x[:4] = [0.0, -0.0, 1e-45, -1e-45]
    go = normal(513, 12)
    tx = torch.from_numpy(x.copy()).requires_grad_()
    torch.relu(tx).backward(torch.from_numpy(go))
    assert_bits_equal(oracle.relu_bwd(x, go), tx.grad.numpy(), "relu backward")
    tx = torch.from_numpy(x.copy()).requires_grad_()
    tx.pow(2.0).backward(torch.from_numpy(go))        # torch: go * (2 * x.pow(1))
    got = oracle.pow_bwd(x, go, 2.0)                   # pow.rs: go * (2 * powf(x, 1))
    assert_bits_equal(got, tx.grad.numpy(), "pow2 backward")


def test_sum_known_answers(oracle):
    ka = golden("known_answers.json")
    for key in ("sum_forward", "sum_21", "sum_276"):
        case = ka[key]
        got = oracle.sum_(np.array(case["x"], np.float32))
        assert abs(float(got) - case["sum"]) <= case.get("tol", 0.0), key
    for key in ("mean_forward", "mean_3_5"):
        case = ka[key]
        got = oracle.mean(np.array(case["x"], np.float32))
        assert abs(float(got) - case["mean"]) <= case["tol"], key


def test_sum_grouping_of_four(oracle):
    # sum.rs:94-105 adds each group of four before touching the accumulator:
    # acc = 1e8 + (((2+2)+2)+2) = 100000008, while a plain running sum loses every 2.
    x = np.array([1e8, 0, 0, 0, 2, 2, 2, 2], np.float32)
    assert float(oracle.sum_(x)) == 100000008.0
    running = np.float32(0)
    for v in x:
        running = np.float32(running + v)
    assert float(running) == 1e8


@pytest.mark.parametrize("n", [0, 1, 3, 4, 5, 4096, 100003])
def test_sum_error_bound_against_fsum(oracle, n):
    x = normal(n, 13)
    exact = math.fsum(float(v) for v in x)
    bound = (n + 1) * np.finfo(np.float32).eps * float(np.sum(np.abs(x), dtype=np.float64)) + 1e-30
    assert abs(float(oracle.sum_(x)) - exact) <= bound
    assert abs(oracle.sum_f64(x) - exact) <= 1e-9 * (1 + abs(exact)) + 1e-6 * n * 1e-10


def test_sum_dim0_against_torch(oracle):
    x = normal((300, 67), 14)
    want = torch.from_numpy(x).double().sum(0).numpy()
    assert max_rel(oracle.sum_dim0(x), want) < 1e-5
    assert max_rel(oracle.sum_dim0_f64(x), want) < 1e-12
    ints = np.arange(12, dtype=np.float32).reshape(4, 3)
    assert oracle.sum_dim0(ints).tolist() == [18.0, 22.0, 26.0]


def test_sum_dim0_chunked_order(oracle):
    """The device's column-sum order, pinned by what fixes it independently:
    a brute-force pure-Python restatement on small inputs (chunk sums from
    +0 in row order, groups of 8 chunk sums, then the groups), exact integer
    sums, the f64 sum to within rounding, and the special values (all -0
    gives +0; a row past a chunk boundary starts a new chunk, which changes
    the bits of a cancelling sum)."""
    def brute(x, w=None):
        rows, cols = x.shape
        out = []
        for c in range(cols):
            chunk_sums = []
            for c0 in range(0, rows, oracle.COLSUM_ROWS):
                s = 0.0
                for r in range(c0, min(c0 + oracle.COLSUM_ROWS, rows)):
                    s += (1.0 if w is None else float(w[r])) * float(x[r, c])
                chunk_sums.append(s)
            total = 0.0
            for g0 in range(0, len(chunk_sums), oracle.COLSUM_GROUP):
                grp = 0.0
                for s in chunk_sums[g0:g0 + oracle.COLSUM_GROUP]:
                    grp += s
                total += grp
            out.append(total)
        return np.array(out, dtype=np.float64).astype(np.float32)

    for rows, cols, seed in ((1, 3, 1), (63, 5, 2), (64, 4, 3), (65, 7, 4), (200, 9, 5), (1100, 3, 6)):
        x = normal((rows, cols), seed)
        w = normal(rows, seed + 50)
        assert bits(oracle.sum_dim0_chunked(x)).tolist() == bits(brute(x)).tolist()
        assert bits(oracle.sum_dim0_chunked(x, w)).tolist() == bits(brute(x, w)).tolist()
        assert max_rel(oracle.sum_dim0_chunked(x), oracle.sum_dim0_f64(x)) < 1e-6
    ints = np.arange(12, dtype=np.float32).reshape(4, 3)
    assert oracle.sum_dim0_chunked(ints).tolist() == [18.0, 22.0, 26.0]
    negz = np.full((130, 2), -0.0, np.float32)
    assert bits(oracle.sum_dim0_chunked(negz)).tolist() == [0, 0]
    # 1 + 2^-30 * 64 rows then -1: chunked, the small terms are kept in the
    # first chunk's f64 sum; a flat fp32 sum would lose them
    x = np.zeros((65, 1), np.float32)
    x[0, 0] = 1.0
    x[1:64, 0] = 2.0 ** -30
    x[64, 0] = -1.0
    assert float(oracle.sum_dim0_chunked(x)[0]) == np.float32(63 * 2.0 ** -30)
    # 10 chunks: 1, seven zeros, then 2^60 and -2^60.  Groups of 8: the first
    # group is 1, the second 2^60 - 2^60 = 0, total 1; chunk by chunk the 1
    # would be lost in 1 + 2^60 (f64) and the total would be 0
    x = np.zeros((10 * 64, 1), np.float32)
    x[0, 0] = 1.0
    x[64 * 8, 0] = 2.0 ** 60
    x[64 * 9, 0] = -(2.0 ** 60)
    assert float(oracle.sum_dim0_chunked(x)[0]) == 1.0


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm_layouts_against_torch_and_brute_force(oracle, ta, tb):
    M, N, K = 13, 7, 19
    a = normal((K, M) if ta else (M, K), 15)
    b = normal((N, K) if tb else (K, N), 16)
    A = torch.from_numpy(a).double()
    B = torch.from_numpy(b).double()
    want = (A.T if ta else A) @ (B.T if tb else B)
    got = oracle.gemm_f64(a, b, ta=ta, tb=tb)
    assert np.allclose(got, want.numpy(), rtol=1e-12, atol=1e-12)
    # brute force on a corner
    Am = a.T if ta else a
    Bm = b.T if tb else b
    for i, j in ((0, 0), (M - 1, N - 1), (5, 3)):
        s = sum(float(Am[i, k]) * float(Bm[k, j]) for k in range(K))
        assert abs(got[i, j] - s) < 1e-9
    got32 = oracle.gemm_f32(a, b, ta=ta, tb=tb)
    assert max_rel(got32, want.numpy()) < 1e-5


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_gemm_f64_blas_path_matches_the_loop(oracle, ta, tb):
    # Large products take numpy's float64 matmul; both paths sum exact f32
    # products in f64, so they agree to f64 rounding and, rounded to f32, in
    # all but a last-place tie or two.
    M, N, K = 96, 80, 777
    a = normal((K, M) if ta else (M, K), 40)
    b = normal((N, K) if tb else (K, N), 41)
    loop = oracle.gemm_f64(a, b, ta=ta, tb=tb, path="loop")
    blas = oracle.gemm_f64(a, b, ta=ta, tb=tb, path="blas")
    assert blas.dtype == np.float64 and blas.shape == (M, N)
    scale = np.abs(a).max() * np.abs(b).max() * K
    assert np.max(np.abs(loop - blas)) <= 1e-13 * scale
    differ = np.count_nonzero(loop.astype(np.float32) != blas.astype(np.float32))
    assert differ <= 2, differ
    # a transposed operand is read through the view, not copied wrongly:
    # brute force on a few elements
    Am = a.T if ta else a
    Bm = b.T if tb else b
    for i, j in ((0, 0), (M - 1, N - 1), (17, 61)):
        s = sum(float(Am[i, k]) * float(Bm[k, j]) for k in range(K))
        assert abs(blas[i, j] - s) <= 1e-12 * scale
    # the automatic choice switches at the documented size
    assert oracle.GEMM_F64_BLAS_MIN_MACS == 1 << 22


def test_gemm_known_answer(oracle):
    ka = golden("known_answers.json")["matmul_2x2"]   # matmul/mod.rs:1145-1195
    a = np.array(ka["a"], np.float32).reshape(2, 2)
    b = np.array(ka["b"], np.float32).reshape(2, 2)
    assert oracle.gemm_f64(a, b).reshape(-1).tolist() == ka["out"]
    g = np.array(ka["grad_output"], np.float32).reshape(2, 2)
    assert oracle.gemm_f64(g, b, tb=True).reshape(-1).tolist() == ka["grad_a"]
    assert oracle.gemm_f64(a, g, ta=True).reshape(-1).tolist() == ka["grad_b"]


def test_adam_correction_factor_closed_form(oracle):
    for beta in (0.9, 0.999):
        for t in (1, 2, 10, 100, 1000):
            exact = 1.0 / (1.0 - float(np.float32(beta)) ** t)
            assert abs(float(oracle.adam_correction_factor(beta, t)) - exact) <= 4e-7 * exact


def test_adam_constant_gradient_closed_form(oracle):
    # m0 = v0 = 0, constant g: m_hat = g and v_hat = g^2 exactly in real
    # arithmetic, so every step moves p by lr * g / (|g| + eps).
    n = 37
    g = uniform(n, 0.1, 2.0, 17) * np.where(np.arange(n) % 2 == 0, 1, -1).astype(np.float32)
    p = normal(n, 18)
    p0 = p.copy()
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    for t in range(1, 21):
        oracle.adam_step(p, g, m, v, t)
        step = 1e-3 * g.astype(np.float64) / (np.abs(g.astype(np.float64)) + 1e-8)
        want = p0.astype(np.float64) - t * step
        assert np.max(np.abs(p - want)) < 2e-6, t


def test_adam_velocity_tail_association(oracle):
    # adam/mod.rs:736-773: c2*(g*g) on the 8-wide AVX2 body, (c2*g)*g on the
    # scalar tail.  Pick g where the two roundings differ and check each
    # position uses its own rule (reading of the reference; no reference
    # vector distinguishes the two, see the oracle header).
    c2 = np.float32(1.0) - np.float32(0.999)
    cand = uniform(4096, 0.5, 2.0, 19)
    body = (c2 * (cand * cand)).astype(np.float32)
    tail = ((c2 * cand) * cand).astype(np.float32)
    g_diff = cand[body != tail][0]
    g = np.full(9, g_diff, np.float32)
    p = np.zeros(9, np.float32)
    m = np.zeros(9, np.float32)
    v = np.zeros(9, np.float32)
    oracle.adam_step(p, g, m, v, 1)
    assert v[0] == np.float32(c2 * np.float32(g_diff * g_diff))
    assert v[8] == np.float32(np.float32(c2 * g_diff) * g_diff)
    assert v[0] != v[8]


def test_sum_order_model_known_answers():
    # the numpy restatement of the GPU sum's partition (the checker of the
    # one-workgroup and two-pass kernels' bits): exact where the sum is, the
    # reference's known answers, and within the f64 bound of math.fsum
    import math
    from conftest import sum_order_model
    ka = golden("known_answers.json")
    for key in ("sum_forward", "sum_21", "sum_276"):
        case = ka[key]
        assert abs(float(sum_order_model(case["x"])) - case["sum"]) <= case.get("tol", 0.0), key
    for key in ("mean_forward", "mean_3_5"):
        case = ka[key]
        assert abs(float(sum_order_model(case["x"], mean=True)) - case["mean"]) <= case["tol"], key
    for n in (1, 3, 1027, 300001):
        ints = np.arange(n, dtype=np.float32) % 97 - 48
        assert sum_order_model(ints) == np.float32(np.sum(ints.astype(np.int64)))
        assert sum_order_model(ints, aligned=False) == np.float32(np.sum(ints.astype(np.int64)))
        sq = np.sum(ints.astype(np.int64) ** 2)
        assert sum_order_model(ints, times=ints) == np.float32(sq)  # products exact in f64
    assert sum_order_model([]) == 0.0
    # past 2048 workgroups a thread takes R consecutive groups of its
    # workgroup's run (R = 4 up to 2^28 inputs; the longer runs past that are
    # pinned on the device against this model): every element counted once
    # (exact integer sums, ragged tails, unaligned) ...
    for n in ((1 << 21) + 4, (1 << 22) + 7, (1 << 24) + 12):
        ints = (np.arange(n, dtype=np.int32) % 97 - 48).astype(np.float32)
        want = np.float32(np.sum(ints, dtype=np.float64))  # exact: integers far below 2^53
        assert sum_order_model(ints) == want, n
        assert sum_order_model(ints, aligned=False) == want, n
        del ints
    # ... and added one after another in that thread: 2^60 + 1 rounds back to
    # 2^60 in f64, so 1, 2^60, -2^60, 1 in a thread's last four groups give
    # exactly 1 (a tree, (1 + 2^60) + (-2^60 + 1), gives 0) and 2^60, -2^60,
    # 1, 1 exactly 2
    big = np.float32(2.0 ** 60)
    for n, run, b, threads in (((1 << 22) + 4, 4, 3, (0, 77, 255)), ((1 << 24) + 12, 4, 4000, (129,))):
        assert -(-n // (1024 * run)) > b  # workgroup b exists
        for t in threads:
            g = 256 * run * b + t  # thread t of workgroup b: groups g, g + 256, ...
            for vals, want in (((1.0, big, -big, 1.0), 1.0), ((big, -big, 1.0, 1.0), 2.0)):
                x = np.zeros(n, np.float32)
                for j, v in enumerate(vals):
                    x[4 * (g + 256 * (run - 4 + j)) + j] = v  # any lane of a group: its quad is v
                assert sum_order_model(x) == np.float32(want), (n, t, vals)
                del x
    x = normal(1 << 21, 5)
    exact = math.fsum(x.astype(np.float64))
    assert abs(float(sum_order_model(x)) - exact) <= 1e-6 * float(np.abs(x).sum(dtype=np.float64))
