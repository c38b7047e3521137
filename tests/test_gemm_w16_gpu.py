"""The 16x16x4 kernel (gemm_f32_w16: M and N multiples of 256, K of 32, at
least one 256x256 tile per CU; the NN, NT and TN layouts, TT keeping the 32x32
kernel): its corners against the f64 product, the column sums' fixed order and
the separate epilogue kernels."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_bits_equal, max_rel, normal

pytestmark = pytest.mark.gpu

# (trans_a, trans_b, M, N, K, operand pitch pad, output pitch pad, C offset in floats)
CASES = [
    (0, 0, 4096, 4096, 32, 0, 0, 0),     # one stage
    (0, 0, 4096, 4096, 96, 0, 0, 0),     # an odd stage count
    (1, 0, 4096, 4096, 32, 0, 0, 0),
    (1, 0, 4096, 4096, 160, 0, 0, 0),
    (0, 1, 4096, 4096, 32, 0, 0, 0),
    (0, 1, 4096, 4096, 96, 0, 0, 0),
    (0, 0, 4096, 4096, 64, 4, 8, 0),     # operand and output pitches past the matrix
    (1, 0, 4096, 4096, 64, 12, 4, 0),
    (0, 1, 4096, 4096, 64, 8, 4, 0),
    (0, 0, 4096, 4096, 64, 0, 0, 1),     # C not 16-byte aligned: element stores
    (1, 0, 4096, 4096, 64, 0, 0, 1),
    (0, 1, 4096, 4096, 64, 0, 0, 1),
    (0, 0, 256, 65536, 64, 0, 0, 0),     # one tile row
    (0, 0, 65536, 256, 64, 0, 0, 0),     # one tile column
    (0, 1, 256, 65536, 64, 0, 0, 0),
    (0, 1, 65536, 256, 64, 0, 0, 0),
]


@pytest.mark.parametrize("ta,tb,M,N,K,pad,cpad,coff", CASES)
def test_w16_products(oracle, ta, tb, M, N, K, pad, cpad, coff):
    from gpu_util import Dev, hip, hip_check, sync

    print(f"[w16] ta={ta} tb={tb} M={M} N={N} K={K} pad={pad} cpad={cpad} coff={coff}", flush=True)
    a = normal((K, M) if ta else (M, K), 21)
    b = normal((N, K) if tb else (K, N), 22)

    def padded(x):  # the matrix in a buffer whose row pitch is `pad` floats longer
        out = np.zeros((x.shape[0], x.shape[1] + pad), np.float32)
        out[:, : x.shape[1]] = x
        return out

    lda, ldb = a.shape[1] + pad, b.shape[1] + pad
    ldc = N + cpad
    c0 = np.full((M, ldc), np.nan, np.float32)
    da, db, dc = Dev.of(padded(a)), Dev.of(padded(b)), Dev.of(c0, offset=coff)
    hip_check(hip.ts_hip_gemm(ta, tb, M, N, K, da.ptr, lda, db.ptr, ldb, dc.ptr, ldc, None), "ts_hip_gemm")
    sync()
    out = dc.get((M, ldc))
    got = out[:, :N]
    want = oracle.gemm_f64(a, b, ta=bool(ta), tb=bool(tb))
    assert max_rel(got, want) <= 1e-4
    tol = 1e-4 * np.maximum(np.abs(want), np.sqrt(np.mean(want * want)))
    assert np.all(np.abs(got.astype(np.float64) - want) <= tol)
    if cpad:
        assert np.all(np.isnan(out[:, N:])), "the output pitch's padding was written"


@pytest.mark.parametrize("K", [32, 96, 160])
def test_w16_column_sums(oracle, K):
    # the dW product with its bias gradient: chunks of 64 k rows across the
    # stages of 32, a last chunk of one stage when the stage count is odd
    from gpu_util import Dev, hip, hip_check, sync

    M = N = 4096
    print(f"[w16 colsum] K={K}", flush=True)
    a, b = normal((K, M), 23), normal((K, N), 24)
    da, db = Dev.of(a), Dev.of(b)
    c_new, c_ref, cs = Dev(M * N), Dev(M * N), Dev(N)
    ws = hip.ts_hip_gemm_colsum_workspace_floats(1, M, N, K)
    dws = Dev(max(ws, 2))
    hip_check(hip.ts_hip_gemm_colsum(1, M, N, K, da.ptr, M, db.ptr, N, c_new.ptr, N, cs.ptr, dws.ptr, ws, None),
              "ts_hip_gemm_colsum")
    hip_check(hip.ts_hip_gemm(1, 0, M, N, K, da.ptr, M, db.ptr, N, c_ref.ptr, N, None), "ts_hip_gemm")
    sync()
    assert_bits_equal(cs.get(), oracle.sum_dim0_chunked(b), "column sums vs the oracle's order")
    assert_bits_equal(c_new.get(), c_ref.get(), "product with and without the column sums")


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
@pytest.mark.parametrize("bias,relu,mask", [(1, 1, 1), (1, 0, 0), (0, 1, 0), (0, 0, 1), (1, 1, 0)])
def test_w16_epilogues(ta, tb, bias, relu, mask):
    # bias, relu and the relu-backward mask in the kernel's stores, every
    # combination on every layout it takes: the separate kernels' bits
    from gpu_util import Dev, hip, hip_check, sync

    M = N = 4096
    K = 64
    print(f"[w16 epilogue] ta={ta} tb={tb} bias={bias} relu={relu} mask={mask}", flush=True)
    a = normal((K, M) if ta else (M, K), 25)
    b = normal((N, K) if tb else (K, N), 26)
    vb, vm = normal(N, 27), normal((M, N), 28)
    da, db, dbias, dmask = Dev.of(a), Dev.of(b), Dev.of(vb), Dev.of(vm)
    lda, ldb = a.shape[1], b.shape[1]
    fused, ref = Dev(M * N), Dev(M * N)
    ws = hip.ts_hip_gemm_workspace_floats(M, N, K)
    dws = Dev(max(ws, 1))
    hip_check(hip.ts_hip_gemm_fused(ta, tb, M, N, K, da.ptr, lda, db.ptr, ldb, dbias.ptr if bias else None, relu,
                                    dmask.ptr if mask else None, fused.ptr, N, dws.ptr if ws else None, ws, None),
              "ts_hip_gemm_fused")
    hip_check(hip.ts_hip_gemm(ta, tb, M, N, K, da.ptr, lda, db.ptr, ldb, ref.ptr, N, None), "ts_hip_gemm")
    if bias:
        hip_check(hip.ts_hip_bias_add(ref.ptr, dbias.ptr, ref.ptr, M, N, 0, None), "bias")
    if relu:
        hip_check(hip.ts_hip_relu(ref.ptr, ref.ptr, M * N, None), "relu")
    if mask:
        hip_check(hip.ts_hip_relu_backward(dmask.ptr, ref.ptr, ref.ptr, M * N, None), "mask")
    sync()
    assert_bits_equal(fused.get(), ref.get(), f"ta={ta} tb={tb} bias={bias} relu={relu} mask={mask}")
