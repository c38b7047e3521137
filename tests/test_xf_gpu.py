"""Operand transforms (ts_hip_gemm_fused_xf, ts_hip_gemm_colsum_xf): an
elementwise chain applied to an operand as the product loads it gives the
bits of the same product on an operand that holds the transformed values
(computed here in numpy float32, whose single IEEE operations are the
device's), for every kernel that takes transforms: register-staged tiles
(aligned and not, a partial k tile, both layouts of each operand), the
narrow kernel with its column sums, the one-k-tile kernel with a mask
epilogue, and the column strips; the product kinds that take none refuse
them."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import assert_bits_equal, normal

pytestmark = pytest.mark.gpu


def _ffi():
    from train_station_amd import _ffi as F
    return F


def _xf(ops):
    F = _ffi()
    x = F.OperandXf()
    x.n_ops = len(ops)
    for i, (code, imm) in enumerate(ops):
        x.code[i] = F.XF_CODES[code]
        x.imm[i] = imm
    return x


def _apply(v, ops):
    v = v.astype(np.float32).copy()
    for code, imm in ops:
        c = np.float32(imm)
        if code == "add_s": v = v + c
        elif code == "sub_s": v = v - c
        elif code == "mul_s": v = v * c
        elif code == "div_s": v = v / c
        elif code == "rsub_s": v = c - v
        elif code == "rdiv_s": v = c / v
        elif code == "relu": v = np.where(v > 0, v, np.float32(0))
        elif code == "relu_bwd_s": v = np.where(v > 0, c, np.float32(0))
        elif code == "square": v = v * v
        v = v.astype(np.float32)
    return v


MSE = [("mul_s", 2.0), ("mul_s", 1.0 / 10240)]    # the MSE gradient of config 4: (d * 2) * (1/n)
RELU_SEED = [("relu_bwd_s", 1.0)]                  # relu's backward of the seed (config 1)
OTHER = [("relu", 0.0), ("div_s", 3.0), ("rsub_s", 0.0), ("square", 0.0)]

# (ta, tb, M, N, K, which operand, chain, colsum, mask, offset)
CASES = [
    (1, 0, 784, 128, 32, "b", RELU_SEED, True, False, 0),    # config 1's dW + db: 64x64 tiles and strips
    (1, 0, 784, 128, 40, "b", MSE, True, False, 0),          # a partial last k tile
    (1, 0, 700, 300, 77, "b", OTHER, True, False, 1),        # unaligned: element loads
    (1, 0, 1024, 10, 1024, "b", MSE, True, False, 0),        # config 4's dW2 + db2: narrow kernel
    (1, 0, 512, 12, 1000, "b", RELU_SEED, True, False, 0),   # narrow, a partial last chunk
    (0, 1, 1024, 1024, 10, "a", MSE, False, True, 0),        # config 4's dX2: one k tile, mask epilogue
    (0, 0, 300, 260, 130, "a", OTHER, False, False, 0),      # register tiles, A k-contiguous
    (1, 1, 300, 260, 130, "a", MSE, False, False, 0),        # A transposed
    (0, 1, 300, 260, 130, "b", RELU_SEED, False, False, 0),  # B transposed
    (0, 0, 300, 260, 130, "b", OTHER, False, False, 0),      # B k-major
    (0, 0, 64, 128, 784, "b", MSE, False, False, 0),         # narrow kernel, B k-major
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}{c[1]}-{c[2]}x{c[3]}x{c[4]}-{c[5]}" for c in CASES])
def test_transformed_operand_has_the_bits_of_a_transformed_buffer(case):
    from gpu_util import Dev, hip, hip_check, sync
    ta, tb, M, N, K, side, ops, colsum, mask, off = case
    print(f"[xf] {case}", flush=True)
    assert hip.ts_hip_gemm_takes_xf(ta, tb, M, N, K, int(colsum)) == 1
    a = normal((K, M) if ta else (M, K), 41)
    b = normal((N, K) if tb else (K, N), 42)
    a[0, :3] = 0.0  # zeros through the chain
    lda, ldb = a.shape[1], b.shape[1]
    ax, bx = (_apply(a, ops), b) if side == "a" else (a, _apply(b, ops))
    da, db = Dev.of(a, off), Dev.of(b, off)
    dax, dbx = Dev.of(ax, off), Dev.of(bx, off)
    x = _xf(ops)
    xa, xb = (ctypes.byref(x), None) if side == "a" else (None, ctypes.byref(x))
    got, want = Dev(M * N), Dev(M * N)
    if colsum:
        cs_got, cs_want = Dev(N), Dev(N)
        ws = hip.ts_hip_gemm_colsum_workspace_floats(ta, M, N, K)
        dws = Dev(ws + 2)
        hip_check(hip.ts_hip_gemm_colsum_xf(ta, M, N, K, da.ptr, lda, xa, db.ptr, ldb, xb, got.ptr, N,
                                            cs_got.ptr, dws.ptr, ws, None), "colsum_xf")
        hip_check(hip.ts_hip_gemm_colsum(ta, M, N, K, dax.ptr, lda, dbx.ptr, ldb, want.ptr, N, cs_want.ptr,
                                         dws.ptr, ws, None), "colsum")
        sync()
        assert_bits_equal(cs_got.get(), cs_want.get(), "column sums")
    else:
        mk = Dev.of(normal((M, N), 43)) if mask else None
        ws = hip.ts_hip_gemm_workspace_floats(M, N, K)
        dws = Dev(ws + 2)
        hip_check(hip.ts_hip_gemm_fused_xf(ta, tb, M, N, K, da.ptr, lda, xa, db.ptr, ldb, xb, None, 0,
                                           mk.ptr if mk else None, got.ptr, N, dws.ptr, ws, None), "fused_xf")
        hip_check(hip.ts_hip_gemm_fused(ta, tb, M, N, K, dax.ptr, lda, dbx.ptr, ldb, None, 0,
                                        mk.ptr if mk else None, want.ptr, N, dws.ptr, ws, None), "fused")
    sync()
    assert_bits_equal(got.get(), want.get(), "product")


def test_refused_transforms_and_shapes():
    from gpu_util import Dev, hip
    M, N, K = 300, 260, 130
    a, b, c = Dev(M * K), Dev(K * N), Dev(M * N)
    for ops in ([("sub_s", 0.5)], [("div_s", -3.0)], [("rdiv_s", 1.0)], [("add_s", 1.0)]):  # +0 not kept
        x = _xf(ops)
        assert hip.ts_hip_gemm_fused_xf(0, 0, M, N, K, a.ptr, K, None, b.ptr, N, ctypes.byref(x), None, 0, None,
                                        c.ptr, N, None, 0, None) == 100001, ops
    x = _xf([("mul_s", 2.0)] * 4)
    x.n_ops = 5                                   # past TS_HIP_XF_MAX_OPS
    assert hip.ts_hip_gemm_fused_xf(0, 0, M, N, K, a.ptr, K, ctypes.byref(x), b.ptr, N, None, None, 0, None,
                                    c.ptr, N, None, 0, None) == 100001
    x = _xf([("mul_s", 2.0)])
    x.code[0] = 9                                 # no such op
    assert hip.ts_hip_gemm_fused_xf(0, 0, M, N, K, a.ptr, K, ctypes.byref(x), b.ptr, N, None, None, 0, None,
                                    c.ptr, N, None, 0, None) == 100001
    # products whose kernels take no transform: the LDS-DMA tiles, a split K
    for ta, tb, m, n, k, cs in ((0, 0, 8192, 4096, 4096, 0), (1, 0, 4096, 4096, 8192, 1), (0, 0, 32, 128, 16384, 0)):
        assert hip.ts_hip_gemm_takes_xf(ta, tb, m, n, k, cs) == 0, (m, n, k)
    big = 4096 * 4096
    da, db, dc = Dev(big), Dev(big), Dev(big)
    x = _xf([("mul_s", 2.0)])
    assert hip.ts_hip_gemm_fused_xf(0, 0, 4096, 4096, 4096, da.ptr, 4096, None, db.ptr, 4096, ctypes.byref(x),
                                    None, 0, None, dc.ptr, 4096, None, 0, None) == 100001
