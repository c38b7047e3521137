"""ts_hip_gemm_colsum: a weight gradient C = op(A) . B with the bias gradient
colsum[n] = sum_k B[k][n] beside it.  Every kernel path is covered (the
256x256 LDS-DMA tiles, the register-staged 64/128/256 tiles with aligned and
unaligned operands, the narrow one-pass kernel and the sliced skinny kernel
for N <= 16, an MFMA split-K product, trans_a == 0, ragged K); on each, C has the bits of ts_hip_gemm
and colsum the bits of ts_hip_sum_dim0, both restated by the oracle (the
column sum's fixed chunk order, oracle.sum_dim0_chunked, bit for bit; the
product within the matmul tolerance of the f64 product)."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_bits_equal, max_rel, normal

pytestmark = pytest.mark.gpu

# (trans_a, M, N, K, B row pitch, B offset in floats): the path each takes
CASES = [
    (1, 4096, 4096, 8192, 4096, 0),   # 256x256 LDS-DMA tiles (config 5's dW)
    (1, 4096, 4096, 1000, 4096, 0),   # LDS-DMA, 31 two-sub-tile stages and a partial last sub-tile
    (1, 784, 1024, 1024, 1024, 0),    # 64x64 register tiles (config 4's dW1)
    (1, 2048, 2048, 1000, 2048, 0),   # 128x128 tiles, K not a multiple of 16 or 64
    (1, 4096, 4096, 520, 4097, 1),    # unaligned B: 256x256 register tiles, element loads
    (1, 700, 300, 77, 300, 0),        # 64x64 tiles, a partial last k tile
    (1, 1024, 10, 1024, 10, 0),       # narrow (N <= 16, config 4's dW2): workgroup 0 adds the chunks
    (1, 20000, 7, 300, 7, 0),         # narrow, many row blocks, ragged wave ranges
    (1, 512, 12, 5000, 12, 0),        # narrow, 79 chunks: a partial last chunk and a partial last group
    (1, 64, 10, 16384, 10, 0),        # sliced skinny kernel (long K, few rows): the slice sum's extra workgroup
    (1, 16400, 3, 8256, 3, 0),        # narrow, K past its chunk table: the product, then a column-sum pass
    (1, 32, 128, 784, 128, 0),        # narrow kernel, 8 column blocks (the README step's dW shape, transposed)
    (1, 32, 128, 16384, 128, 0),      # MFMA split-K: the column sum runs as its own pass
    (0, 512, 256, 640, 256, 0),       # trans_a == 0 through the narrow kernel
    (0, 2048, 2048, 100, 2048, 0),    # trans_a == 0 on 128x128 tiles: product, then the column sum pass
    (1, 64, 64, 5, 64, 0),            # K shorter than one tile
    (1, 0, 33, 130, 33, 0),           # no product: the column sums alone
    (1, 50, 40, 0, 40, 0),            # empty contraction: C = 0, colsum = 0
]


@pytest.mark.parametrize("ta,M,N,K,ldb,off", CASES)
def test_gemm_colsum_bits(oracle, ta, M, N, K, ldb, off):
    from gpu_util import Dev, hip, hip_check, init, sync

    init()
    print(f"[colsum] ta={ta} M={M} N={N} K={K} ldb={ldb} off={off}", flush=True)
    a = normal((K, M) if ta else (M, K), 3)
    bfull = normal((K, ldb), 4)
    b = bfull[:, :N]
    da, db = Dev.of(a), Dev.of(bfull, offset=off)
    lda = a.shape[1] if a.size else max(M, 1)
    c_ref, c_new = Dev(max(M * N, 1)), Dev(max(M * N, 1))
    cs_new, cs_ref = Dev(N), Dev(N)
    ws = hip.ts_hip_gemm_colsum_workspace_floats(ta, M, N, K)
    dws = Dev(max(ws, 2))
    hip_check(hip.ts_hip_gemm_colsum(ta, M, N, K, da.ptr, lda, db.ptr, ldb, c_new.ptr, N, cs_new.ptr,
                                     dws.ptr if ws else None, ws, None), "ts_hip_gemm_colsum")
    if M:
        hip_check(hip.ts_hip_gemm(ta, 0, M, N, K, da.ptr, lda, db.ptr, ldb, c_ref.ptr, N, None), "ts_hip_gemm")
    if ldb == N and off == 0:
        ws0 = hip.ts_hip_sum_dim0_workspace_floats(K, N)
        dws0 = Dev(max(ws0, 2))
        hip_check(hip.ts_hip_sum_dim0(db.ptr, K, N, cs_ref.ptr, dws0.ptr, ws0, None), "ts_hip_sum_dim0")
    sync()
    got = cs_new.get()
    assert_bits_equal(got, oracle.sum_dim0_chunked(b) if K else np.zeros(N, np.float32), "colsum vs oracle")
    if ldb == N and off == 0:
        assert_bits_equal(got, cs_ref.get(), "colsum vs ts_hip_sum_dim0")
    if M:
        cg = c_new.get((M, N))
        assert_bits_equal(cg, c_ref.get((M, N)), "product vs ts_hip_gemm")
        if K and M * N * K <= (1 << 34):
            assert max_rel(cg, oracle.gemm_f64(a, b, ta=bool(ta), tb=False)) <= 1e-5


def test_gemm_colsum_allocates_its_workspace_when_none_is_given(oracle):
    """workspace == NULL: the split temporary and chunk sums come from the
    stream-ordered allocator, with the same bits."""
    from gpu_util import Dev, hip, hip_check, init, sync

    init()
    for ta, M, N, K in ((1, 1024, 10, 1024), (1, 32, 128, 784), (0, 300, 200, 100)):
        a, b = normal((K, M) if ta else (M, K), 5), normal((K, N), 6)
        da, db, c, cs = Dev.of(a), Dev.of(b), Dev(M * N), Dev(N)
        hip_check(hip.ts_hip_gemm_colsum(ta, M, N, K, da.ptr, a.shape[1], db.ptr, N, c.ptr, N, cs.ptr, None, 0,
                                         None), "ts_hip_gemm_colsum")
        sync()
        assert_bits_equal(cs.get(), oracle.sum_dim0_chunked(b), f"ta={ta} {M}x{N}x{K}")


def test_gemm_colsum_refuses_bad_arguments():
    from gpu_util import Dev, hip, init

    init()
    a, b, c = Dev(64 * 64), Dev(64 * 64), Dev(64 * 64)
    cs = Dev(64)
    K = 16384  # a split-K product: it needs a workspace
    ws = hip.ts_hip_gemm_colsum_workspace_floats(1, 32, 128, K)
    assert ws > 0
    small = Dev(ws)
    # no column-sum output; a workspace that is too small
    assert hip.ts_hip_gemm_colsum(1, 64, 64, 64, a.ptr, 64, b.ptr, 64, c.ptr, 64, None, None, 0, None) != 0
    aa, bb, cc, cc2 = Dev(K * 32), Dev(K * 128), Dev(32 * 128), Dev(128)
    assert hip.ts_hip_gemm_colsum(1, 32, 128, K, aa.ptr, 32, bb.ptr, 128, cc.ptr, 128, cc2.ptr, small.ptr,
                                  ws - 1, None) == 100003


def test_column_sum_order_on_special_values(oracle):
    """Cases whose bits depend on the order: a 1 that survives only because
    groups of 8 chunks are summed from +0 (chunk by chunk it would be lost
    next to 2^60), columns of -0 (give +0), and a column whose first chunk
    keeps 63 terms of 2^-30 that a flat fp32 sum would drop.  Through the
    standalone column sum and the fused dW product alike."""
    from gpu_util import Dev, hip, hip_check, init, sync

    init()
    rows, cols = 10 * 64, 64
    x = np.zeros((rows, cols), np.float32)
    x[0, 0] = 1.0
    x[64 * 8, 0] = 2.0 ** 60
    x[64 * 9, 0] = -(2.0 ** 60)
    x[:, 1] = -0.0
    x[0, 2] = 1.0
    x[1:64, 2] = 2.0 ** -30
    x[64, 2] = -1.0
    x[:, 3:] = normal((rows, cols - 3), 21)
    want = oracle.sum_dim0_chunked(x)
    assert want[0] == 1.0 and want[2] == np.float32(63 * 2.0 ** -30)
    dx, out = Dev.of(x), Dev(cols)
    ws = hip.ts_hip_sum_dim0_workspace_floats(rows, cols)
    dws = Dev(ws)
    hip_check(hip.ts_hip_sum_dim0(dx.ptr, rows, cols, out.ptr, dws.ptr, ws, None), "ts_hip_sum_dim0")
    sync()
    assert_bits_equal(out.get(), want, "ts_hip_sum_dim0")
    # 64 output rows: a split-K product, then the column-sum pass; 4096: 64x64
    # tiles with the chunks spread over 64 tile rows; 4 columns: the narrow
    # kernel's workgroup 0
    for M, N in ((64, cols), (4096, cols), (4096, 4)):
        a = normal((rows, M), 22)
        xs = np.ascontiguousarray(x[:, :N])
        dxs, c, cs = Dev.of(xs), Dev(M * N), Dev(N)
        ws = hip.ts_hip_gemm_colsum_workspace_floats(1, M, N, rows)
        dws = Dev(max(ws, 2))
        hip_check(hip.ts_hip_gemm_colsum(1, M, N, rows, da_ptr(Dev, a), M, dxs.ptr, N, c.ptr, N, cs.ptr, dws.ptr, ws,
                                         None), "ts_hip_gemm_colsum")
        sync()
        assert_bits_equal(cs.get(), want[:N], f"ts_hip_gemm_colsum M={M} N={N}")


_keep = []


def da_ptr(Dev, a):
    d = Dev.of(a)
    _keep.append(d)  # alive until the test module ends
    return d.ptr


# tall inputs: past 16 groups of 8 chunks the group sums run as a pass of
# their own, then one dependent add per group (the order is unchanged)
@pytest.mark.parametrize("rows,cols", [(8192, 7), (8193, 3), (9 * 8192 + 5, 5), ((1 << 17) + 37, 16),
                                       (40000, 259)])
def test_tall_column_sums(oracle, rows, cols):
    from gpu_util import Dev, hip, hip_check, init, sync

    init()
    print(f"[colsum tall] {rows}x{cols}", flush=True)
    x = normal((rows, cols), 31)
    # large terms that cancel across groups, and a small one they would
    # swallow if a group's sum were formed in another order
    x[64 * 8 * 3, 0] = 2.0 ** 50
    x[64 * 8 * 7, 0] = -(2.0 ** 50)
    x[64 * 8 * 5 + 1, 0] = 1.5
    want = oracle.sum_dim0_chunked(x)
    dx, out = Dev.of(x), Dev(cols)
    ws = hip.ts_hip_sum_dim0_workspace_floats(rows, cols)
    assert ws == 2 * ((rows + 63) // 64) * cols
    dws = Dev(ws)
    hip_check(hip.ts_hip_sum_dim0(dx.ptr, rows, cols, out.ptr, dws.ptr, ws, None), "ts_hip_sum_dim0")
    sync()
    assert_bits_equal(out.get(), want, f"tall column sums {rows}x{cols}")
