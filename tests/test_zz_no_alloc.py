"""ts_hip_gemm_noalloc: the allocation-free form of ts_hip_gemm (its split-K
temporary from a fixed device array).  Called through the C-ABI and checked
bit for bit against ts_hip_gemm -- the same kernels -- and against the f64
oracle GEMM at the matmul tolerance, on two calls in a row, the second with a
smaller problem (the array keeps the first call's slices), then an unsplit
product and an empty contraction."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import assert_bits_equal, max_rel, normal

pytestmark = pytest.mark.gpu

SCRATCH_FLOATS = 1 << 21

# (trans_a, trans_b, M, N, K): the first two split K (few output tiles and a
# K longer than the one-pass narrow kernel takes), the second's slices smaller
# than the first's; then a product the narrow kernel takes (the README step's
# forward shape: no scratch), an unsplit tiled product, two on the 16x16x4
# kernel of exact 256x256 tilings and an empty contraction
CASES = [(0, 0, 32, 128, 16384), (1, 0, 16, 64, 8448), (0, 0, 32, 128, 784), (0, 1, 300, 260, 130),
         (1, 0, 4096, 4096, 64), (0, 1, 4096, 4096, 64), (0, 0, 8, 8, 0)]


def _operands(ta, tb, M, N, K, seed):
    a = normal((K, M) if ta else (M, K), seed)
    b = normal((N, K) if tb else (K, N), seed + 1)
    return a, b


def test_noalloc_matches_gemm_on_consecutive_calls(oracle):
    from gpu_util import Dev, hip, hip_check, init, sync

    init()
    for i, (ta, tb, M, N, K) in enumerate(CASES):
        print(f"[noalloc] case {i}: ta={ta} tb={tb} M={M} N={N} K={K}", flush=True)
        need = hip.ts_hip_gemm_workspace_floats(M, N, K)
        assert need <= SCRATCH_FLOATS
        if i < 2:
            assert need > 0, "the first two cases must take the split path"
        a, b = _operands(ta, tb, M, N, K, 10 * i)
        da, db = Dev.of(a), Dev.of(b)
        lda, ldb = a.shape[1], b.shape[1]
        c_ref, c_new = Dev(M * N), Dev(M * N)
        c_ref.put(np.full(M * N, np.nan, np.float32))
        c_new.put(np.full(M * N, np.nan, np.float32))
        hip_check(hip.ts_hip_gemm(ta, tb, M, N, K, da.ptr, lda, db.ptr, ldb, c_ref.ptr, N, None), "ts_hip_gemm")
        hip_check(hip.ts_hip_gemm_noalloc(ta, tb, M, N, K, da.ptr, lda, db.ptr, ldb, c_new.ptr, N, None),
                  "ts_hip_gemm_noalloc")
        sync()
        got, want = c_new.get((M, N)), c_ref.get((M, N))
        assert_bits_equal(got, want, f"case {i}")
        if K:
            assert max_rel(got, oracle.gemm_f64(a, b, ta=bool(ta), tb=bool(tb))) <= 1e-5
        else:
            assert not got.any()


def test_noalloc_on_the_library_stream_in_a_loop(oracle):
    # repeated calls alternating the two split shapes on a non-default stream:
    # each result equals the first, so no call sees another's slices
    from gpu_util import Dev, hip, hip_check, init, sync

    init()
    st = ctypes.c_void_p()
    hip_check(hip.ts_hip_stream_create(ctypes.byref(st)), "stream")
    try:
        shapes = CASES[:2]
        ops = [_operands(*s[:2], *s[2:], 5 + j) for j, s in enumerate(shapes)]
        devs = [(Dev.of(a), Dev.of(b)) for a, b in ops]
        outs = [[Dev(s[2] * s[3]) for _ in range(3)] for s in shapes]
        for r in range(3):
            for j, (ta, tb, M, N, K) in enumerate(shapes):
                da, db = devs[j]
                hip_check(hip.ts_hip_gemm_noalloc(ta, tb, M, N, K, da.ptr, ops[j][0].shape[1], db.ptr,
                                                  ops[j][1].shape[1], outs[j][r].ptr, N, st), "noalloc")
        hip_check(hip.ts_hip_stream_synchronize(st), "sync")
        sync()
        for j, (ta, tb, M, N, K) in enumerate(shapes):
            first = outs[j][0].get((M, N))
            for r in (1, 2):
                assert_bits_equal(outs[j][r].get((M, N)), first, f"shape {j} repeat {r}")
            assert max_rel(first, oracle.gemm_f64(*ops[j], ta=bool(ta), tb=bool(tb))) <= 1e-5
    finally:
        hip.ts_hip_stream_destroy(st)
