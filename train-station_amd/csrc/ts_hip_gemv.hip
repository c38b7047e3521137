// Vector cases of matmul (tensor/ops/matmul/mod.rs:263-632) and their
// backward (grad_fn/ops/matmul.rs:17-60): matrix-vector and vector-matrix
// products and the outer product.  All are HBM-bound (one read of the
// matrix), so they run as bandwidth kernels rather than on the MFMA tiles.
//
//   gemv, trans 0: y[r] = sum_c A[r][c] x[c]   one wave per row, lanes stride
//                  the row (dwordx4), f64 partials, a shuffle tree
//   gemv, trans 1: y[c] = sum_r x[r] A[r][c]   the weighted column sum of the
//                  bias-gradient reduction (f64 partials over row chunks)
//   outer:         out[i][j] = a[i] * b[j]     (compute_outer_product, fp32)
#include "ts_hip_internal.h"

namespace tship {

constexpr int kRowsPerBlock = kBlock / 64;

__global__ __launch_bounds__(kBlock) void gemv_rows(const float *__restrict__ A, size_t rows, size_t cols,
                                                    size_t lda, const float *__restrict__ x,
                                                    float *__restrict__ y, int vec) {
    const size_t r = static_cast<size_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    double acc = 0.0;
    if (r < rows) {
        const float *row = A + r * lda;
        size_t c = 0;
        if (vec) {
            const float4 *a4 = reinterpret_cast<const float4 *>(row);
            const float4 *x4 = reinterpret_cast<const float4 *>(x);
            const size_t c4 = cols / 4;
            for (size_t v = lane; v < c4; v += 64) {
                const float4 p = a4[v], q = x4[v];
                acc += (double)p.x * q.x + (double)p.y * q.y + (double)p.z * q.z + (double)p.w * q.w;
            }
            c = 4 * c4;
        }
        for (size_t i = c + lane; i < cols; i += 64) acc += (double)row[i] * x[i];
    }
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) acc += __shfl_xor(acc, d, 64);
    if (lane == 0 && r < rows) y[r] = static_cast<float>(acc);
}

__global__ __launch_bounds__(kBlock) void outer_product(const float *__restrict__ a, size_t m,
                                                        const float *__restrict__ b, size_t n,
                                                        float *__restrict__ out) {
    const size_t total = m * n;
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; i < total; i += stride)
        out[i] = a[i / n] * b[i % n];
}

}  // namespace tship

using namespace tship;

extern "C" {

size_t ts_hip_gemv_workspace_floats(int trans, size_t rows, size_t cols) {
    return trans ? ts_hip_sum_dim0_workspace_floats(rows, cols) : 0;
}

int ts_hip_gemv(int trans, size_t rows, size_t cols, const float *A, size_t lda, const float *x, float *y,
                float *workspace, size_t workspace_floats, void *stream) {
    if (trans) return launch_colsum(A, x, rows, cols, lda, y, workspace, workspace_floats, stream);
    if (rows == 0) return TS_HIP_OK;
    if (!y) return TS_HIP_EINVAL;
    if (cols == 0) return ts_hip_fill(y, 0.0f, rows, stream);
    if (!A || !x || lda < cols) return TS_HIP_EINVAL;
    const int vec = aligned16(A) && aligned16(x) && lda % 4 == 0;
    const size_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
    if (blocks > 0x7fffffffULL) return TS_HIP_EINVAL;
    launch(gemv_rows, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, as_stream(stream), A,
                       rows, cols, lda, x, y, vec);
    return launch_status();
}

int ts_hip_outer(const float *a, size_t m, const float *b, size_t n, float *out, void *stream) {
    if (m == 0 || n == 0) return TS_HIP_OK;
    if (!a || !b || !out) return TS_HIP_EINVAL;
    launch(outer_product, dim3(grid_for(m * n)), dim3(kBlock), 0, as_stream(stream), a, m, b, n, out);
    return launch_status();
}

}  // extern "C"
