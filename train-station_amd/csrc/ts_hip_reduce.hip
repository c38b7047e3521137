// Reductions of the gradtrack step: the scalar loss (sum / mean) and the
// bias-gradient column reduction sum_dims(&[0]).  Both are deterministic
// two-pass trees: per-thread f64 accumulation over a fixed slice, a wave64
// shuffle reduction, an LDS combine across the workgroup's four waves, one
// f64 partial per workgroup, then a single-workgroup pass in fixed order.
// No floating-point atomics, so every run gives the same bits.
#include "ts_hip_internal.h"

namespace tship {

// Pass 1: workgroup b sums the float4 groups b, b+G, b+2G, ... (all threads
// of the grid stride together) and writes one f64 partial.  PROD: the terms
// are x[i] * y[i] formed in f64 (a dot product).
template <bool PROD>
__global__ __launch_bounds__(kBlock) void sum_partial(const float *__restrict__ x, const float *__restrict__ y,
                                                      size_t n, size_t n4, double *__restrict__ partial) {
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    const size_t t = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
    double acc = 0.0;
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    const float4 *y4 = reinterpret_cast<const float4 *>(y);
    for (size_t v = t; v < n4; v += stride) {
        const float4 q = x4[v];
        if (PROD) {
            const float4 r = y4[v];
            acc += (double)q.x * (double)r.x + (double)q.y * (double)r.y + (double)q.z * (double)r.z +
                   (double)q.w * (double)r.w;
        } else {
            acc += (double)q.x + (double)q.y + (double)q.z + (double)q.w;
        }
    }
    for (size_t i = 4 * n4 + t; i < n; i += stride) acc += PROD ? (double)x[i] * (double)y[i] : (double)x[i];
    double r = block_sum(acc);
    if (threadIdx.x == 0) partial[blockIdx.x] = r;
}

// Pass 2: one workgroup adds the partials in a fixed order.  MEAN divides the
// fp32 sum by (float)n, as reductions/mean.rs:104 does.
template <bool MEAN>
__global__ __launch_bounds__(kBlock) void sum_final(const double *__restrict__ partial,
                                                    size_t nparts, size_t n, float *out) {
    double acc = 0.0;
    size_t i = threadIdx.x;
    for (; i + kBlock * 7 < nparts; i += kBlock * 8) {  // eight loads in flight
        double v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = partial[i + kBlock * j];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc += v[j];
    }
    for (; i < nparts; i += kBlock) acc += partial[i];
    double r = block_sum(acc);
    if (threadIdx.x == 0) {
        float s = static_cast<float>(r);
        out[0] = MEAN ? s / static_cast<float>(n) : s;
    }
}

int launch_sum_final(const double *partial, size_t nparts, size_t n, float *out, bool mean, hipStream_t s) {
    if (mean) launch(sum_final<true>, dim3(1), dim3(kBlock), 0, s, partial, nparts, n, out);
    else launch(sum_final<false>, dim3(1), dim3(kBlock), 0, s, partial, nparts, n, out);
    return launch_status();
}

template <bool MEAN>
static int launch_sum(const float *x, const float *y, size_t n, float *out, float *workspace, size_t ws,
                      void *stream) {
    if (!out) return TS_HIP_EINVAL;
    hipStream_t s = as_stream(stream);
    if (n == 0) {  // sum.rs:82-83 / mean.rs:51-53: empty input gives 0
        return ts_hip_fill(out, 0.0f, 1, stream);
    }
    if (!x) return TS_HIP_EINVAL;
    const size_t blocks = sum_blocks(n);
    if (!workspace || ws < 2 * blocks) return TS_HIP_EWORKSPACE;
    if ((reinterpret_cast<uintptr_t>(workspace) & 7u) != 0) return TS_HIP_EINVAL;
    double *partial = reinterpret_cast<double *>(workspace);
    size_t n4 = (aligned16(x) && (!y || aligned16(y))) ? n / 4 : 0;
    if (y)
        launch(sum_partial<true>, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, x, y, n,
                           n4, partial);
    else
        launch(sum_partial<false>, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, x, y, n,
                           n4, partial);
    int st = launch_status();
    if (st) return st;
    return launch_sum_final(partial, blocks, n, out, MEAN, s);
}

// ---- column reduction [rows, cols] -> [cols] --------------------------------

// Pass 1: a workgroup owns 64 column units (float4 groups of 4 adjacent
// columns when cols % 4 == 0, single columns otherwise) and one chunk of
// rows; its four waves take every fourth row of the chunk, each wave reading
// 1 KiB contiguously per row with eight rows in flight per thread.  The four
// row lanes are combined in LDS in a fixed order and one f64 partial per
// column and chunk is written.  Chunks are sized so that the grid has about
// 2048 workgroups.
constexpr size_t kDim0MaxChunks = 128;
constexpr int kDim0Cols = 64;  // column units per workgroup
constexpr int kDim0Unroll = 8;

static size_t dim0_chunks(size_t rows, size_t cols) {
    const size_t units = (cols % 4 == 0) ? cols / 4 : cols;
    const size_t col_blocks = (units + kDim0Cols - 1) / kDim0Cols;
    size_t want = 2048 / (col_blocks ? col_blocks : 1);
    size_t by_rows = (rows + 15) / 16;                    // at least 16 rows per chunk
    size_t c = want < by_rows ? want : by_rows;
    if (c > kDim0MaxChunks) c = kDim0MaxChunks;
    return c < 1 ? 1 : c;
}

// W: row r is weighted by w[r] (in f64) -- a transposed matrix-vector product.
template <bool VEC, bool W>
__global__ __launch_bounds__(kBlock) void dim0_partial(const float *__restrict__ x, const float *__restrict__ w,
                                                       size_t rows, size_t cols, size_t rows_per_chunk,
                                                       double *__restrict__ partial) {
    constexpr int L = VEC ? 4 : 1;  // columns per unit
    __shared__ double lds[kBlock / kDim0Cols][kDim0Cols][L];
    const size_t units = VEC ? cols / 4 : cols;
    const int cl = threadIdx.x % kDim0Cols, rl = threadIdx.x / kDim0Cols;
    constexpr int RL = kBlock / kDim0Cols;  // row lanes
    const size_t u = static_cast<size_t>(blockIdx.x) * kDim0Cols + cl;
    const size_t r0 = static_cast<size_t>(blockIdx.y) * rows_per_chunk;
    size_t r1 = r0 + rows_per_chunk;
    if (r1 > rows) r1 = rows;
    double acc[L];
#pragma unroll
    for (int c = 0; c < L; ++c) acc[c] = 0.0;
    auto load = [&](size_t r, float (&q)[L]) {
        if (VEC) {
            const float4 v = reinterpret_cast<const float4 *>(x)[r * units + u];
            q[0] = v.x; q[L > 1 ? 1 : 0] = v.y; q[L > 2 ? 2 : 0] = v.z; q[L > 3 ? 3 : 0] = v.w;
        } else {
            q[0] = x[r * cols + u];
        }
    };
    if (u < units) {
        size_t r = r0 + rl;
        for (; r + RL * (kDim0Unroll - 1) < r1; r += RL * kDim0Unroll) {
            float q[kDim0Unroll][L];
#pragma unroll
            for (int k = 0; k < kDim0Unroll; ++k) load(r + RL * k, q[k]);
#pragma unroll
            for (int k = 0; k < kDim0Unroll; ++k) {
                const double wr = W ? (double)w[r + RL * k] : 1.0;
#pragma unroll
                for (int c = 0; c < L; ++c) acc[c] += wr * q[k][c];
            }
        }
        for (; r < r1; r += RL) {
            float q[L];
            load(r, q);
            const double wr = W ? (double)w[r] : 1.0;
#pragma unroll
            for (int c = 0; c < L; ++c) acc[c] += wr * q[c];
        }
    }
#pragma unroll
    for (int c = 0; c < L; ++c) lds[rl][cl][c] = acc[c];
    __syncthreads();
    // thread t writes column (unit t / L, component t % L) of this workgroup
    for (int t = threadIdx.x; t < kDim0Cols * L; t += kBlock) {
        const int g = t / L, c = t % L;
        const size_t col = (static_cast<size_t>(blockIdx.x) * kDim0Cols + g) * L + c;
        if (col < cols) {
            double sum = lds[0][g][c];
#pragma unroll
            for (int k = 1; k < RL; ++k) sum += lds[k][g][c];
            partial[static_cast<size_t>(blockIdx.y) * cols + col] = sum;
        }
    }
}

// Pass 2: a workgroup owns 16 columns; 16 chunk lanes each add every 16th
// chunk partial, then the 16 lane sums are added in order.
__global__ __launch_bounds__(kBlock) void dim0_final(const double *__restrict__ partial,
                                                     size_t chunks, size_t cols,
                                                     float *__restrict__ out) {
    __shared__ double lds[16][17];
    const int cl = threadIdx.x & 15, kl = threadIdx.x >> 4;
    const size_t c = static_cast<size_t>(blockIdx.x) * 16 + cl;
    double acc = 0.0;
    if (c < cols) {
        size_t k = kl;
        for (; k + 16 * 7 < chunks; k += 16 * 8) {  // eight loads in flight
            double v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = partial[(k + 16 * j) * cols + c];
#pragma unroll
            for (int j = 0; j < 8; ++j) acc += v[j];
        }
        for (; k < chunks; k += 16) acc += partial[k * cols + c];
    }
    lds[kl][cl] = acc;
    __syncthreads();
    if (threadIdx.x < 16 && c < cols) {
        double sum = 0.0;
#pragma unroll
        for (int k = 0; k < 16; ++k) sum += lds[k][cl];
        out[c] = static_cast<float>(sum);
    }
}

// out[c] = sum_r w[r] * x[r][c] (w == nullptr: plain column sums) for a
// row-major [rows, cols] matrix with leading dimension ld.
int launch_colsum(const float *x, const float *w, size_t rows, size_t cols, size_t ld, float *out,
                  float *workspace, size_t workspace_floats, void *stream) {
    if (cols == 0) return TS_HIP_OK;
    if (!out) return TS_HIP_EINVAL;
    if (rows == 0) return ts_hip_fill(out, 0.0f, cols, stream);
    if (!x || ld != cols) return TS_HIP_EINVAL;
    const size_t chunks = dim0_chunks(rows, cols);
    if (!workspace || workspace_floats < 2 * chunks * cols) return TS_HIP_EWORKSPACE;
    if ((reinterpret_cast<uintptr_t>(workspace) & 7u) != 0) return TS_HIP_EINVAL;
    const size_t rows_per_chunk = (rows + chunks - 1) / chunks;
    double *partial = reinterpret_cast<double *>(workspace);
    hipStream_t s = as_stream(stream);
    const bool vec = (cols % 4 == 0) && aligned16(x);
    const size_t units = vec ? cols / 4 : cols;
    const size_t col_blocks = (units + kDim0Cols - 1) / kDim0Cols;
    if (col_blocks > 0x7fffffffULL) return TS_HIP_EINVAL;
    dim3 grid1(static_cast<unsigned>(col_blocks), static_cast<unsigned>(chunks));
    if (vec && w) launch((dim0_partial<true, true>), grid1, dim3(kBlock), 0, s, x, w, rows, cols, rows_per_chunk, partial);
    else if (vec) launch((dim0_partial<true, false>), grid1, dim3(kBlock), 0, s, x, w, rows, cols, rows_per_chunk, partial);
    else if (w) launch((dim0_partial<false, true>), grid1, dim3(kBlock), 0, s, x, w, rows, cols, rows_per_chunk, partial);
    else launch((dim0_partial<false, false>), grid1, dim3(kBlock), 0, s, x, w, rows, cols, rows_per_chunk, partial);
    int st = launch_status();
    if (st) return st;
    launch(dim0_final, dim3(static_cast<unsigned>((cols + 15) / 16)), dim3(kBlock), 0, s,
                       partial, chunks, cols, out);
    return launch_status();
}

}  // namespace tship

using namespace tship;

extern "C" {

size_t ts_hip_sum_workspace_floats(size_t n) { return 2 * sum_blocks(n); }

int ts_hip_sum(const float *x, size_t n, float *out, float *workspace, size_t workspace_floats,
               void *stream) {
    return launch_sum<false>(x, nullptr, n, out, workspace, workspace_floats, stream);
}

int ts_hip_mean(const float *x, size_t n, float *out, float *workspace, size_t workspace_floats,
                void *stream) {
    return launch_sum<true>(x, nullptr, n, out, workspace, workspace_floats, stream);
}

size_t ts_hip_sum_dim0_workspace_floats(size_t rows, size_t cols) {
    return 2 * dim0_chunks(rows, cols) * cols;
}

int ts_hip_sum_dim0(const float *x, size_t rows, size_t cols, float *out, float *workspace,
                    size_t workspace_floats, void *stream) {
    return launch_colsum(x, nullptr, rows, cols, cols, out, workspace, workspace_floats, stream);
}

int ts_hip_dot(const float *a, const float *b, size_t n, float *out, float *workspace, size_t workspace_floats,
               void *stream) {
    if (n && !b) return TS_HIP_EINVAL;
    return launch_sum<false>(a, b, n, out, workspace, workspace_floats, stream);
}

}  // extern "C"
