// Reductions of the gradtrack step: the scalar loss (sum / mean) and the
// bias-gradient column reduction sum_dims(&[0]).  Both are deterministic
// two-pass trees: per-thread f64 accumulation over a fixed slice, a wave64
// shuffle reduction, an LDS combine across the workgroup's four waves, one
// f64 partial per workgroup, then a single-workgroup pass in fixed order.
// No floating-point atomics, so every run gives the same bits.
#include "ts_hip_internal.h"

namespace tship {

// Pass 1: workgroup b sums its run of float4 groups [b * 256R, (b + 1) * 256R)
// (thread t: b * 256R + t, + 256, ...), then the elements past the groups
// with a grid stride, and writes one f64 partial (the partition of
// sum_blocks / sum_run).  PROD: the terms are x[i] * y[i] formed in f64 (a
// dot product).
template <bool PROD>
__global__ __launch_bounds__(kBlock) void sum_partial(const float *__restrict__ x, const float *__restrict__ y,
                                                      size_t n, size_t n4, size_t run,
                                                      double *__restrict__ partial) {
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    const size_t t = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
    const size_t base = static_cast<size_t>(blockIdx.x) * kBlock * run;
    const size_t end = base + kBlock * run < n4 ? base + kBlock * run : n4;
    double acc = 0.0;
    const float4 *x4 = reinterpret_cast<const float4 *>(x);
    const float4 *y4 = reinterpret_cast<const float4 *>(y);
    for (size_t v = base + threadIdx.x; v < end; v += kBlock) {
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
    // partials t, t + 256, ... added in order; loads issued D at a time before
    // any is added (the partials come from every XCD's L2 through memory: one
    // latency per round, so 16384 partials take one round of 64)
    auto rounds = [&](auto d) {
        constexpr int D = decltype(d)::value;
        for (; i + kBlock * (D - 1) < nparts; i += kBlock * D) {
            double v[D];
#pragma unroll
            for (int j = 0; j < D; ++j) v[j] = partial[i + kBlock * j];
            // every load issued before the first add (left to itself the
            // scheduler moves each load down to its add, a few in flight)
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < D; ++j) acc += v[j];
        }
    };
    rounds(std::integral_constant<int, 64>{});
    rounds(std::integral_constant<int, 16>{});
    rounds(std::integral_constant<int, 4>{});
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

// Both passes in one workgroup (sum_small_body): at most small_blocks<PROD>()
// first-pass workgroups and the float4 path.
template <bool PROD, bool MEAN>
__global__ __launch_bounds__(kBlock) void sum_small(const float *__restrict__ x, const float *__restrict__ y,
                                                    size_t n, size_t n4, int blocks, float *out) {
    sum_small_body<PROD, MEAN>(x, y, n, n4, blocks, out);
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
    if (blocks <= static_cast<size_t>(y ? small_blocks<true>() : small_blocks<false>()) && n4 == n / 4) {
        // one launch, the same bits
        const int nb = static_cast<int>(blocks);
        if (y) launch(sum_small<true, MEAN>, dim3(1), dim3(kBlock), 0, s, x, y, n, n4, nb, out);
        else launch(sum_small<false, MEAN>, dim3(1), dim3(kBlock), 0, s, x, y, n, n4, nb, out);
        return launch_status();
    }
    const size_t run = sum_run(n);
    if (y)
        launch(sum_partial<true>, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, x, y, n, n4, run,
               partial);
    else
        launch(sum_partial<false>, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, x, y, n, n4, run,
               partial);
    int st = launch_status();
    if (st) return st;
    return launch_sum_final(partial, blocks, n, out, MEAN, s);
}

// ---- column reduction [rows, cols] -> [cols] --------------------------------
//
// The sum's order is fixed (see kColsumRows): each chunk of 64 rows is added
// row by row, groups of 8 chunk sums in chunk order, the group sums in group
// order, all in f64 from +0, then rounded to fp32.  The GEMM kernels that
// produce a bias gradient alongside the weight gradient follow the same
// order, so either path gives the same bits.
//
// Pass 1: thread (column unit u, chunk c) adds its chunk's rows in order (a
// column unit is a float4 of 4 adjacent columns when cols % 4 == 0 and x is
// 16-byte aligned, else one column), 16 rows in flight at a time, and writes
// one f64 partial per column and chunk.
// W: row r is weighted by w[r] (in f64) -- a transposed matrix-vector product.
// Workgroup b takes column block b % col_blocks of chunk b / col_blocks.
template <bool VEC, bool W>
__global__ __launch_bounds__(kBlock) void colsum_chunks(const float *__restrict__ x, const float *__restrict__ w,
                                                        size_t rows, size_t cols, size_t ld, size_t col_blocks,
                                                        double *__restrict__ partial) {
    constexpr int L = VEC ? 4 : 1;  // columns per unit
    constexpr int kFly = 16;        // rows in flight
    const size_t units = VEC ? cols / 4 : cols;
    const size_t chunk = blockIdx.x / col_blocks;
    const size_t u = (blockIdx.x % col_blocks) * kBlock + threadIdx.x;
    if (u >= units) return;
    const size_t r0 = chunk * kColsumRows;
    const size_t r1 = r0 + kColsumRows < rows ? r0 + kColsumRows : rows;
    double acc[L];
#pragma unroll
    for (int c = 0; c < L; ++c) acc[c] = 0.0;
    auto load = [&](size_t r, float (&q)[L]) {
        if (VEC) {
            const float4 v = *reinterpret_cast<const float4 *>(x + r * ld + 4 * u);
            q[0] = v.x; q[L > 1 ? 1 : 0] = v.y; q[L > 2 ? 2 : 0] = v.z; q[L > 3 ? 3 : 0] = v.w;
        } else {
            q[0] = x[r * ld + u];
        }
    };
    size_t r = r0;
    for (; r + kFly <= r1; r += kFly) {
        float q[kFly][L];
#pragma unroll
        for (int k = 0; k < kFly; ++k) load(r + k, q[k]);
#pragma unroll
        for (int k = 0; k < kFly; ++k) {
            const double wr = W ? (double)w[r + k] : 1.0;
#pragma unroll
            for (int c = 0; c < L; ++c) acc[c] += W ? wr * q[k][c] : (double)q[k][c];
        }
    }
    for (; r < r1; ++r) {
        float q[L];
        load(r, q);
        const double wr = W ? (double)w[r] : 1.0;
#pragma unroll
        for (int c = 0; c < L; ++c) acc[c] += W ? wr * q[c] : (double)q[c];
    }
#pragma unroll
    for (int c = 0; c < L; ++c) partial[chunk * cols + u * L + c] = acc[c];
}

// Pass 2: a workgroup takes 16 columns; in rounds of 16 groups, thread
// (group lane gl, column cl) adds its group's chunk sums (8 loads in flight),
// and the group sums are added in group order by the first lane.
__global__ __launch_bounds__(kBlock) void colsum_final(const double *__restrict__ partial, size_t chunks,
                                                       size_t cols, float *__restrict__ out) {
    constexpr int G = static_cast<int>(kColsumGroup);
    __shared__ double gs[16][17];
    const int cl = threadIdx.x & 15, gl = threadIdx.x >> 4;
    const size_t c = static_cast<size_t>(blockIdx.x) * 16 + cl;
    const size_t groups = (chunks + G - 1) / G;
    double total = 0.0;
    for (size_t g0 = 0; g0 < groups; g0 += 16) {  // uniform
        const size_t g = g0 + gl;
        double sum = 0.0;
        if (c < cols && g < groups) {
            double v[G];
#pragma unroll
            for (int j = 0; j < G; ++j) v[j] = g * G + j < chunks ? partial[(g * G + j) * cols + c] : 0.0;
#pragma unroll
            for (int j = 0; j < G; ++j) sum += v[j];
        }
        gs[gl][cl] = sum;
        __syncthreads();
        if (gl == 0)
            for (int j = 0; j < 16; ++j) total += gs[j][cl];  // groups past the end add +0
        __syncthreads();
    }
    if (gl == 0 && c < cols) out[c] = static_cast<float>(total);
}

// Many groups (tall inputs): the group sums first, in parallel -- thread
// (group g, column c) adds chunk sums 8g .. 8g+7 in order from +0, as
// colsum_final's lanes do, and writes the result over chunk sum 8g (only that
// thread reads or writes those slots) -- then colsum_groups_final adds them in
// group order.  The same additions in the same order, so the same bits; the
// serial part is one dependent add per group instead of a round of loads,
// two barriers and 16 adds per 16 groups.
__global__ __launch_bounds__(kBlock) void colsum_groups(double *__restrict__ partial, size_t chunks, size_t cols) {
    constexpr int G = static_cast<int>(kColsumGroup);
    const size_t groups = (chunks + G - 1) / G;
    const size_t t = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (t >= groups * cols) return;
    const size_t g = t / cols, c = t % cols;
    double v[G];
#pragma unroll
    for (int j = 0; j < G; ++j) v[j] = g * G + j < chunks ? partial[(g * G + j) * cols + c] : 0.0;
    double sum = 0.0;
#pragma unroll
    for (int j = 0; j < G; ++j) sum += v[j];
    partial[g * G * cols + c] = sum;
}

// A workgroup takes 16 columns; in rounds of 256 groups thread (gl, cl)
// loads the group sums of groups g0 + 16*gl .. +15 (16 in flight) into LDS,
// and the first lane of each column adds the round's 256 in group order.
constexpr int kGroupsPerLane = 16;
__global__ __launch_bounds__(kBlock) void colsum_groups_final(const double *__restrict__ partial, size_t chunks,
                                                              size_t cols, float *__restrict__ out) {
    constexpr int G = static_cast<int>(kColsumGroup), R = 16 * kGroupsPerLane;
    __shared__ double gs[R][17];
    const int cl = threadIdx.x & 15, gl = threadIdx.x >> 4;
    const size_t c = static_cast<size_t>(blockIdx.x) * 16 + cl;
    const size_t groups = (chunks + G - 1) / G;
    double total = 0.0;
    for (size_t g0 = 0; g0 < groups; g0 += R) {  // uniform
        double v[kGroupsPerLane];
#pragma unroll
        for (int k = 0; k < kGroupsPerLane; ++k) {
            const size_t g = g0 + static_cast<size_t>(gl) * kGroupsPerLane + k;
            v[k] = (c < cols && g < groups) ? partial[g * G * cols + c] : 0.0;
        }
#pragma unroll
        for (int k = 0; k < kGroupsPerLane; ++k) gs[gl * kGroupsPerLane + k][cl] = v[k];
        __syncthreads();
        if (gl == 0)
            for (int j = 0; j < R; ++j) total += gs[j][cl];  // groups past the end add +0
        __syncthreads();
    }
    if (gl == 0 && c < cols) out[c] = static_cast<float>(total);
}

// Past this many groups of chunk sums the group sums run as a pass of their own.
constexpr size_t kColsumSerialGroups = 16;

int launch_colsum_final(double *partial, size_t chunks, size_t cols, float *out, hipStream_t s) {
    const size_t groups = (chunks + kColsumGroup - 1) / kColsumGroup;
    const dim3 grid(static_cast<unsigned>((cols + 15) / 16));
    if (groups <= kColsumSerialGroups) {
        launch(colsum_final, grid, dim3(kBlock), 0, s, partial, chunks, cols, out);
        return launch_status();
    }
    const size_t threads = groups * cols;
    if ((threads + kBlock - 1) / kBlock > 0x7fffffffULL) return TS_HIP_EINVAL;
    // the group sums overwrite chunk sums in place (partial is the caller's workspace)
    launch(colsum_groups, dim3(static_cast<unsigned>((threads + kBlock - 1) / kBlock)), dim3(kBlock), 0, s, partial,
           chunks, cols);
    const int st = launch_status();
    if (st) return st;
    launch(colsum_groups_final, grid, dim3(kBlock), 0, s, partial, chunks, cols, out);
    return launch_status();
}

// out[c] = sum_r w[r] * x[r][c] (w == nullptr: plain column sums) for a
// row-major [rows, cols] matrix with leading dimension ld >= cols.
int launch_colsum(const float *x, const float *w, size_t rows, size_t cols, size_t ld, float *out,
                  float *workspace, size_t workspace_floats, void *stream) {
    if (cols == 0) return TS_HIP_OK;
    if (!out) return TS_HIP_EINVAL;
    if (rows == 0) return ts_hip_fill(out, 0.0f, cols, stream);
    if (!x || ld < cols) return TS_HIP_EINVAL;
    const size_t chunks = colsum_chunk_count(rows);
    if (!workspace || workspace_floats < 2 * chunks * cols) return TS_HIP_EWORKSPACE;
    if ((reinterpret_cast<uintptr_t>(workspace) & 7u) != 0) return TS_HIP_EINVAL;
    double *partial = reinterpret_cast<double *>(workspace);
    hipStream_t s = as_stream(stream);
    const bool vec = (cols % 4 == 0) && (ld % 4 == 0) && aligned16(x);
    const size_t units = vec ? cols / 4 : cols;
    const size_t col_blocks = (units + kBlock - 1) / kBlock;
    if (col_blocks * chunks > 0x7fffffffULL) return TS_HIP_EINVAL;
    const dim3 grid1(static_cast<unsigned>(col_blocks * chunks));
    if (vec && w) launch((colsum_chunks<true, true>), grid1, dim3(kBlock), 0, s, x, w, rows, cols, ld, col_blocks, partial);
    else if (vec) launch((colsum_chunks<true, false>), grid1, dim3(kBlock), 0, s, x, w, rows, cols, ld, col_blocks, partial);
    else if (w) launch((colsum_chunks<false, true>), grid1, dim3(kBlock), 0, s, x, w, rows, cols, ld, col_blocks, partial);
    else launch((colsum_chunks<false, false>), grid1, dim3(kBlock), 0, s, x, w, rows, cols, ld, col_blocks, partial);
    int st = launch_status();
    if (st) return st;
    return launch_colsum_final(partial, chunks, cols, out, s);
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
    return 2 * colsum_chunk_count(rows) * cols;
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
