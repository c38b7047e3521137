// Shape-general kernels: NumPy broadcasting (tensor/ops/broadcasting.rs:
// 299-478) and sums over any set of axes (sum_dims / mean_dims,
// tensor/reductions/{sum,mean}.rs, and the gradient reduction of
// grad_fn/utils.rs:23-60), up to rank 8.
//
// broadcast_gather: out[i] = src[offset of i's coordinates], with the source
// strides of broadcast axes set to 0 -- the reference materialises the same
// values with broadcast_copy_data.  HBM-bound: 4 B written per element, the
// source read through the caches.
//
// reduce_axes: output element o (keepdim layout) sums the input elements
// whose kept coordinates equal o's, in f64, in a fixed order: G lanes per
// output (1, 64 or 256, chosen from the shape) each add a strided share of
// the reduced index space, then a shuffle / LDS tree combines them.
#include "ts_hip_internal.h"

namespace tship {

constexpr int kMaxRank = 8;

struct Layout {
    int rank;
    uint64_t dims[kMaxRank];
    uint64_t src_stride[kMaxRank];  // element stride in the source per output axis
};

__global__ __launch_bounds__(kBlock) void broadcast_gather(const float *__restrict__ src,
                                                           float *__restrict__ out, size_t n,
                                                           Layout L, float scale, int use_scale) {
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        size_t rem = i, off = 0;
        for (int k = L.rank - 1; k >= 0; --k) {
            const uint64_t c = rem % L.dims[k];
            rem /= L.dims[k];
            off += c * L.src_stride[k];
        }
        const float v = src[off];
        out[i] = use_scale ? v * scale : v;
    }
}

struct Reduction {
    int kept_rank, red_rank;
    uint64_t kept_dims[kMaxRank], kept_stride[kMaxRank];  // input strides of the kept axes
    uint64_t red_dims[kMaxRank], red_stride[kMaxRank];    // input strides of the reduced axes
    uint64_t n_out, n_red;
};

__device__ inline uint64_t kept_offset(const Reduction &R, uint64_t o) {
    uint64_t off = 0;
    for (int k = R.kept_rank - 1; k >= 0; --k) {
        off += (o % R.kept_dims[k]) * R.kept_stride[k];
        o /= R.kept_dims[k];
    }
    return off;
}

__device__ inline uint64_t red_offset(const Reduction &R, uint64_t r) {
    uint64_t off = 0;
    for (int k = R.red_rank - 1; k >= 0; --k) {
        off += (r % R.red_dims[k]) * R.red_stride[k];
        r /= R.red_dims[k];
    }
    return off;
}

// G lanes per output; G = 1 (a thread per output), 64 (a wave) or 256 (a workgroup)
template <int G>
__global__ __launch_bounds__(kBlock) void reduce_axes(const float *__restrict__ x, float *__restrict__ out,
                                                      Reduction R, float scale, int use_scale) {
    constexpr int kPerBlock = kBlock / G;
    const uint64_t o = static_cast<uint64_t>(blockIdx.x) * kPerBlock + threadIdx.x / G;
    const int lane = threadIdx.x % G;
    double acc = 0.0;
    if (o < R.n_out) {
        const uint64_t base = kept_offset(R, o);
        for (uint64_t r = lane; r < R.n_red; r += G) acc += static_cast<double>(x[base + red_offset(R, r)]);
    }
    if (G >= 64) {
#pragma unroll
        for (int d = 32; d > 0; d >>= 1) acc += __shfl_xor(acc, d, 64);
    }
    if (G == 256) {
        __shared__ double part[kBlock / 64];
        if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
        __syncthreads();
        if (threadIdx.x == 0) acc = ((part[0] + part[1]) + part[2]) + part[3];
    }
    if (lane == 0 && o < R.n_out) {
        const float s = static_cast<float>(acc);
        out[o] = use_scale ? s * scale : s;
    }
}

// ---- transposing two axes (transform/transpose.rs:156-208, materialised) ----
//
// out = src with axes d0 < d1 swapped, both row-major.  Viewing the source as
// [P, D0, M, D1, Q], the output is [P, D1, M, D0, Q].
//
// Q == 1 (d1 is the last axis, as in a matrix transpose): each (p, m) plane
// moves in 64 x 64 tiles through LDS, so a wave reads 64 consecutive floats
// of a source row and writes 64 consecutive floats of an output row; the LDS
// row pitch of 65 floats keeps the column reads conflict-free.  HBM-bound:
// 8 B per element.  Q > 1: runs of Q contiguous floats keep their order, a
// thread per element, reads and writes both along q.

struct TransposeDims {
    uint64_t P, D0, M, D1, Q;
    uint64_t tiles0, tiles1;  // 64-wide tiles along D0 and D1
};

__global__ __launch_bounds__(256) void transpose_tiles(const float *__restrict__ src, float *__restrict__ out,
                                                       TransposeDims T) {
    __shared__ float tile[64][65];
    const uint64_t per_plane = T.tiles0 * T.tiles1;
    const uint64_t b = blockIdx.x;
    const uint64_t plane = b / per_plane, t = b - plane * per_plane;
    const uint64_t i0 = (t / T.tiles1) * 64, j0 = (t % T.tiles1) * 64;
    const uint64_t p = plane / T.M, m = plane - p * T.M;
    const int c = static_cast<int>(threadIdx.x & 63u), r = static_cast<int>(threadIdx.x >> 6);
    // src[p, i, m, j] at ((p * D0 + i) * M + m) * D1 + j
    const float *sb = src + (p * T.D0 * T.M + m) * T.D1;
    const uint64_t in_row = T.M * T.D1;
    float v[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const uint64_t i = i0 + r + 4 * k, j = j0 + c;
        v[k] = (i < T.D0 && j < T.D1) ? sb[i * in_row + j] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) tile[r + 4 * k][c] = v[k];
    __syncthreads();
    // out[p, j, m, i] at ((p * D1 + j) * M + m) * D0 + i
    float *ob = out + (p * T.D1 * T.M + m) * T.D0;
    const uint64_t out_row = T.M * T.D0;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const uint64_t j = j0 + r + 4 * k, i = i0 + c;
        if (i < T.D0 && j < T.D1) ob[j * out_row + i] = tile[c][r + 4 * k];
    }
}

__global__ __launch_bounds__(kBlock) void transpose_runs(const float *__restrict__ src, float *__restrict__ out,
                                                         TransposeDims T, uint64_t n) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t o = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; o < n; o += stride) {
        uint64_t rest = o / T.Q;
        const uint64_t q = o - rest * T.Q;
        const uint64_t i = rest % T.D0;
        rest /= T.D0;
        const uint64_t m = rest % T.M;
        rest /= T.M;
        const uint64_t j = rest % T.D1, p = rest / T.D1;
        out[o] = src[(((p * T.D0 + i) * T.M + m) * T.D1 + j) * T.Q + q];
    }
}

}  // namespace tship

using namespace tship;

extern "C" {

int ts_hip_transpose(const float *src, const size_t *dims, size_t rank, size_t d0, size_t d1, float *out,
                     void *stream) {
    if (rank > 0 && !dims) return TS_HIP_EINVAL;
    if (d0 >= rank || d1 >= rank) return TS_HIP_EINVAL;
    uint64_t n = 1;
    for (size_t k = 0; k < rank; ++k) n *= dims[k];
    if (n == 0) return TS_HIP_OK;
    if (!src || !out) return TS_HIP_EINVAL;
    if (d0 == d1) return ts_hip_copy(src, out, n, stream);
    if (d0 > d1) {
        const size_t t = d0;
        d0 = d1;
        d1 = t;
    }
    TransposeDims T{1, dims[d0], 1, dims[d1], 1, 0, 0};
    for (size_t k = 0; k < d0; ++k) T.P *= dims[k];
    for (size_t k = d0 + 1; k < d1; ++k) T.M *= dims[k];
    for (size_t k = d1 + 1; k < rank; ++k) T.Q *= dims[k];
    hipStream_t s = as_stream(stream);
    if (T.Q == 1) {
        T.tiles0 = (T.D0 + 63) / 64;
        T.tiles1 = (T.D1 + 63) / 64;
        const uint64_t blocks = T.P * T.M * T.tiles0 * T.tiles1;
        if (blocks > 0x7fffffffULL) return TS_HIP_EINVAL;
        launch(transpose_tiles, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, src, out, T);
    } else {
        launch(transpose_runs, dim3(grid_for(n)), dim3(kBlock), 0, s, src, out, T, n);
    }
    return launch_status();
}


int ts_hip_broadcast_copy(const float *src, const size_t *src_dims, size_t src_rank, float *out,
                          const size_t *out_dims, size_t out_rank, float scale, int use_scale,
                          void *stream) {
    if (out_rank > static_cast<size_t>(kMaxRank) || src_rank > out_rank) return TS_HIP_EINVAL;
    if ((src_rank && !src_dims) || (out_rank && !out_dims)) return TS_HIP_EINVAL;
    size_t n = 1;
    for (size_t k = 0; k < out_rank; ++k) n *= out_dims[k];
    if (n == 0) return TS_HIP_OK;
    if (!src || !out) return TS_HIP_EINVAL;
    Layout L{};
    L.rank = static_cast<int>(out_rank);
    // source axes align to the right; a source axis of size 1 (or a missing one) repeats
    size_t stride = 1;
    for (size_t k = out_rank; k-- > 0;) {
        L.dims[k] = out_dims[k];
        const size_t j = k + src_rank - out_rank;  // wraps when the source lacks the axis
        if (k + src_rank >= out_rank) {
            const size_t d = src_dims[j];
            if (d != out_dims[k] && d != 1) return TS_HIP_EINVAL;
            L.src_stride[k] = (d == 1) ? 0 : stride;
            stride *= d;
        } else {
            L.src_stride[k] = 0;
        }
    }
    if (L.rank == 0) {  // scalar to scalar
        L.rank = 1;
        L.dims[0] = 1;
        L.src_stride[0] = 0;
    }
    launch(broadcast_gather, dim3(grid_for(n)), dim3(kBlock), 0, as_stream(stream), src, out, n, L,
                       scale, use_scale);
    return launch_status();
}

int ts_hip_reduce_sum(const float *x, const size_t *dims, size_t rank, unsigned reduce_mask, float *out,
                      float scale, int use_scale, void *stream) {
    if (rank > static_cast<size_t>(kMaxRank) || (rank && !dims)) return TS_HIP_EINVAL;
    if (rank < 32 && (reduce_mask >> rank) != 0) return TS_HIP_EINVAL;
    Reduction R{};
    uint64_t stride = 1, n_in = 1;
    uint64_t st[kMaxRank];
    for (size_t k = rank; k-- > 0;) {
        st[k] = stride;
        stride *= dims[k];
    }
    n_in = stride;
    R.n_out = 1;
    R.n_red = 1;
    for (size_t k = 0; k < rank; ++k) {
        if ((reduce_mask >> k) & 1u) {
            R.red_dims[R.red_rank] = dims[k];
            R.red_stride[R.red_rank++] = st[k];
            R.n_red *= dims[k];
        } else {
            R.kept_dims[R.kept_rank] = dims[k];
            R.kept_stride[R.kept_rank++] = st[k];
            R.n_out *= dims[k];
        }
    }
    if (R.n_out == 0) return TS_HIP_OK;
    if (!out) return TS_HIP_EINVAL;
    if (n_in == 0) return ts_hip_fill(out, 0.0f, R.n_out, stream);  // empty sums are 0
    if (!x) return TS_HIP_EINVAL;
    if (R.kept_rank == 0) {  // everything reduced: one output
        R.kept_rank = 1;
        R.kept_dims[0] = 1;
        R.kept_stride[0] = 0;
    }
    if (R.red_rank == 0) {
        R.red_rank = 1;
        R.red_dims[0] = 1;
        R.red_stride[0] = 0;
    }
    hipStream_t s = as_stream(stream);
    const uint64_t cus = static_cast<uint64_t>(device_cu_count());
    if (R.n_out >= cus * 256 || R.n_red < 64) {
        const uint64_t blocks = (R.n_out + kBlock - 1) / kBlock;
        if (blocks > 0x7fffffffULL) return TS_HIP_EINVAL;
        launch(reduce_axes<1>, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, x, out, R,
                           scale, use_scale);
    } else if (R.n_out >= cus * 4) {
        const uint64_t blocks = (R.n_out + 3) / 4;
        launch(reduce_axes<64>, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, x, out, R,
                           scale, use_scale);
    } else {
        launch(reduce_axes<256>, dim3(static_cast<unsigned>(R.n_out)), dim3(kBlock), 0, s, x, out,
                           R, scale, use_scale);
    }
    return launch_status();
}

}  // extern "C"
