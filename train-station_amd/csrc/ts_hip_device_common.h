// Device helpers shared by the library's kernels and by the elementwise
// programs compiled at run time (ts_hip_map.hip), which include this header
// through hipRTC: plain device code, no host API.
#pragma once

namespace tship {

constexpr int kBlock = 256;  // 4 wave64 per workgroup

typedef float f4v_t __attribute__((ext_vector_type(4)));

// A pack of element offsets, C... = 0 .. W-1 (W consecutive elements per thread).
template <unsigned long... C>
struct Seq {};

// ---- the scalar sum's tree (ts_hip_sum, and the fused sum of ts_hip_map,
// which must give the same bits) ----------------------------------------------

__device__ inline double wave_sum(double v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Sum of a workgroup's per-thread values, returned to thread 0.
__device__ inline double block_sum(double v) {
    __shared__ double lds[kBlock / 64];
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) lds[wave] = v;
    __syncthreads();
    double r = 0.0;
    if (threadIdx.x == 0) {
#pragma unroll
        for (int w = 0; w < kBlock / 64; ++w) r += lds[w];
    }
    return r;
}

}  // namespace tship
