// Shared helpers of the gfx950 backend (device code and launchers).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "ts_hip.h"
#include "ts_hip_device_common.h"

namespace tship {

// Status of a launch: the error the runtime recorded for it, if any.
inline int launch_status() {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? TS_HIP_OK : static_cast<int>(e);
}

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// The calling thread's kernel timing window (ts_hip_timing_begin/end), or null.
struct TimingWindow {
    hipEvent_t start, stop;
    int kernels;
};
TimingWindow *timing_window();

// Products held by the calling thread's open launch group
// (ts_hip_launch_group_begin): true while any is held.  A kernel launched
// while they are held is launched after them (flush_launch_group first), so
// the stream sees every launch in the order it was issued.
bool launch_group_holding();
void flush_launch_group();

template <typename... KArgs, typename... Args>
inline void launch_now(void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t lds, hipStream_t s,
                       Args... args);

// Every kernel of the library is launched through here: a plain launch, or,
// inside a timing window, one that carries the window's events in its
// dispatch (the first kernel the start event, each kernel the stop event).
template <typename... KArgs, typename... Args>
inline void launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t lds, hipStream_t s,
                   Args... args) {
    if (launch_group_holding()) flush_launch_group();
    launch_now(kernel, grid, block, lds, s, args...);
}

template <typename... KArgs, typename... Args>
inline void launch_now(void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t lds, hipStream_t s,
                       Args... args) {
    TimingWindow *w = timing_window();
    if (!w) {
        kernel<<<grid, block, lds, s>>>(args...);
        return;
    }
    hipExtLaunchKernelGGL(kernel, grid, block, lds, s, w->kernels == 0 ? w->start : nullptr, w->stop, 0u,
                          static_cast<KArgs>(args)...);
    ++w->kernels;
}

// The same for a kernel of a code object compiled at run time (the compiled
// elementwise programs of ts_hip_map): blocks workgroups of `threads`.
inline hipError_t launch_module(hipFunction_t f, unsigned blocks, unsigned threads, hipStream_t s, void **params) {
    if (launch_group_holding()) flush_launch_group();
    TimingWindow *w = timing_window();
    if (!w) return hipModuleLaunchKernel(f, blocks, 1, 1, threads, 1, 1, 0, s, params, nullptr);
    const hipError_t e = hipExtModuleLaunchKernel(f, blocks * threads, 1, 1, threads, 1, 1, 0, s, params, nullptr,
                                                  w->kernels == 0 ? w->start : nullptr, w->stop, 0u);
    if (e == hipSuccess) ++w->kernels;
    return e;
}

// Number of compute units of the current device (cached per device).
int device_cu_count();

// Grid size for a grid-stride kernel covering `units` work items with
// kBlock threads each handling `per_thread` items: enough workgroups to fill
// every CU several times over, never more than the work needs.
inline unsigned grid_for(size_t units, size_t per_thread = 1) {
    size_t per_block = static_cast<size_t>(kBlock) * per_thread;
    size_t need = (units + per_block - 1) / per_block;
    size_t cap = static_cast<size_t>(device_cu_count()) * 16;
    if (need > cap) need = cap;
    return static_cast<unsigned>(need < 1 ? 1 : need);
}

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Non-temporal 16-byte store / load (the nt cache policy): for streams that
// are written, or read, once per kernel.
__device__ __forceinline__ void store_nt(float4 *p, float4 v) {
    const f4v_t r = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(r, reinterpret_cast<f4v_t *>(p));
}
__device__ __forceinline__ float4 load_nt(const float4 *p) {
    const f4v_t r = __builtin_nontemporal_load(reinterpret_cast<const f4v_t *>(p));
    return make_float4(r.x, r.y, r.z, r.w);
}

// ---- the scalar sum's partition (ts_hip_sum, and the fused sum of ts_hip_map,
// which must give the same bits) ----------------------------------------------

//
// First-pass workgroup b takes the float4 groups [b * 256R, (b + 1) * 256R)
// (those below n4), R = sum_run(n) groups per thread: thread t adds groups
// b * 256R + t, + 256, ... in order, then the single elements past the groups,
// 4 * n4 + T, T + 256 * blocks, ... (T = 256b + t, a grid stride).  Up to
// kSumFlatBlocks workgroups a thread takes one group; past that four, in as
// many workgroups as that takes (at most kSumMaxBlocks, then more groups per
// thread).  Each workgroup covers a contiguous range and ends after a few
// groups, so the hardware hands the next one to whichever CU frees first.
// With a fixed grid striding over the whole input (2048 workgroups, a group
// per thread per step), workgroups of one launch took from 0.3x to 1.5x
// their median time and the launch ended with the slowest: the same
// 24 B/element pass over 2^26 elements with its sum took 334 us that way and
// 297 us with four groups per thread here.
constexpr size_t kSumChunk = 1024;  // inputs per first-pass workgroup at one group of 4 per thread
constexpr size_t kSumFlatBlocks = 2048;
constexpr size_t kSumRun = 4;
constexpr size_t kSumMaxBlocks = 65536;

// Groups per thread of the first pass over n inputs.
inline size_t sum_run(size_t n) {
    if ((n + kSumChunk - 1) / kSumChunk <= kSumFlatBlocks) return 1;
    const size_t r = (n + kSumChunk * kSumMaxBlocks - 1) / (kSumChunk * kSumMaxBlocks);
    return r < kSumRun ? kSumRun : r;
}

// First-pass workgroups over n inputs (every group and element covered:
// 1024 * R * blocks >= n).
inline size_t sum_blocks(size_t n) {
    const size_t per = kSumChunk * sum_run(n);
    const size_t b = (n + per - 1) / per;
    return b < 1 ? 1 : b;
}

// Both passes of the sum in one workgroup, for at most small_blocks<PROD>()
// first-pass workgroups and the float4 path (n4 == n / 4): the operations,
// and so the bits, of the first pass's workgroups and the second pass.  With
// that few workgroups the grid stride covers every float4 group, so virtual
// thread (b, t) of first-pass workgroup b has at most one group and one tail
// element; thread t holds them for every b (all loads in flight at once),
// each b's wave sums are formed as block_sum forms them and added in wave
// order from +0 (a partial), and thread t then adds partials t, t + 256, ...
// from +0 as the second pass's threads do, combined as block_sum combines
// them.  Run by every thread of a workgroup of at least kBlock threads: the
// threads past kBlock take no values but reach the barriers.  out[0] is
// written by thread 0.  Used by ts_hip_sum's one-launch path and by the
// workgroup a weight-gradient product appends to add up its B operand.
constexpr int kSumSmallBlocks = 16;
// a product's two operands take twice the registers: half as many workgroups
template <bool PROD>
constexpr int small_blocks() { return PROD ? kSumSmallBlocks / 2 : kSumSmallBlocks; }

template <bool PROD, bool MEAN>
__device__ __forceinline__ void sum_small_body(const float *x, const float *y, size_t n, size_t n4, int blocks,
                                               float *out) {
    constexpr int NB = small_blocks<PROD>();
    constexpr int kWaves = kBlock / 64;
    __shared__ double wsum[NB][kWaves];
    __shared__ double parts[NB];
    __shared__ double fin[kWaves];
    const int t = static_cast<int>(threadIdx.x), lane = t & 63, wave = t >> 6;
    if (wave < kWaves) {  // uniform per wave
        // every load issued before any is used (a load consumed in its own
        // conditional block is waited for there, one latency per block):
        // addresses clamped into the input, values past it not added.  The
        // tail (n - 4*n4 < 4 elements) falls to threads 0..2 of block 0.
        const size_t ti = 4 * n4 + t < n ? 4 * n4 + t : n - 1;
        const float tx = x[ti], ty = PROD ? y[ti] : 0.0f;
        float4 q[NB], qy[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            q[b] = qy[b] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (b < blocks && n4 > 0) {  // uniform
                const size_t v = static_cast<size_t>(b) * kBlock + t;
                const size_t vc = v < n4 ? v : n4 - 1;
                q[b] = reinterpret_cast<const float4 *>(x)[vc];
                if (PROD) qy[b] = reinterpret_cast<const float4 *>(y)[vc];
            }
        }
        double acc[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            acc[b] = 0.0;
            const size_t v = static_cast<size_t>(b) * kBlock + t;
            if (b < blocks && v < n4) {
                if (PROD)
                    acc[b] += (double)q[b].x * (double)qy[b].x + (double)q[b].y * (double)qy[b].y +
                              (double)q[b].z * (double)qy[b].z + (double)q[b].w * (double)qy[b].w;
                else
                    acc[b] += (double)q[b].x + (double)q[b].y + (double)q[b].z + (double)q[b].w;
            }
        }
        if (4 * n4 + t < n) acc[0] += PROD ? (double)tx * (double)ty : (double)tx;
        // every workgroup's butterfly formed (independent chains the compiler
        // interleaves; one behind a branch each would run one after another),
        // the unused ones dropped
        double ws[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) ws[b] = wave_sum(acc[b]);
#pragma unroll
        for (int b = 0; b < NB; ++b)
            if (b < blocks && lane == 0) wsum[b][wave] = ws[b];
    }
    __syncthreads();
    if (t < blocks) {
        double r = 0.0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) r += wsum[t][w];
        parts[t] = r;
    }
    __syncthreads();
    if (wave < kWaves) {  // block_sum over the first kBlock threads
        double a = 0.0;
        if (t < blocks) a += parts[t];
        a = wave_sum(a);
        if (lane == 0) fin[wave] = a;
    }
    __syncthreads();
    if (t == 0) {
        double r = 0.0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) r += fin[w];
        const float s = static_cast<float>(r);
        out[0] = MEAN ? s / static_cast<float>(n) : s;
    }
}

// The sum's second pass: one workgroup adds the nparts f64 partials in a fixed
// order and writes the fp32 sum (divided by (float)n when mean) to out[0].
int launch_sum_final(const double *partial, size_t nparts, size_t n, float *out, bool mean, hipStream_t s);

// ---- the column sum's order (ts_hip_sum_dim0, and the bias gradient the
// weight-gradient GEMM produces alongside its product, which must give the
// same bits) ---------------------------------------------------------------------
//
// Rows are taken in chunks of kColsumRows: a chunk's rows are added in row
// order, a group of kColsumGroup consecutive chunks' sums in chunk order, the
// group sums in group order -- each sum in f64 starting from +0 -- and the
// total is rounded to fp32 once.  (Starting from +0 no partial is ever -0, so
// zero padding past the last row or chunk changes nothing.)
constexpr size_t kColsumRows = 64;
constexpr size_t kColsumGroup = 8;

__host__ __device__ inline size_t colsum_chunk_count(size_t rows) { return (rows + kColsumRows - 1) / kColsumRows; }

// Weighted column sums out[c] = sum_r w[r] * x[r][c] (w == nullptr: plain
// column sums) in that order; workspace as ts_hip_sum_dim0_workspace_floats.
int launch_colsum(const float *x, const float *w, size_t rows, size_t cols, size_t ld, float *out,
                  float *workspace, size_t workspace_floats, void *stream);

// The column sum's second pass: out[c] = the chunk sums partial[k * cols + c]
// added by groups as above, rounded to fp32.
int launch_colsum_final(double *partial, size_t chunks, size_t cols, float *out, hipStream_t s);

}  // namespace tship
