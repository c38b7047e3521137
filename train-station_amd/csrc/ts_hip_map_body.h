// The loop of a fused elementwise pass (ts_hip_map of include/ts_hip.h),
// shared by the interpreter of ts_hip_map.hip and by the programs compiled at
// run time, which include this header through hipRTC (plain device code).
//
// A pass evaluates a program of elementwise ops over up to five inputs, four
// consecutive elements per thread: the elements' register files are arrays
// r0 .. r3 of TS_HIP_MAP_REGS floats.  The program policy P supplies
//   P::run(a, i0, zmin, Seq<C...>, r...)  the ops, over W = sizeof...(C) elements
//   P::in_reg(a, j)                      the register of per-element input j
//   P::out_reg(a, o), P::red_reg(a)      the registers stored to output o / summed
// The interpreter reads all of these from the program at run time; a compiled
// program has them as constants, so its register files are plain registers.
#pragma once

#include "ts_hip.h"
#include "ts_hip_device_common.h"

namespace tship {

constexpr int kMapIn = TS_HIP_MAP_MAX_INPUTS;
constexpr int kMapOps = TS_HIP_MAP_MAX_OPS;
constexpr int kMapOut = TS_HIP_MAP_MAX_OUTPUTS;
constexpr int kMapRegs = TS_HIP_MAP_REGS;
static_assert(kMapRegs == 16 && kMapIn <= kMapRegs, "the register file is a power-of-two tuple");
// A division checked for zero divisors, as the launcher rewrites it: the op
// loop then never reads an op's flags (read there, the byte came through a
// vector load whose wait drained the next group's input loads at every
// division).
constexpr uint8_t kMapDivChecked = TS_HIP_MAP_SQUARE + 1;

using Seq1 = Seq<0>;
using Seq4 = Seq<0, 1, 2, 3>;

struct MapArgsK {
    ts_hip_map_program p;
    size_t n, n4, tail_start, check_start;
    size_t run;  // float4 groups per thread (the sum's partition, sum_run)
    unsigned long long *zero_index;
    bool vec;  // every input and output is 16-byte aligned
    double *partial;  // reduce: one f64 partial per workgroup
    // the inputs read per element (not scalar), compacted: pointer and register
    const float *vin[kMapIn];
    int vreg[kMapIn];
};

// Every input of element(s) i0 .. into its register (the register of input k
// is k): a constant or scalar input's one value, else the element(s).
template <unsigned long... C, class... R>
__device__ __forceinline__ void load_inputs(const MapArgsK &a, size_t i0, bool vec4, Seq<C...>, R &...r) {
    const ts_hip_map_program &p = a.p;
#pragma unroll
    for (int k = 0; k < kMapIn; ++k) {
        if (k >= static_cast<int>(p.n_inputs)) break;
        const float *in = p.inputs[k];
        if (p.const_inputs & (1u << k)) {
            ((r[k] = p.const_values[k]), ...);
        } else if (p.scalar_inputs & (1u << k)) {
            const float s = in[0];
            ((r[k] = s), ...);
        } else if (vec4) {
            const float4 q = *reinterpret_cast<const float4 *>(in + i0);
            const float v[4] = {q.x, q.y, q.z, q.w};
            ((r[k] = v[C]), ...);
        } else {
            ((r[k] = in[i0 + C]), ...);
        }
    }
}

template <class P, unsigned long... C, class... R>
__device__ __forceinline__ void store_outputs(const MapArgsK &a, size_t i0, bool vec4, Seq<C...>, R &...r) {
    const ts_hip_map_program &p = a.p;
#pragma unroll
    for (int o = 0; o < kMapOut; ++o) {
        if (o >= static_cast<int>(p.n_outputs)) break;
        const int q = P::out_reg(a, o);
        float *out = p.outputs[o];
        if (vec4) {
            // ordinary stores: the value is usually read again soon (a
            // gradient by the next op, a forward value by its consumer)
            float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            ((v[C] = r[q]), ...);
            *reinterpret_cast<float4 *>(out + i0) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
            ((out[i0 + C] = r[q]), ...);
        }
    }
}

// Groups of four elements in ts_hip_sum's partition: workgroup b takes the
// groups [b * 256R, (b + 1) * 256R), R = a.run, thread t groups b * 256R + t,
// + 256, ..., then the elements past the groups with a grid stride (with a
// reduction each group's four values added in f64 left to right, then the
// remaining elements, so the sum has the bits of ts_hip_sum over the stored
// values); the next group's inputs loaded before the current group is
// evaluated, so a wave keeps loads in flight while it computes.
//
// 16-byte aligned operands, NV inputs read per element and NO stored values
// known at compile time: every iteration then issues exactly NV loads and NO
// stores (the next group's index clamped into range, a division's zero check
// kept in a register and reported after the loop), so the compiler's load
// counters are exact and the loop waits only for the next group's loads,
// never for its own stores to complete.
template <bool REDUCE, int NV, int NO, class P>
__device__ __forceinline__ void map_vec_body(const MapArgsK &a) {
    const size_t t = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    const size_t base = static_cast<size_t>(blockIdx.x) * kBlock * a.run;
    const size_t end = base + kBlock * a.run < a.n4 ? base + kBlock * a.run : a.n4;
    const size_t g0 = base + threadIdx.x;
    const int rq = P::red_reg(a);
    double acc = 0.0;
    unsigned long long zmin = ~0ull;
    float sv[kMapIn];  // scalar and constant inputs, read once
#pragma unroll
    for (int k = 0; k < kMapIn; ++k)
        sv[k] = k >= static_cast<int>(a.p.n_inputs)           ? 0.0f
                : (a.p.const_inputs & (1u << k))            ? a.p.const_values[k]
                : (a.p.scalar_inputs & (1u << k))           ? a.p.inputs[k][0]
                                                            : 0.0f;
    f4v_t nx[NV > 0 ? NV : 1];  // the next group's per-element inputs
    auto fetch = [&](size_t g) {
#pragma unroll
        for (int j = 0; j < NV; ++j) nx[j] = *reinterpret_cast<const f4v_t *>(a.vin[j] + 4 * g);
    };
    if (g0 < end) fetch(g0);
    for (size_t g = g0; g < end; g += kBlock) {
        float r0[kMapRegs], r1[kMapRegs], r2[kMapRegs], r3[kMapRegs];
#pragma unroll
        for (int k = 0; k < kMapIn; ++k) {
            r0[k] = sv[k];
            r1[k] = sv[k];
            r2[k] = sv[k];
            r3[k] = sv[k];
        }
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int k = P::in_reg(a, j);
            r0[k] = nx[j][0];
            r1[k] = nx[j][1];
            r2[k] = nx[j][2];
            r3[k] = nx[j][3];
        }
        const size_t gn = g + kBlock < end ? g + kBlock : end - 1;  // in range: the same loads every step
        fetch(gn);
        P::run(a, 4 * g, zmin, Seq4{}, r0, r1, r2, r3);
#pragma unroll
        for (int o = 0; o < NO; ++o) {
            const int q = P::out_reg(a, o);
            f4v_t v;
            v[0] = r0[q];
            v[1] = r1[q];
            v[2] = r2[q];
            v[3] = r3[q];
            *reinterpret_cast<f4v_t *>(a.p.outputs[o] + 4 * g) = v;
        }
        if (REDUCE) acc += (double)r0[rq] + (double)r1[rq] + (double)r2[rq] + (double)r3[rq];
    }
    for (size_t i = 4 * a.n4 + t; i < a.n; i += stride) {
        float r0[kMapRegs];
        load_inputs(a, i, false, Seq1{}, r0);
        P::run(a, i, zmin, Seq1{}, r0);
        store_outputs<P>(a, i, false, Seq1{}, r0);
        if (REDUCE) acc += (double)r0[rq];
    }
    if (zmin != ~0ull) atomicMin(a.zero_index, zmin);
    if (REDUCE) {
        const double s = block_sum(acc);
        if (threadIdx.x == 0) a.partial[blockIdx.x] = s;
    }
}

// Any alignment and counts: the same evaluation with element loads.
template <bool REDUCE, class P>
__device__ __forceinline__ void map_any_body(const MapArgsK &a) {
    const size_t t = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    const size_t base = static_cast<size_t>(blockIdx.x) * kBlock * a.run;
    const size_t end = base + kBlock * a.run < a.n4 ? base + kBlock * a.run : a.n4;
    const int rq = P::red_reg(a);
    double acc = 0.0;
    unsigned long long zmin = ~0ull;
    for (size_t g = base + threadIdx.x; g < end; g += kBlock) {
        float r0[kMapRegs], r1[kMapRegs], r2[kMapRegs], r3[kMapRegs];
        load_inputs(a, 4 * g, a.vec, Seq4{}, r0, r1, r2, r3);
        P::run(a, 4 * g, zmin, Seq4{}, r0, r1, r2, r3);
        store_outputs<P>(a, 4 * g, a.vec, Seq4{}, r0, r1, r2, r3);
        if (REDUCE) acc += (double)r0[rq] + (double)r1[rq] + (double)r2[rq] + (double)r3[rq];
    }
    for (size_t i = 4 * a.n4 + t; i < a.n; i += stride) {
        float r0[kMapRegs];
        load_inputs(a, i, false, Seq1{}, r0);
        P::run(a, i, zmin, Seq1{}, r0);
        store_outputs<P>(a, i, false, Seq1{}, r0);
        if (REDUCE) acc += (double)r0[rq];
    }
    if (zmin != ~0ull) atomicMin(a.zero_index, zmin);
    if (REDUCE) {
        const double s = block_sum(acc);
        if (threadIdx.x == 0) a.partial[blockIdx.x] = s;
    }
}

}  // namespace tship
