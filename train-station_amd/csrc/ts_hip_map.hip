// Fused elementwise programs: one pass evaluates a short list of the
// elementwise operations of the gradtrack step (the same formulas, in the same
// fp32 order, as their separate kernels in ts_hip_elementwise.hip) over up to
// five inputs and stores up to four of the values, optionally adding one of
// them up as ts_hip_sum / ts_hip_mean would.  The host records a chain of
// elementwise ops as such a program and runs it when a value is first needed,
// so intermediates nobody reads are never written and shared inputs are read
// once.
//
// Registers: r[0 .. n_inputs) hold the inputs, r[kMapIn + k] the value of op
// k.  Each thread evaluates four consecutive elements at once; the register
// file is four arrays indexed by uniform (scalar) indices, which the compiler
// keeps in VGPRs (indexed moves), and each op's code selects its formula by a
// uniform branch.  An indexed array takes a power-of-two register tuple, so
// the limits (5 inputs + 11 ops = 16 registers, the config-2 backward as one
// program) keep the file at 4 x 16 VGPRs and the kernel at 4 waves per SIMD.
#include <utility>

#include "ts_hip_internal.h"

namespace tship {

constexpr int kMapIn = TS_HIP_MAP_MAX_INPUTS;
constexpr int kMapOps = TS_HIP_MAP_MAX_OPS;
constexpr int kMapOut = TS_HIP_MAP_MAX_OUTPUTS;
constexpr int kMapRegs = kMapIn + kMapOps;

struct MapArgsK {
    ts_hip_map_program p;
    size_t n, n4, tail_start, check_start;
    unsigned long long *zero_index;
    bool vec;  // every input and output is 16-byte aligned
    double *partial;  // reduce: one f64 partial per workgroup
    // the inputs read per element (not scalar), compacted: pointer and register
    const float *vin[kMapIn];
    int vreg[kMapIn];
};

// The register file of W consecutive elements: one local array per element,
// passed as a parameter pack so every element's array is named at compile
// time (a pointer chosen at run time, a 2-D array or arrays wrapped in one
// struct go to scratch; separate arrays with uniform indices stay in VGPRs,
// read and written with indexed moves).  C... are the elements' offsets.
template <size_t... C, class... R>
__device__ __forceinline__ void run_program(const MapArgsK &a, size_t i0, unsigned long long &zmin,
                                            std::index_sequence<C...>, R &...r) {
    constexpr int W = sizeof...(C);
    const ts_hip_map_program &p = a.p;
    // The compiler keeps this a loop (each op's fields read from the kernel
    // arguments, its result written with an indexed move).  Forced unrolled
    // (a compile-time op index: fields in scalar registers, static
    // destinations) and with the fields read one op ahead, the config-2
    // programs both ran 7% slower; unrolled, the kernel's code is ~6x larger.
#pragma unroll
    for (int k = 0; k < kMapOps; ++k) {
        if (k >= static_cast<int>(p.n_ops)) break;
        const ts_hip_map_op op = p.ops[k];
        // operands read once, the op's values formed in temporaries, the
        // register file written once after the switch (writing it in every
        // case makes the compiler keep several copies of it)
        const float x[W] = {r[op.a]...};
        const float y[W] = {r[op.b]...};
        float v[W];
        switch (op.code) {
            case TS_HIP_MAP_ADD: ((v[C] = x[C] + y[C]), ...); break;
            case TS_HIP_MAP_SUB: ((v[C] = x[C] - y[C]), ...); break;
            case TS_HIP_MAP_MUL: ((v[C] = x[C] * y[C]), ...); break;
            case TS_HIP_MAP_DIV: {
                if ((op.flags & TS_HIP_MAP_CHECKED) && a.zero_index) {
                    // the first zero divisor this thread sees (reported once, after its loop)
                    auto check = [&](float d, size_t i) {
                        if (i >= a.check_start && d == 0.0f && i < zmin) zmin = i;
                    };
                    (check(y[C], i0 + C), ...);
                }
                ((v[C] = x[C] / y[C]), ...);
                break;
            }
            case TS_HIP_MAP_NEG:  // core/utils.rs:847-870: 0 - x on the AVX2 body, -x on the tail
                ((v[C] = (i0 + C < a.tail_start) ? 0.0f - x[C] : -x[C]), ...);
                break;
            case TS_HIP_MAP_RELU: ((v[C] = x[C] > 0.0f ? x[C] : 0.0f), ...); break;
            // grad_fn/ops/relu.rs: x > 0 ? go : 0 (a = x, b = go)
            case TS_HIP_MAP_RELU_BWD: ((v[C] = x[C] > 0.0f ? y[C] : 0.0f), ...); break;
            case TS_HIP_MAP_ADD_S: ((v[C] = x[C] + op.imm), ...); break;
            case TS_HIP_MAP_SUB_S: ((v[C] = x[C] - op.imm), ...); break;
            case TS_HIP_MAP_MUL_S: ((v[C] = x[C] * op.imm), ...); break;
            case TS_HIP_MAP_DIV_S: ((v[C] = x[C] / op.imm), ...); break;
            default: ((v[C] = x[C] * x[C]), ...); break;  // TS_HIP_MAP_SQUARE: pow_scalar(2)
        }
        const int d = kMapIn + static_cast<int>(k);
        ((r[d] = v[C]), ...);
    }
}

template <size_t... C, class... R>
__device__ __forceinline__ void load_inputs(const MapArgsK &a, size_t i0, bool vec4, std::index_sequence<C...>,
                                            R &...r) {
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

template <size_t... C, class... R>
__device__ __forceinline__ void store_outputs(const MapArgsK &a, size_t i0, bool vec4, std::index_sequence<C...>,
                                              R &...r) {
    const ts_hip_map_program &p = a.p;
#pragma unroll
    for (int o = 0; o < kMapOut; ++o) {
        if (o >= static_cast<int>(p.n_outputs)) break;
        const int q = p.output_regs[o];
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

// Groups of four elements, grid-stride: thread t takes groups t, t + stride,
// ... (with a reduction the grid and order of ts_hip_sum's first pass: each
// group's four values added in f64 left to right, then the remainder, so the
// sum has the bits of ts_hip_sum over the stored values), the next group's
// inputs loaded before the current group is evaluated, so a wave keeps loads
// in flight while it computes.
//
// map_program_vec: 16-byte aligned operands, NV inputs read per element and NO
// stored values known at compile time.  Every iteration then issues exactly
// NV loads and NO stores (the next group's index clamped into range, a
// division's zero check kept in a register and reported after the loop), so
// the compiler's load counters are exact: the loop waits only for the next
// group's loads, never for its own stores to complete.
template <bool REDUCE, int NV, int NO>
__global__ __launch_bounds__(kBlock) void map_program_vec(MapArgsK a) {
    const size_t t = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    const int rq = a.p.reduce_reg;
    const auto seq = std::make_index_sequence<4>{};
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
    if (t < a.n4) fetch(t);
    for (size_t g = t; g < a.n4; g += stride) {
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
            const int k = a.vreg[j];
            r0[k] = nx[j][0];
            r1[k] = nx[j][1];
            r2[k] = nx[j][2];
            r3[k] = nx[j][3];
        }
        const size_t gn = g + stride < a.n4 ? g + stride : a.n4 - 1;  // in range: the same loads every step
        fetch(gn);
        run_program(a, 4 * g, zmin, seq, r0, r1, r2, r3);
#pragma unroll
        for (int o = 0; o < NO; ++o) {
            const int q = a.p.output_regs[o];
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
        const auto one = std::make_index_sequence<1>{};
        load_inputs(a, i, false, one, r0);
        run_program(a, i, zmin, one, r0);
        store_outputs(a, i, false, one, r0);
        if (REDUCE) acc += (double)r0[rq];
    }
    if (zmin != ~0ull) atomicMin(a.zero_index, zmin);
    if (REDUCE) {
        const double s = block_sum(acc);
        if (threadIdx.x == 0) a.partial[blockIdx.x] = s;
    }
}

// Any alignment and counts: the same evaluation with element loads.
template <bool REDUCE>
__global__ __launch_bounds__(kBlock) void map_program_kernel(MapArgsK a) {
    const size_t t = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
    const size_t stride = static_cast<size_t>(gridDim.x) * kBlock;
    const int rq = a.p.reduce_reg;
    const auto seq = std::make_index_sequence<4>{};
    double acc = 0.0;
    unsigned long long zmin = ~0ull;
    for (size_t g = t; g < a.n4; g += stride) {
        float r0[kMapRegs], r1[kMapRegs], r2[kMapRegs], r3[kMapRegs];
        load_inputs(a, 4 * g, a.vec, seq, r0, r1, r2, r3);
        run_program(a, 4 * g, zmin, seq, r0, r1, r2, r3);
        store_outputs(a, 4 * g, a.vec, seq, r0, r1, r2, r3);
        if (REDUCE) acc += (double)r0[rq] + (double)r1[rq] + (double)r2[rq] + (double)r3[rq];
    }
    for (size_t i = 4 * a.n4 + t; i < a.n; i += stride) {
        float r0[kMapRegs];
        const auto one = std::make_index_sequence<1>{};
        load_inputs(a, i, false, one, r0);
        run_program(a, i, zmin, one, r0);
        store_outputs(a, i, false, one, r0);
        if (REDUCE) acc += (double)r0[rq];
    }
    if (zmin != ~0ull) atomicMin(a.zero_index, zmin);
    if (REDUCE) {
        const double s = block_sum(acc);
        if (threadIdx.x == 0) a.partial[blockIdx.x] = s;
    }
}

// The launch: the counted form for aligned operands, the general one else.
template <bool REDUCE, int NV, int NO>
static void launch_vec_as(const MapArgsK &a, dim3 grid, hipStream_t s) {
    launch(map_program_vec<REDUCE, NV, NO>, grid, dim3(kBlock), 0, s, a);
}

template <bool REDUCE, int NV>
static void launch_vec_no(const MapArgsK &a, int no, dim3 grid, hipStream_t s) {
    switch (no) {
        case 0: launch_vec_as<REDUCE, NV, 0>(a, grid, s); break;
        case 1: launch_vec_as<REDUCE, NV, 1>(a, grid, s); break;
        case 2: launch_vec_as<REDUCE, NV, 2>(a, grid, s); break;
        case 3: launch_vec_as<REDUCE, NV, 3>(a, grid, s); break;
        default: launch_vec_as<REDUCE, NV, 4>(a, grid, s); break;
    }
}

template <bool REDUCE>
static void launch_map(const MapArgsK &a, int nv, dim3 grid, hipStream_t s) {
    if (!a.vec) {
        launch(map_program_kernel<REDUCE>, grid, dim3(kBlock), 0, s, a);
        return;
    }
    const int no = static_cast<int>(a.p.n_outputs);
    switch (nv) {
        case 0: launch_vec_no<REDUCE, 0>(a, no, grid, s); break;
        case 1: launch_vec_no<REDUCE, 1>(a, no, grid, s); break;
        case 2: launch_vec_no<REDUCE, 2>(a, no, grid, s); break;
        case 3: launch_vec_no<REDUCE, 3>(a, no, grid, s); break;
        case 4: launch_vec_no<REDUCE, 4>(a, no, grid, s); break;
        default: launch_vec_no<REDUCE, 5>(a, no, grid, s); break;
    }
}

}  // namespace tship

using namespace tship;

extern "C" size_t ts_hip_map_workspace_floats(size_t n) { return 2 * sum_blocks(n); }

extern "C" int ts_hip_map(const ts_hip_map_program *prog, size_t n, size_t tail_start, size_t zero_check_start,
                          unsigned long long *zero_index, float *sum_out, int mean, float *workspace,
                          size_t workspace_floats, void *stream) {
    if (!prog) return TS_HIP_EINVAL;
    const ts_hip_map_program &p = *prog;
    if (p.n_inputs > kMapIn || p.n_ops > kMapOps || p.n_outputs > kMapOut) return TS_HIP_EINVAL;
    const bool reduce = sum_out != nullptr;
    auto holds_value = [&](int r) {  // an input's register or a computed op's
        return (r >= 0 && r < static_cast<int>(p.n_inputs)) || (r >= kMapIn && r < kMapIn + static_cast<int>(p.n_ops));
    };
    if (reduce && !holds_value(p.reduce_reg)) return TS_HIP_EINVAL;
    if (!reduce && p.n_outputs == 0) return TS_HIP_EINVAL;
    // every register read must be an input or an earlier op's value
    for (uint32_t k = 0; k < p.n_ops; ++k) {
        const ts_hip_map_op &op = p.ops[k];
        auto ok = [&](int r) { return r < static_cast<int>(p.n_inputs) || (r >= kMapIn && r < kMapIn + static_cast<int>(k)); };
        if (!ok(op.a) || !ok(op.b) || op.code > TS_HIP_MAP_SQUARE) return TS_HIP_EINVAL;
    }
    for (uint32_t o = 0; o < p.n_outputs; ++o) {
        const int q = p.output_regs[o];
        if (!p.outputs[o] || !holds_value(q)) return TS_HIP_EINVAL;
    }
    // per-element inputs: neither scalar nor constant
    const uint32_t one_value = p.scalar_inputs | p.const_inputs;
    bool vec = true;
    for (uint32_t k = 0; k < p.n_inputs; ++k) {
        if (!(p.const_inputs & (1u << k)) && !p.inputs[k]) return TS_HIP_EINVAL;
        if (!(one_value & (1u << k))) vec = vec && aligned16(p.inputs[k]);
    }
    for (uint32_t o = 0; o < p.n_outputs; ++o) vec = vec && aligned16(p.outputs[o]);
    hipStream_t s = as_stream(stream);
    if (n == 0) return reduce ? ts_hip_fill(sum_out, 0.0f, 1, stream) : TS_HIP_OK;
    MapArgsK a{};
    a.p = p;
    a.n = n;
    // the group structure is n / 4 whatever the alignment (loads and stores
    // fall back to single elements), so a fused sum keeps ts_hip_sum's order
    a.n4 = n / 4;
    a.tail_start = tail_start;
    a.check_start = zero_check_start;
    a.zero_index = zero_index;
    a.vec = vec;
    int nv = 0;
    for (uint32_t k = 0; k < p.n_inputs; ++k)
        if (!(one_value & (1u << k))) {
            a.vin[nv] = p.inputs[k];
            a.vreg[nv] = static_cast<int>(k);
            ++nv;
        }
    if (!reduce) {
        const size_t rest = n - 4 * a.n4;
        const size_t threads = a.n4 > rest ? a.n4 : rest;
        // a group per thread up to 16 workgroups per CU, then several per
        // thread (the prefetch overlaps them): a small program is one short
        // round of loads, not a chain of them
        const unsigned blocks = grid_for(threads, 1);
        launch_map<false>(a, nv, dim3(blocks), s);
        return launch_status();
    }
    const size_t blocks = sum_blocks(n);
    if (!workspace || workspace_floats < 2 * blocks) return TS_HIP_EWORKSPACE;
    if ((reinterpret_cast<uintptr_t>(workspace) & 7u) != 0) return TS_HIP_EINVAL;
    a.partial = reinterpret_cast<double *>(workspace);
    launch_map<true>(a, nv, dim3(static_cast<unsigned>(blocks)), s);
    const int st = launch_status();
    if (st != TS_HIP_OK) return st;
    return launch_sum_final(a.partial, blocks, n, sum_out, mean != 0, s);
}
