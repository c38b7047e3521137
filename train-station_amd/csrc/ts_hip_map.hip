// Fused elementwise programs: one pass evaluates a short list of the
// elementwise operations of the gradtrack step (the same formulas, in the same
// fp32 order, as their separate kernels in ts_hip_elementwise.hip) over up to
// five inputs and stores up to four of the values, optionally adding one of
// them up as ts_hip_sum / ts_hip_mean would.  The host records a chain of
// elementwise ops as such a program and runs it when a value is first needed,
// so intermediates nobody reads are never written and shared inputs are read
// once.
//
// Two ways to run a program, with the same bits (the same fp32 operations in
// the same order over the same loop, ts_hip_map_body.h):
// * the interpreter below: r[0 .. n_inputs) start with the inputs; op k
//   writes r[d_k], the register the host assigned it.  Each thread evaluates
//   four consecutive elements at once; the register file is four arrays
//   indexed by uniform (scalar) indices, which the compiler keeps in VGPRs
//   (indexed moves), and each op's code selects its formula by a uniform
//   branch.  An indexed array takes a power-of-two register tuple: 16
//   registers keep the file at 4 x 16 VGPRs and the kernel at 4 waves per
//   SIMD.
// * a compiled program: for a program shape (ops, registers, inputs read per
//   element, stored values, reduction) met again, the same loop with the ops
//   written out as straight-line code is compiled at run time (hipRTC) and
//   cached for the process; its registers are plain registers, and no op is
//   dispatched per element (ts_hip_map_jit_mode).
#include <hip/hiprtc.h>

#include <atomic>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "ts_hip_internal.h"
#include "ts_hip_map_body.h"

namespace tship {

// The interpreter: every field of the program read at run time.
struct Interp {
    __device__ static int in_reg(const MapArgsK &a, int j) { return a.vreg[j]; }
    __device__ static int out_reg(const MapArgsK &a, int o) { return a.p.output_regs[o]; }
    __device__ static int red_reg(const MapArgsK &a) { return a.p.reduce_reg; }

    // The register file of W consecutive elements: one local array per
    // element, passed as a parameter pack so every element's array is named
    // at compile time (a pointer chosen at run time, a 2-D array or arrays
    // wrapped in one struct go to scratch; separate arrays with uniform
    // indices stay in VGPRs, read and written with indexed moves).  C... are
    // the elements' offsets.
    template <unsigned long... C, class... R>
    __device__ static __forceinline__ void run(const MapArgsK &a, size_t i0, unsigned long long &zmin, Seq<C...>,
                                               R &...r) {
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
                case TS_HIP_MAP_DIV: ((v[C] = x[C] / y[C]), ...); break;
                case kMapDivChecked: {
                    // the first zero divisor this thread sees (reported once, after its loop)
                    auto check = [&](float d, size_t i) {
                        if (i >= a.check_start && d == 0.0f && i < zmin) zmin = i;
                    };
                    (check(y[C], i0 + C), ...);
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
            const int d = op.d;
            ((r[d] = v[C]), ...);
        }
    }
};

template <bool REDUCE, int NV, int NO>
__global__ __launch_bounds__(kBlock) void map_program_vec(MapArgsK a) {
    map_vec_body<REDUCE, NV, NO, Interp>(a);
}

template <bool REDUCE>
__global__ __launch_bounds__(kBlock) void map_program_kernel(MapArgsK a) {
    map_any_body<REDUCE, Interp>(a);
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

// ---- programs compiled at run time ----------------------------------------------

// The headers the compiled source includes, as text (generated from the files
// at build time), and the two C headers hipRTC lacks, as aliases of its own
// fixed-width types.
#include "ts_hip_jit_headers.inc"

constexpr char kRtcStdint[] =
    "#pragma once\n"
    "typedef __hip_internal::uint8_t uint8_t;\ntypedef __hip_internal::uint16_t uint16_t;\n"
    "typedef __hip_internal::uint32_t uint32_t;\ntypedef __hip_internal::uint64_t uint64_t;\n"
    "typedef __hip_internal::int8_t int8_t;\ntypedef __hip_internal::int16_t int16_t;\n"
    "typedef __hip_internal::int32_t int32_t;\ntypedef __hip_internal::int64_t int64_t;\n"
    "typedef unsigned long uintptr_t;\n";
constexpr char kRtcStddef[] = "#pragma once\n";

// The straight-line form of one op, for W elements: the interpreter's formula
// of its code, with the registers and the op's index fixed.
static std::string jit_op(const ts_hip_map_op &op, int k) {
    const std::string a = std::to_string(op.a), b = std::to_string(op.b), d = std::to_string(op.d);
    const std::string imm = "a.p.ops[" + std::to_string(k) + "].imm";
    std::string v;
    switch (op.code) {
        case TS_HIP_MAP_ADD: v = "((v[C] = x[C] + y[C]), ...);"; break;
        case TS_HIP_MAP_SUB: v = "((v[C] = x[C] - y[C]), ...);"; break;
        case TS_HIP_MAP_MUL: v = "((v[C] = x[C] * y[C]), ...);"; break;
        case TS_HIP_MAP_DIV: v = "((v[C] = x[C] / y[C]), ...);"; break;
        case kMapDivChecked:
            v = "auto check = [&](float q, size_t i) { if (i >= a.check_start && q == 0.0f && i < zmin) zmin = i; };\n"
                "        (check(y[C], i0 + C), ...);\n        ((v[C] = x[C] / y[C]), ...);";
            break;
        case TS_HIP_MAP_NEG: v = "((v[C] = (i0 + C < a.tail_start) ? 0.0f - x[C] : -x[C]), ...);"; break;
        case TS_HIP_MAP_RELU: v = "((v[C] = x[C] > 0.0f ? x[C] : 0.0f), ...);"; break;
        case TS_HIP_MAP_RELU_BWD: v = "((v[C] = x[C] > 0.0f ? y[C] : 0.0f), ...);"; break;
        case TS_HIP_MAP_ADD_S: v = "((v[C] = x[C] + " + imm + "), ...);"; break;
        case TS_HIP_MAP_SUB_S: v = "((v[C] = x[C] - " + imm + "), ...);"; break;
        case TS_HIP_MAP_MUL_S: v = "((v[C] = x[C] * " + imm + "), ...);"; break;
        case TS_HIP_MAP_DIV_S: v = "((v[C] = x[C] / " + imm + "), ...);"; break;
        default: v = "((v[C] = x[C] * x[C]), ...);"; break;  // TS_HIP_MAP_SQUARE
    }
    return "    {  // op " + std::to_string(k) + "\n        const float x[W] = {r[" + a + "]...};\n" +
           "        const float y[W] = {r[" + b + "]...};\n        float v[W];\n        " + v +
           "\n        ((r[" + d + "] = v[C]), ...);\n    }\n";
}

// A register table as a constant expression of its index: j == 0 ? r0 : ...
static std::string jit_table(const int *regs, int count) {
    std::string s;
    for (int i = 0; i + 1 < count; ++i) s += "j == " + std::to_string(i) + " ? " + std::to_string(regs[i]) + " : ";
    return s + std::to_string(count > 0 ? regs[count - 1] : 0);
}

// The source of the compiled form of a's program (aligned operands; NV
// inputs read per element, NO stored values, a reduction or not).
static std::string jit_source(const MapArgsK &a, bool reduce, int nv, int no) {
    int outs[kMapOut];
    for (int o = 0; o < kMapOut; ++o) outs[o] = o < no ? a.p.output_regs[o] : 0;
    std::string s =
        "#include \"ts_hip_map_body.h\"\n"
        "namespace tship {\n"
        "struct Compiled {\n"
        "    __device__ static constexpr int in_reg(const MapArgsK &, int j) { return " + jit_table(a.vreg, nv) + "; }\n"
        "    __device__ static constexpr int out_reg(const MapArgsK &, int j) { return " + jit_table(outs, no) + "; }\n"
        "    __device__ static constexpr int red_reg(const MapArgsK &) { return " +
        std::to_string(reduce ? a.p.reduce_reg : 0) + "; }\n"
        "    template <unsigned long... C, class... R>\n"
        "    __device__ static __forceinline__ void run(const MapArgsK &a, size_t i0, unsigned long long &zmin,\n"
        "                                               Seq<C...>, R &...r) {\n"
        "    constexpr int W = sizeof...(C);\n";
    for (uint32_t k = 0; k < a.p.n_ops; ++k) s += jit_op(a.p.ops[k], static_cast<int>(k));
    s += "    (void)a; (void)i0; (void)zmin;\n    }\n};\n}  // namespace tship\n"
         "extern \"C\" __global__ __launch_bounds__(256) void ts_hip_map_compiled(tship::MapArgsK a) {\n"
         "    tship::map_vec_body<" + std::string(reduce ? "true" : "false") + ", " + std::to_string(nv) + ", " +
         std::to_string(no) + ", tship::Compiled>(a);\n}\n";
    return s;
}

// hipRTC options: the library's own numerics (no contraction, IEEE division
// and square root, denormals kept, no packed fp32 instructions).
static const char *const kRtcOptions[] = {"--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
                                          "-fhip-fp32-correctly-rounded-divide-sqrt",
                                          "-fno-gpu-flush-denormals-to-zero", "-Xclang", "-target-feature",
                                          "-Xclang", "-packed-fp32-ops"};

// A compiled program's code object, or empty with the compiler's log in *log.
static std::vector<char> jit_compile(const std::string &src, std::string *log) {
    const char *headers[] = {kJitHeaderTsHip, kJitHeaderDeviceCommon, kJitHeaderMapBody, kRtcStdint, kRtcStddef};
    const char *names[] = {"ts_hip.h", "ts_hip_device_common.h", "ts_hip_map_body.h", "stdint.h", "stddef.h"};
    hiprtcProgram prog;
    std::vector<char> code;
    if (hiprtcCreateProgram(&prog, src.c_str(), "ts_hip_map_compiled.hip", 5, headers, names) != HIPRTC_SUCCESS) {
        *log = "hiprtcCreateProgram failed";
        return code;
    }
    const int nopt = static_cast<int>(sizeof(kRtcOptions) / sizeof(kRtcOptions[0]));
    if (hiprtcCompileProgram(prog, nopt, kRtcOptions) == HIPRTC_SUCCESS) {
        size_t size = 0;
        if (hiprtcGetCodeSize(prog, &size) == HIPRTC_SUCCESS && size > 0) {
            code.resize(size);
            if (hiprtcGetCode(prog, code.data()) != HIPRTC_SUCCESS) code.clear();
        }
    } else {
        size_t size = 0;
        hiprtcGetProgramLogSize(prog, &size);
        log->assign(size, '\0');
        if (size) hiprtcGetProgramLog(prog, &(*log)[0]);
    }
    hiprtcDestroyProgram(&prog);
    return code;
}

struct JitEntry {
    int uses = 0;
    bool tried = false;
    hipModule_t module = nullptr;
    hipFunction_t function = nullptr;  // null: not compiled (yet, or it failed)
};

static std::mutex g_jit_mutex;
static std::unordered_map<std::string, JitEntry> g_jit;  // by device and program shape
static std::atomic<int> g_jit_mode{1};
static std::atomic<size_t> g_jit_compiled{0}, g_jit_failed{0};
static std::string g_jit_log;  // the last failure's compiler log

// The program shape the compiled form depends on: everything but the
// pointers, the constants' values and the immediates (read at run time).
static std::string jit_key(int device, const MapArgsK &a, bool reduce, int nv, int no) {
    std::string k;
    auto put = [&](unsigned v) { k.push_back(static_cast<char>(v & 0xffu)); };
    put(static_cast<unsigned>(device));
    put(reduce);
    put(static_cast<unsigned>(nv));
    put(static_cast<unsigned>(no));
    put(a.p.n_inputs);
    put(a.p.scalar_inputs);
    put(a.p.const_inputs);
    put(static_cast<unsigned>(reduce ? a.p.reduce_reg : 0));
    for (int j = 0; j < nv; ++j) put(static_cast<unsigned>(a.vreg[j]));
    for (int o = 0; o < no; ++o) put(a.p.output_regs[o]);
    for (uint32_t i = 0; i < a.p.n_ops; ++i) {
        put(a.p.ops[i].code);
        put(a.p.ops[i].a);
        put(a.p.ops[i].b);
        put(a.p.ops[i].d);
    }
    return k;
}

// The compiled kernel for a's program, compiling it on its second use (mode
// 1) or first (mode 2); null: run the interpreter.
static hipFunction_t jit_function(const MapArgsK &a, bool reduce, int nv, int no) {
    const int mode = g_jit_mode.load(std::memory_order_relaxed);
    if (mode == 0 || !a.vec) return nullptr;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lock(g_jit_mutex);
    JitEntry &c = g_jit[jit_key(device, a, reduce, nv, no)];
    ++c.uses;
    if (!c.tried && c.uses >= (mode == 2 ? 1 : 2)) {
        c.tried = true;
        std::string log;
        const std::vector<char> code = jit_compile(jit_source(a, reduce, nv, no), &log);
        if (!code.empty() && hipModuleLoadData(&c.module, code.data()) == hipSuccess &&
            hipModuleGetFunction(&c.function, c.module, "ts_hip_map_compiled") == hipSuccess) {
            g_jit_compiled.fetch_add(1);
        } else {
            (void)hipGetLastError();
            c.function = nullptr;
            g_jit_failed.fetch_add(1);
            g_jit_log = log.empty() ? "code object load failed" : log;
        }
    }
    return c.function;
}

// The program is well formed: counts within the limits, known op codes, every
// register read written first (by the inputs, or by an earlier op), something
// stored or summed, and every stored or summed register written.
static bool program_ok(const ts_hip_map_program &p, bool reduce) {
    if (p.n_inputs > kMapIn || p.n_ops > kMapOps || p.n_outputs > kMapOut) return false;
    uint32_t written = (1u << p.n_inputs) - 1u;
    auto holds_value = [&](int r) { return r >= 0 && r < kMapRegs && ((written >> r) & 1u); };
    for (uint32_t k = 0; k < p.n_ops; ++k) {
        const ts_hip_map_op &op = p.ops[k];
        if (!holds_value(op.a) || !holds_value(op.b) || op.d >= kMapRegs || op.code > TS_HIP_MAP_SQUARE) return false;
        written |= 1u << op.d;
    }
    if (reduce ? !holds_value(p.reduce_reg) : p.n_outputs == 0) return false;
    for (uint32_t o = 0; o < p.n_outputs; ++o)
        if (!holds_value(p.output_regs[o])) return false;
    return true;
}

}  // namespace tship

using namespace tship;

extern "C" int ts_hip_map_jit_mode(int mode) {
    if (mode < 0 || mode > 2) return -1;
    return g_jit_mode.exchange(mode);
}

extern "C" int ts_hip_map_jit_stats(size_t *compiled, size_t *failed) {
    if (compiled) *compiled = g_jit_compiled.load();
    if (failed) *failed = g_jit_failed.load();
    return TS_HIP_OK;
}

extern "C" const char *ts_hip_map_jit_log(void) {
    std::lock_guard<std::mutex> lock(g_jit_mutex);
    return g_jit_log.c_str();
}

extern "C" size_t ts_hip_map_jit_source(const ts_hip_map_program *prog, int reduce, char *buf, size_t cap) {
    if (!prog || !program_ok(*prog, reduce != 0)) return 0;
    MapArgsK a{};
    a.p = *prog;
    for (uint32_t k = 0; k < a.p.n_ops; ++k)
        if (a.p.ops[k].code == TS_HIP_MAP_DIV && (a.p.ops[k].flags & TS_HIP_MAP_CHECKED)) a.p.ops[k].code = kMapDivChecked;
    int nv = 0;
    for (uint32_t k = 0; k < a.p.n_inputs; ++k)
        if (!((a.p.scalar_inputs | a.p.const_inputs) & (1u << k))) a.vreg[nv++] = static_cast<int>(k);
    const std::string s = jit_source(a, reduce != 0, nv, static_cast<int>(a.p.n_outputs));
    if (buf && cap) {
        const size_t m = s.size() < cap - 1 ? s.size() : cap - 1;
        s.copy(buf, m);
        buf[m] = '\0';
    }
    return s.size() + 1;
}

extern "C" size_t ts_hip_map_workspace_floats(size_t n) { return 2 * sum_blocks(n); }

extern "C" int ts_hip_map(const ts_hip_map_program *prog, size_t n, size_t tail_start, size_t zero_check_start,
                          unsigned long long *zero_index, float *sum_out, int mean, float *workspace,
                          size_t workspace_floats, void *stream) {
    if (!prog || !program_ok(*prog, sum_out != nullptr)) return TS_HIP_EINVAL;
    const ts_hip_map_program &p = *prog;
    const bool reduce = sum_out != nullptr;
    for (uint32_t o = 0; o < p.n_outputs; ++o)
        if (!p.outputs[o]) return TS_HIP_EINVAL;
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
    for (uint32_t k = 0; k < p.n_ops; ++k)
        if (p.ops[k].code == TS_HIP_MAP_DIV && (p.ops[k].flags & TS_HIP_MAP_CHECKED) && zero_index)
            a.p.ops[k].code = kMapDivChecked;
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
    // the sum's partition with or without a sum: a group per thread up to
    // 2048 workgroups, then four per thread in short workgroups (a fixed grid
    // striding over the input ends with its slowest workgroup)
    const unsigned blocks = static_cast<unsigned>(sum_blocks(n));
    a.run = sum_run(n);
    if (reduce) {
        if (!workspace || workspace_floats < 2 * static_cast<size_t>(blocks)) return TS_HIP_EWORKSPACE;
        if ((reinterpret_cast<uintptr_t>(workspace) & 7u) != 0) return TS_HIP_EINVAL;
        a.partial = reinterpret_cast<double *>(workspace);
    }
    if (hipFunction_t f = jit_function(a, reduce, nv, static_cast<int>(p.n_outputs))) {
        void *params[] = {&a};
        const hipError_t e = launch_module(f, blocks, kBlock, s, params);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return static_cast<int>(e);
        }
    } else if (reduce) {
        launch_map<true>(a, nv, dim3(blocks), s);
    } else {
        launch_map<false>(a, nv, dim3(blocks), s);
    }
    const int st = launch_status();
    if (st != TS_HIP_OK || !reduce) return st;
    return launch_sum_final(a.partial, blocks, n, sum_out, mean != 0, s);
}
