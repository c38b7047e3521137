// Bandwidth-bound elementwise kernels of the gradtrack step, forward and
// backward.  Every kernel is a grid-stride loop over float4 (dwordx4) groups
// with a scalar tail; the per-element arithmetic is the reference's, in its
// order, with no contraction (-ffp-contract=off) and IEEE division/sqrt, so
// results are bit-identical to train-station's CPU path.
#include "ts_hip_internal.h"
#include "ts_hip_libm.h"

namespace tship {

// One element of an n-ary map.  `i` is the flat element index, needed by the
// operations whose formula depends on position (negate's tail rule, the
// division-by-zero check).
struct AddOp { static constexpr int NIN = 2, NOUT = 1;
    __device__ void operator()(size_t, const float *x, float *y) const { y[0] = x[0] + x[1]; } };
struct SubOp { static constexpr int NIN = 2, NOUT = 1;
    __device__ void operator()(size_t, const float *x, float *y) const { y[0] = x[0] - x[1]; } };
struct MulOp { static constexpr int NIN = 2, NOUT = 1;
    __device__ void operator()(size_t, const float *x, float *y) const { y[0] = x[0] * x[1]; } };

struct DivOp {
    static constexpr int NIN = 2, NOUT = 1;
    size_t check_start;
    unsigned long long *zero_index;
    __device__ void operator()(size_t i, const float *x, float *y) const {
        if (zero_index && i >= check_start && x[1] == 0.0f) atomicMin(zero_index, (unsigned long long)i);
        y[0] = x[0] / x[1];
    }
};

struct AddScalarOp { static constexpr int NIN = 1, NOUT = 1; float s;
    __device__ void operator()(size_t, const float *x, float *y) const { y[0] = x[0] + s; } };
struct SubScalarOp { static constexpr int NIN = 1, NOUT = 1; float s;
    __device__ void operator()(size_t, const float *x, float *y) const { y[0] = x[0] - s; } };
struct MulScalarOp { static constexpr int NIN = 1, NOUT = 1; float s;
    __device__ void operator()(size_t, const float *x, float *y) const { y[0] = x[0] * s; } };
struct DivScalarOp { static constexpr int NIN = 1, NOUT = 1; float s;
    __device__ void operator()(size_t, const float *x, float *y) const { y[0] = x[0] / s; } };

// core/utils.rs:847-870: 0 - x on the AVX2 body, -x on the scalar tail.
struct NegOp {
    static constexpr int NIN = 1, NOUT = 1;
    size_t tail_start;
    __device__ void operator()(size_t i, const float *x, float *y) const {
        y[0] = (i < tail_start) ? 0.0f - x[0] : -x[0];
    }
};

struct ReluOp { static constexpr int NIN = 1, NOUT = 1;
    __device__ void operator()(size_t, const float *x, float *y) const {
        y[0] = x[0] > 0.0f ? x[0] : 0.0f; } };

struct Pow2Op { static constexpr int NIN = 1, NOUT = 1;
    __device__ void operator()(size_t, const float *x, float *y) const { y[0] = x[0] * x[0]; } };
struct PowHalfOp { static constexpr int NIN = 1, NOUT = 1;
    __device__ void operator()(size_t, const float *x, float *y) const { y[0] = sqrtf(x[0]); } };
struct PowOp { static constexpr int NIN = 1, NOUT = 1; float e;
    __device__ void operator()(size_t, const float *x, float *y) const { y[0] = powf(x[0], e); } };

struct FillOp { static constexpr int NIN = 0, NOUT = 1; float v;
    __device__ void operator()(size_t, const float *, float *y) const { y[0] = v; } };

// The fill value is read from device memory once per thread.
struct FillFromOp {
    static constexpr int NIN = 0, NOUT = 1;
    const float *src;
    float mult;
    int use_mult;
    __device__ void operator()(size_t, const float *, float *y) const {
        y[0] = use_mult ? mult * src[0] : src[0];
    }
};

// ---- activations (tensor/ops/{exp,log,sqrt,tanh,sigmoid,leaky_relu}.rs) ----
// The reference calls f32::exp / ln / tanh, i.e. the host libm's expf / logf /
// tanhf: glibc's evaluations, restated in ts_hip_libm.h, so every value has
// the host libm's bits.
struct ExpOp { static constexpr int NIN = 1, NOUT = 1;
    __device__ void operator()(size_t, const float *x, float *y) const { y[0] = libm::expf_glibc(x[0]); } };
struct LogOp { static constexpr int NIN = 1, NOUT = 1;
    __device__ void operator()(size_t, const float *x, float *y) const { y[0] = libm::logf_glibc(x[0]); } };
// sqrt.rs: _mm256_sqrt_ps / f32::sqrt, both correctly rounded, as sqrtf is here
struct SqrtOp { static constexpr int NIN = 1, NOUT = 1;
    __device__ void operator()(size_t, const float *x, float *y) const { y[0] = sqrtf(x[0]); } };
struct TanhOp { static constexpr int NIN = 1, NOUT = 1;
    __device__ void operator()(size_t, const float *x, float *y) const { y[0] = libm::tanhf_fdlibm(x[0]); } };
// sigmoid.rs:9-21, the two-branch stable form
struct SigmoidOp { static constexpr int NIN = 1, NOUT = 1;
    __device__ void operator()(size_t, const float *x, float *y) const {
        const float v = x[0];
        if (v >= 0.0f) {
            const float z = libm::expf_glibc(-v);
            y[0] = 1.0f / (1.0f + z);
        } else {
            const float z = libm::expf_glibc(v);
            y[0] = z / (1.0f + z);
        }
    } };
// leaky_relu.rs: x > 0 ? x : slope * x (the AVX2 blend and the scalar tail agree)
struct LeakyReluOp { static constexpr int NIN = 1, NOUT = 1; float slope;
    __device__ void operator()(size_t, const float *x, float *y) const {
        y[0] = x[0] > 0.0f ? x[0] : slope * x[0]; } };

// grad_fn/ops/log.rs: inv = 1 / x, then go * inv.  Inputs (x, go).
struct LogBwdOp { static constexpr int NIN = 2, NOUT = 1;
    __device__ void operator()(size_t, const float *x, float *y) const {
        const float inv = 1.0f / x[0];
        y[0] = x[1] * inv; } };
// grad_fn/ops/sqrt.rs: inv = 1 / s, scaled = inv * 0.5, go * scaled.  Inputs (s, go).
struct SqrtBwdOp { static constexpr int NIN = 2, NOUT = 1;
    __device__ void operator()(size_t, const float *x, float *y) const {
        const float inv = 1.0f / x[0];
        const float scaled = inv * 0.5f;
        y[0] = x[1] * scaled; } };
// grad_fn/ops/tanh.rs: go * (1 - t*t).  Inputs (t, go).
struct TanhBwdOp { static constexpr int NIN = 2, NOUT = 1;
    __device__ void operator()(size_t, const float *x, float *y) const {
        const float t = x[0];
        y[0] = x[1] * (1.0f - t * t); } };
// grad_fn/ops/sigmoid.rs: (go * s) * (1 - s).  Inputs (s, go).
struct SigmoidBwdOp { static constexpr int NIN = 2, NOUT = 1;
    __device__ void operator()(size_t, const float *x, float *y) const {
        const float s = x[0];
        y[0] = x[1] * s * (1.0f - s); } };
// grad_fn/ops/leaky_relu.rs: x > 0 ? go : slope * go.  Inputs (x, go).
struct LeakyReluBwdOp { static constexpr int NIN = 2, NOUT = 1; float slope;
    __device__ void operator()(size_t, const float *x, float *y) const {
        y[0] = x[0] > 0.0f ? x[1] : slope * x[1]; } };

// grad_fn/ops/relu.rs:4-17
struct ReluBwdOp { static constexpr int NIN = 2, NOUT = 1;
    __device__ void operator()(size_t, const float *x, float *y) const {
        y[0] = x[0] > 0.0f ? x[1] : 0.0f; } };

// grad_fn/ops/pow.rs:5-27 (powf(x, 1) == x, so e == 2 is go * (2 * x))
struct PowBwdOp {
    static constexpr int NIN = 2, NOUT = 1;
    float e;
    __device__ void operator()(size_t, const float *x, float *y) const {
        float local;
        if (e == 0.0f) local = 0.0f;
        else if (e == 2.0f) local = e * x[0];
        else local = e * powf(x[0], e - 1.0f);
        y[0] = x[1] * local;
    }
};

// grad_fn/ops/mul.rs:4-49: inputs (go, a, b) -> (go*b, go*a)
struct MulBwdOp { static constexpr int NIN = 3, NOUT = 2;
    __device__ void operator()(size_t, const float *x, float *y) const {
        y[0] = x[0] * x[2];
        y[1] = x[0] * x[1];
    } };

// grad_fn/ops/div.rs:4-49: inputs (go, a, b) -> (go/b, neg((go*a)/(b*b)))
struct DivBwdOp {
    static constexpr int NIN = 3, NOUT = 2;
    size_t tail_start, check_start;
    unsigned long long *zero_index;
    __device__ void operator()(size_t i, const float *x, float *y) const {
        const float go = x[0], a = x[1], b = x[2];
        const float bb = b * b;
        if (zero_index && i >= check_start && (b == 0.0f || bb == 0.0f))
            atomicMin(zero_index, (unsigned long long)i);
        y[0] = go / b;
        const float q = (go * a) / bb;
        y[1] = (i < tail_start) ? 0.0f - q : -q;
    }
};

struct MapArgs {
    const float *in[3];
    float *out[2];
};

// One float4 group per thread (thread t < n4 takes elements 4t .. 4t+3) and
// the scalar remainder [4*n4, n) by the first threads; n4 is 0 when any
// pointer is not 16-byte aligned, and then every element is scalar.  NT:
// vector results are written with non-temporal stores, so the output streams
// to HBM instead of displacing the inputs in L2 / MALL (measured +4% on data
// that is not cached, +30% on data that is).  The gradients that a column
// sum reads right after (ReLU and pow backward, whose outputs feed the bias
// gradient) keep ordinary stores: the sum then finds them in MALL, which
// saves more (-16% on that sum) than the store policy costs.
template <class Op, bool NT>
__global__ __launch_bounds__(kBlock) void map_kernel(MapArgs args, size_t n, size_t n4, Op op) {
    const size_t t = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (t < n4) {
        float4 xin[Op::NIN > 0 ? Op::NIN : 1];
#pragma unroll
        for (int k = 0; k < Op::NIN; ++k) xin[k] = reinterpret_cast<const float4 *>(args.in[k])[t];
        float4 yout[Op::NOUT];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float xs[Op::NIN > 0 ? Op::NIN : 1], ys[Op::NOUT];
#pragma unroll
            for (int k = 0; k < Op::NIN; ++k) xs[k] = reinterpret_cast<const float *>(&xin[k])[c];
            op(4 * t + c, xs, ys);
#pragma unroll
            for (int k = 0; k < Op::NOUT; ++k) reinterpret_cast<float *>(&yout[k])[c] = ys[k];
        }
#pragma unroll
        for (int k = 0; k < Op::NOUT; ++k) {
            if (!args.out[k]) continue;
            float4 *o = reinterpret_cast<float4 *>(args.out[k]) + t;
            if (NT) store_nt(o, yout[k]);
            else *o = yout[k];
        }
    }
    const size_t i = 4 * n4 + t;
    if (i < n) {
        float xs[Op::NIN > 0 ? Op::NIN : 1], ys[Op::NOUT];
#pragma unroll
        for (int k = 0; k < Op::NIN; ++k) xs[k] = args.in[k][i];
        op(i, xs, ys);
#pragma unroll
        for (int k = 0; k < Op::NOUT; ++k)
            if (args.out[k]) args.out[k][i] = ys[k];
    }
}

template <class Op, bool NT = true>
static int launch_map(const float *const *in, float *const *out, size_t n, Op op, void *stream) {
    if (n == 0) return TS_HIP_OK;
    MapArgs args{};
    bool vec = true, any_out = false;
    for (int k = 0; k < Op::NIN; ++k) {
        if (!in[k]) return TS_HIP_EINVAL;
        args.in[k] = in[k];
        vec = vec && aligned16(in[k]);
    }
    for (int k = 0; k < Op::NOUT; ++k) {
        args.out[k] = out[k];
        if (out[k]) { any_out = true; vec = vec && aligned16(out[k]); }
    }
    if (!any_out) return TS_HIP_EINVAL;
    const size_t n4 = vec ? n / 4 : 0;
    const size_t rest = n - 4 * n4;
    const size_t threads = n4 > rest ? n4 : rest;
    const size_t blocks = (threads + kBlock - 1) / kBlock;
    if (blocks > 0x7fffffffULL) return TS_HIP_EINVAL;
    launch((map_kernel<Op, NT>), dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0,
                       as_stream(stream), args, n, n4, op);
    return launch_status();
}

template <class Op, bool NT = true>
static int map1(const float *x, float *out, size_t n, Op op, void *stream) {
    const float *in[1] = {x};
    float *o[1] = {out};
    return launch_map<Op, NT>(in, o, n, op, stream);
}

template <class Op, bool NT = true>
static int map2(const float *a, const float *b, float *out, size_t n, Op op, void *stream) {
    const float *in[2] = {a, b};
    float *o[1] = {out};
    return launch_map<Op, NT>(in, o, n, op, stream);
}

// Row broadcast [rows,cols] op [cols]: blockIdx.x walks column groups,
// blockIdx.y strides over rows, so each thread loads its vector value(s) once.
// The reference materialises the broadcast operand and then runs the
// same-shape kernel (ops/broadcasting.rs:362-478), so element (r,c) is
// x[r][c] op v[c] (or v[c] op x[r][c]) either way.
struct RowArgs {
    int op;  // 0 add, 1 sub, 2 mul, 3 div
    bool vec_first;
    size_t rows, cols, check_start;
    unsigned long long *zero_index;
};

__device__ inline float row_op(const RowArgs &a, size_t flat, float x, float v) {
    const float l = a.vec_first ? v : x, r = a.vec_first ? x : v;
    switch (a.op) {
        case 0: return l + r;
        case 1: return l - r;
        case 2: return l * r;
        default:
            if (a.zero_index && flat >= a.check_start && r == 0.0f)
                atomicMin(a.zero_index, (unsigned long long)flat);
            return l / r;
    }
}

__global__ __launch_bounds__(kBlock) void row_broadcast_vec4(const float4 *__restrict__ x,
                                                             const float4 *__restrict__ v,
                                                             float4 *__restrict__ out, RowArgs a) {
    const size_t cols4 = a.cols / 4;
    size_t c4 = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (c4 >= cols4) return;
    const float4 b = v[c4];
    for (size_t r = blockIdx.y; r < a.rows; r += gridDim.y) {
        const size_t q = r * cols4 + c4;
        const float4 xv = x[q];
        float4 o;
        o.x = row_op(a, 4 * q + 0, xv.x, b.x);
        o.y = row_op(a, 4 * q + 1, xv.y, b.y);
        o.z = row_op(a, 4 * q + 2, xv.z, b.z);
        o.w = row_op(a, 4 * q + 3, xv.w, b.w);
        store_nt(out + q, o);
    }
}

__global__ __launch_bounds__(kBlock) void row_broadcast_scalar(const float *__restrict__ x,
                                                               const float *__restrict__ v,
                                                               float *__restrict__ out,
                                                               RowArgs a) {
    size_t c = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (c >= a.cols) return;
    const float b = v[c];
    for (size_t r = blockIdx.y; r < a.rows; r += gridDim.y) {
        const size_t q = r * a.cols + c;
        out[q] = row_op(a, q, x[q], b);
    }
}

}  // namespace tship

using namespace tship;

extern "C" {

int ts_hip_add(const float *a, const float *b, float *out, size_t n, void *stream) {
    return map2(a, b, out, n, AddOp{}, stream);
}
int ts_hip_sub(const float *a, const float *b, float *out, size_t n, void *stream) {
    return map2(a, b, out, n, SubOp{}, stream);
}
int ts_hip_mul(const float *a, const float *b, float *out, size_t n, void *stream) {
    return map2(a, b, out, n, MulOp{}, stream);
}
int ts_hip_div(const float *a, const float *b, float *out, size_t n, size_t zero_check_start,
               unsigned long long *zero_index, void *stream) {
    return map2(a, b, out, n, DivOp{zero_check_start, zero_index}, stream);
}
int ts_hip_add_scalar(const float *x, float s, float *out, size_t n, void *stream) {
    return map1(x, out, n, AddScalarOp{s}, stream);
}
int ts_hip_sub_scalar(const float *x, float s, float *out, size_t n, void *stream) {
    return map1(x, out, n, SubScalarOp{s}, stream);
}
int ts_hip_mul_scalar(const float *x, float s, float *out, size_t n, void *stream) {
    return map1(x, out, n, MulScalarOp{s}, stream);
}
int ts_hip_div_scalar(const float *x, float s, float *out, size_t n, void *stream) {
    return map1(x, out, n, DivScalarOp{s}, stream);
}
int ts_hip_neg(const float *x, float *out, size_t n, size_t tail_start, void *stream) {
    return map1(x, out, n, NegOp{tail_start}, stream);
}
int ts_hip_relu(const float *x, float *out, size_t n, void *stream) {
    return map1(x, out, n, ReluOp{}, stream);
}
int ts_hip_pow_scalar(const float *x, float e, float *out, size_t n, void *stream) {
    // ordinary stores for the square: in the MSE loss the mean reads it right
    // after and then finds it in MALL
    if (e == 2.0f) return map1<Pow2Op, false>(x, out, n, Pow2Op{}, stream);
    if (e == 0.5f) return map1(x, out, n, PowHalfOp{}, stream);
    return map1(x, out, n, PowOp{e}, stream);
}
int ts_hip_fill(float *out, float value, size_t n, void *stream) {
    float *o[1] = {out};
    return launch_map<FillOp>(nullptr, o, n, FillOp{value}, stream);
}
int ts_hip_copy(const float *src, float *dst, size_t n, void *stream) {
    if (n == 0) return TS_HIP_OK;
    if (!src || !dst) return TS_HIP_EINVAL;
    if (launch_group_holding()) flush_launch_group();  // after the products a launch group holds
    return static_cast<int>(
        hipMemcpyAsync(dst, src, n * sizeof(float), hipMemcpyDeviceToDevice, as_stream(stream)));
}

int ts_hip_row_broadcast(int op, const float *x, const float *v, float *out, size_t rows,
                         size_t cols, int vec_first, size_t zero_check_start,
                         unsigned long long *zero_index, void *stream) {
    if (op < 0 || op > 3) return TS_HIP_EINVAL;
    if (rows == 0 || cols == 0) return TS_HIP_OK;
    if (!x || !v || !out) return TS_HIP_EINVAL;
    RowArgs a{op, vec_first != 0, rows, cols, zero_check_start, zero_index};
    const bool vec = (cols % 4 == 0) && aligned16(x) && aligned16(v) && aligned16(out);
    size_t ncols = vec ? cols / 4 : cols;
    unsigned gx = static_cast<unsigned>((ncols + kBlock - 1) / kBlock);
    // enough workgroups in y to cover the device several times
    size_t want = static_cast<size_t>(device_cu_count()) * 8 / gx;
    unsigned gy = static_cast<unsigned>(want < 1 ? 1 : (want > rows ? rows : want));
    if (gy > 65535) gy = 65535;
    dim3 grid(gx, gy);
    hipStream_t s = as_stream(stream);
    if (vec)
        launch(row_broadcast_vec4, grid, dim3(kBlock), 0, s,
                           reinterpret_cast<const float4 *>(x), reinterpret_cast<const float4 *>(v),
                           reinterpret_cast<float4 *>(out), a);
    else
        launch(row_broadcast_scalar, grid, dim3(kBlock), 0, s, x, v, out, a);
    return launch_status();
}

int ts_hip_bias_add(const float *x, const float *bias, float *out, size_t rows, size_t cols,
                    int bias_first, void *stream) {
    return ts_hip_row_broadcast(0, x, bias, out, rows, cols, bias_first, 0, nullptr, stream);
}

int ts_hip_fill_from_device(float *out, const float *src, float multiplier, int use_multiplier,
                            size_t n, void *stream) {
    if (!src) return TS_HIP_EINVAL;
    float *o[1] = {out};
    return launch_map<FillFromOp>(nullptr, o, n, FillFromOp{src, multiplier, use_multiplier},
                                  stream);
}

int ts_hip_exp(const float *x, float *out, size_t n, void *stream) { return map1(x, out, n, ExpOp{}, stream); }
int ts_hip_log(const float *x, float *out, size_t n, void *stream) { return map1(x, out, n, LogOp{}, stream); }
int ts_hip_sqrt(const float *x, float *out, size_t n, void *stream) { return map1(x, out, n, SqrtOp{}, stream); }
int ts_hip_tanh(const float *x, float *out, size_t n, void *stream) { return map1(x, out, n, TanhOp{}, stream); }
int ts_hip_sigmoid(const float *x, float *out, size_t n, void *stream) {
    return map1(x, out, n, SigmoidOp{}, stream);
}
int ts_hip_leaky_relu(const float *x, float negative_slope, float *out, size_t n, void *stream) {
    return map1(x, out, n, LeakyReluOp{negative_slope}, stream);
}
int ts_hip_log_backward(const float *x, const float *go, float *gi, size_t n, void *stream) {
    return map2(x, go, gi, n, LogBwdOp{}, stream);
}
int ts_hip_sqrt_backward(const float *y, const float *go, float *gi, size_t n, void *stream) {
    return map2(y, go, gi, n, SqrtBwdOp{}, stream);
}
int ts_hip_tanh_backward(const float *y, const float *go, float *gi, size_t n, void *stream) {
    return map2(y, go, gi, n, TanhBwdOp{}, stream);
}
int ts_hip_sigmoid_backward(const float *y, const float *go, float *gi, size_t n, void *stream) {
    return map2(y, go, gi, n, SigmoidBwdOp{}, stream);
}
int ts_hip_leaky_relu_backward(const float *x, const float *go, float *gi, size_t n, float negative_slope,
                               void *stream) {
    return map2(x, go, gi, n, LeakyReluBwdOp{negative_slope}, stream);
}

int ts_hip_relu_backward(const float *x, const float *go, float *gi, size_t n, void *stream) {
    return map2<ReluBwdOp, false>(x, go, gi, n, ReluBwdOp{}, stream);
}
int ts_hip_pow_backward(const float *x, const float *go, float *gi, size_t n, float e,
                        void *stream) {
    return map2<PowBwdOp, false>(x, go, gi, n, PowBwdOp{e}, stream);
}
int ts_hip_mul_backward(const float *go, const float *a, const float *b, float *ga, float *gb,
                        size_t n, void *stream) {
    const float *in[3] = {go, a, b};
    float *o[2] = {ga, gb};
    return launch_map(in, o, n, MulBwdOp{}, stream);
}
int ts_hip_div_backward(const float *go, const float *a, const float *b, float *ga, float *gb,
                        size_t n, size_t tail_start, size_t zero_check_start,
                        unsigned long long *zero_index, void *stream) {
    const float *in[3] = {go, a, b};
    float *o[2] = {ga, gb};
    return launch_map(in, o, n, DivBwdOp{tail_start, zero_check_start, zero_index}, stream);
}

}  // extern "C"
