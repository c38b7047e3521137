// Tensor construction, recorded forward ops and their backward formulas.
// Each op launches one or two kernels of ts_hip.h on the library stream; no
// op synchronises except data()/value().
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <sstream>

#include "ts_hip.h"
#include "ts_host.h"

namespace ts {

std::string dims_str(const std::vector<size_t> &d) {
    std::ostringstream os;
    os << "[";
    for (size_t i = 0; i < d.size(); ++i) os << (i ? ", " : "") << d[i];
    os << "]";
    return os.str();
}

namespace {

void *S() { return Runtime::get().stream(); }

size_t product(const std::vector<size_t> &d) {
    size_t n = 1;
    for (size_t x : d) n *= x;
    return n;
}

// Run one launcher, timed by the profiler when it is enabled.
template <class F>
void launch(KernelClass k, double work, const char *what, F &&f) {
    Profiler &P = Profiler::get();
    P.begin();
    check(f(), what);
    P.end(k, work);
}

// Reference AVX2 body/tail split: 8-wide for negate and Adam
// (core/utils.rs:856-865, adam/mod.rs:727-773), 32-wide unrolled body for the
// division zero check (ops/div.rs:356-417).
size_t tail8(size_t n) { return (n / 8) * 8; }
size_t tail32(size_t n) { return (n / 32) * 32; }

int opcode(GradFn::Kind k) {
    switch (k) {
        case GradFn::Kind::Add: return 0;
        case GradFn::Kind::Sub: return 1;
        case GradFn::Kind::Mul: return 2;
        default: return 3;
    }
}

// out = a op b (same shape)
Tensor same_shape(const float *a, const float *b, const std::vector<size_t> &dims, int op) {
    Tensor out = Tensor::new_uninit(dims);
    const size_t n = out.size();
    float *o = out.dev_mut();
    auto &rt = Runtime::get();
    launch(KernelClass::Elementwise, 12.0 * n, "elementwise", [&] {
        switch (op) {
            case 0: return ts_hip_add(a, b, o, n, S());
            case 1: return ts_hip_sub(a, b, o, n, S());
            case 2: return ts_hip_mul(a, b, o, n, S());
            default: return ts_hip_div(a, b, o, n, tail32(n), rt.zero_index(), S());
        }
    });
    return out;
}

// out[r][c] = m[r][c] op v[c]   (or v[c] op m[r][c] when vec_first)
Tensor row_bcast(const float *m, const float *v, size_t rows, size_t cols, int op, bool vec_first) {
    Tensor out = Tensor::new_uninit({rows, cols});
    const size_t n = rows * cols;
    launch(KernelClass::Elementwise, 8.0 * n + 4.0 * cols, "row broadcast", [&] {
        return ts_hip_row_broadcast(op, m, v, out.dev_mut(), rows, cols, vec_first, tail32(n),
                                    Runtime::get().zero_index(), S());
    });
    return out;
}

Tensor neg_of(const Tensor &x) {
    Tensor out = Tensor::new_uninit(x.dims());
    const size_t n = x.size();
    launch(KernelClass::Elementwise, 8.0 * n, "ts_hip_neg",
           [&] { return ts_hip_neg(x.dev(), out.dev_mut(), n, tail8(n), S()); });
    return out;
}

// grad_fn/utils.rs:23-60 for the shapes the device path records: identical
// shapes (shared, the reference clones) or the row broadcast, reduced with
// sum_dims(&[0]).
Tensor reduce_to(const Tensor &g, const std::vector<size_t> &target) {
    if (g.dims() == target) return g.alias();
    if (g.dims().size() == 2 && target.size() == 1 && target[0] == g.dims()[1]) {
        const size_t rows = g.dims()[0], cols = g.dims()[1];
        Tensor out = Tensor::new_uninit({cols});
        const size_t ws = ts_hip_sum_dim0_workspace_floats(rows, cols);
        Allocation work(ws);
        launch(KernelClass::Reduction, 4.0 * rows * cols + 4.0 * cols, "ts_hip_sum_dim0", [&] {
            return ts_hip_sum_dim0(g.dev(), rows, cols, out.dev_mut(), work.ptr, ws, S());
        });
        return out;
    }
    throw Error("reduce_gradient_to_shape: " + dims_str(g.dims()) + " -> " + dims_str(target) +
                " is not a row broadcast");
}

struct RowBroadcast {
    bool matrix_first;  // the [rows,cols] operand is the left one
    size_t rows, cols;
};

RowBroadcast row_broadcast_shape(const std::vector<size_t> &a, const std::vector<size_t> &b) {
    if (a.size() == 2 && b.size() == 1 && b[0] == a[1]) return {true, a[0], a[1]};
    if (a.size() == 1 && b.size() == 2 && a[0] == b[1]) return {false, b[0], b[1]};
    throw Error("Cannot broadcast tensor shapes " + dims_str(a) + " and " + dims_str(b) +
                ": the device path broadcasts a [N] operand over the rows of a [B, N] operand");
}

// go (full shape) op broadcast(x) where x has shape xs: x itself when xs is
// the full shape, else x broadcast over rows.
Tensor with_bcast(const Tensor &go, const SavedTensor &x, int op) {
    if (x.dims == go.dims()) return same_shape(go.dev(), x.ptr(), go.dims(), op);
    return row_bcast(go.dev(), x.ptr(), go.dims()[0], go.dims()[1], op, false);
}

}  // namespace

size_t next_tensor_id() {
    // tensor/core/mod.rs:131: one process-wide atomic counter
    static std::atomic<size_t> counter{1};
    return counter.fetch_add(1, std::memory_order_relaxed);
}

// ---- construction ---------------------------------------------------------------

Tensor Tensor::new_uninit(std::vector<size_t> dims) {
    Tensor t;
    t.size_ = product(dims);
    t.dims_ = std::move(dims);
    t.id_ = next_tensor_id();
    if (t.size_ > 0) t.alloc_ = std::make_shared<Allocation>(t.size_);
    return t;
}

Tensor Tensor::filled(std::vector<size_t> dims, float v) {
    Tensor t = new_uninit(std::move(dims));
    if (t.size_)
        launch(KernelClass::Elementwise, 4.0 * t.size_, "ts_hip_fill",
               [&] { return ts_hip_fill(t.dev_mut(), v, t.size_, S()); });
    return t;
}

Tensor Tensor::zeros(std::vector<size_t> dims) { return filled(std::move(dims), 0.0f); }
Tensor Tensor::ones(std::vector<size_t> dims) { return filled(std::move(dims), 1.0f); }

// XorShiftRng::new_from_time (random.rs:492-497) hashes the system time; any
// well-mixed 64-bit value of the clock serves (a splitmix64 finaliser of the
// nanosecond count plus a per-process counter, so two calls in the same tick
// still differ).
static uint64_t seed_from_time() {
    static std::atomic<uint64_t> calls{0};
    uint64_t z = static_cast<uint64_t>(std::chrono::system_clock::now().time_since_epoch().count()) +
                 0x9E3779B97F4A7C15ULL * (calls.fetch_add(1, std::memory_order_relaxed) + 1);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

void Tensor::fill_randn(const uint64_t *seed) {
    if (!size_) return;  // random.rs:271-273
    const uint64_t s = seed ? *seed : seed_from_time();
    launch(KernelClass::Elementwise, 4.0 * size_, "ts_hip_randn",
           [&] { return ts_hip_randn(dev_mut(), size_, s, S()); });
}

Tensor Tensor::randn(std::vector<size_t> dims, const uint64_t *seed) {
    Tensor t = new_uninit(std::move(dims));
    t.fill_randn(seed);
    return t;
}

Tensor Tensor::from_slice(const float *data, size_t len, std::vector<size_t> dims) {
    const size_t n = product(dims);
    if (len != n)  // init/data.rs:227-247 returns Err on a length mismatch
        throw Error("Data length " + std::to_string(len) + " doesn't match shape " +
                    dims_str(dims) + " (size " + std::to_string(n) + ")");
    Tensor t = new_uninit(std::move(dims));
    if (n) {
        check(ts_hip_memcpy_async(t.dev_mut(), data, n, 0, S()), "ts_hip_memcpy_async");
        check(ts_hip_stream_synchronize(S()), "ts_hip_stream_synchronize");
    }
    return t;
}

Tensor Tensor::clone() const {
    Tensor t = new_uninit(dims_);
    if (size_)
        launch(KernelClass::Elementwise, 8.0 * size_, "ts_hip_copy",
               [&] { return ts_hip_copy(dev(), t.dev_mut(), size_, S()); });
    return t;
}

Tensor Tensor::alias() const {
    Tensor t;
    t.alloc_ = alloc_;
    t.dims_ = dims_;
    t.size_ = size_;
    t.id_ = next_tensor_id();
    return t;
}

Tensor Tensor::from_saved(const SavedTensor &s) {
    Tensor t;
    t.alloc_ = s.alloc;
    t.dims_ = s.dims;
    t.size_ = product(s.dims);
    t.id_ = next_tensor_id();
    return t;
}

// ---- gradient API ------------------------------------------------------------------

void Tensor::set_requires_grad(bool r) {
    requires_grad_ = r;
    if (!r) grad_.reset();
}

void Tensor::backward(const Tensor *grad_output) { engine_backward(*this, grad_output); }

const Tensor *Tensor::grad_ref() const {
    if (grad_) return grad_.get();
    return accumulated_gradient(id_);
}

std::optional<Tensor> Tensor::grad_by_value() const {
    const Tensor *g = grad_ref();
    if (!g) return std::nullopt;
    return g->clone();  // utils.rs:525-534 returns a clone
}

void Tensor::set_grad(Tensor g) {
    if (requires_grad_) grad_ = std::make_shared<Tensor>(std::move(g));
}

void Tensor::accumulate_grad(Tensor g) {
    if (!requires_grad_) return;
    if (grad_) {
        Tensor acc = same_shape(grad_->dev(), g.dev(), grad_->dims(), 0);
        grad_ = std::make_shared<Tensor>(std::move(acc));
    } else {
        grad_ = std::make_shared<Tensor>(std::move(g));
    }
}

// ---- recorded ops ---------------------------------------------------------------------

void Tensor::record(Tensor &out, std::vector<size_t> input_ids, GradFn fn) const {
    out.requires_grad_ = true;
    register_operation(out.id_, std::move(input_ids), std::move(fn));
}

Tensor Tensor::binary(const Tensor &o, GradFn::Kind kind) const {
    const bool same = dims_ == o.dims_;
    const int op = opcode(kind);
    Tensor out;
    if (same) {
        out = same_shape(dev(), o.dev(), dims_, op);
    } else {
        RowBroadcast rb = row_broadcast_shape(dims_, o.dims_);
        const Tensor &mat = rb.matrix_first ? *this : o;
        const Tensor &vec = rb.matrix_first ? o : *this;
        out = row_bcast(mat.dev(), vec.dev(), rb.rows, rb.cols, op, !rb.matrix_first);
    }
    if ((requires_grad_ || o.requires_grad_) && is_grad_enabled()) {
        GradFn fn{kind};
        if (!same) {
            fn.has_shapes = true;
            fn.shape_a = dims_;
            fn.shape_b = o.dims_;
        }
        if (kind == GradFn::Kind::Mul || kind == GradFn::Kind::Div) fn.saved = {saved(), o.saved()};
        std::vector<size_t> ids;
        if (requires_grad_) ids.push_back(id_);
        if (o.requires_grad_) ids.push_back(o.id_);
        record(out, std::move(ids), std::move(fn));
    }
    return out;
}

Tensor Tensor::add_tensor(const Tensor &o) const { return binary(o, GradFn::Kind::Add); }
Tensor Tensor::sub_tensor(const Tensor &o) const { return binary(o, GradFn::Kind::Sub); }
Tensor Tensor::mul_tensor(const Tensor &o) const { return binary(o, GradFn::Kind::Mul); }
Tensor Tensor::div_tensor(const Tensor &o) const { return binary(o, GradFn::Kind::Div); }

Tensor Tensor::scalar_op(float s, GradFn::Kind kind) const {
    if (kind == GradFn::Kind::DivScalar && s == 0.0f)  // ops/div.rs:511-514
        throw Error("Division by zero: cannot divide tensor by zero scalar");
    Tensor out = new_uninit(dims_);
    launch(KernelClass::Elementwise, 8.0 * size_, "scalar op", [&] {
        switch (kind) {
            case GradFn::Kind::AddScalar: return ts_hip_add_scalar(dev(), s, out.dev_mut(), size_, S());
            case GradFn::Kind::SubScalar: return ts_hip_sub_scalar(dev(), s, out.dev_mut(), size_, S());
            case GradFn::Kind::MulScalar: return ts_hip_mul_scalar(dev(), s, out.dev_mut(), size_, S());
            default: return ts_hip_div_scalar(dev(), s, out.dev_mut(), size_, S());
        }
    });
    if (requires_grad_ && is_grad_enabled()) {
        GradFn fn{kind};
        fn.scalar = s;
        record(out, {id_}, std::move(fn));
    }
    return out;
}

Tensor Tensor::add_scalar(float s) const { return scalar_op(s, GradFn::Kind::AddScalar); }
Tensor Tensor::sub_scalar(float s) const { return scalar_op(s, GradFn::Kind::SubScalar); }
Tensor Tensor::mul_scalar(float s) const { return scalar_op(s, GradFn::Kind::MulScalar); }
Tensor Tensor::div_scalar(float s) const { return scalar_op(s, GradFn::Kind::DivScalar); }

Tensor Tensor::relu() const {
    Tensor out = new_uninit(dims_);
    launch(KernelClass::Elementwise, 8.0 * size_, "ts_hip_relu",
           [&] { return ts_hip_relu(dev(), out.dev_mut(), size_, S()); });
    if (requires_grad_ && is_grad_enabled()) {
        GradFn fn{GradFn::Kind::Relu};
        // The reference saves its input (ops/relu.rs:80-87); the output has
        // the same sign test (relu(x) > 0 exactly when x > 0) and keeps the
        // input buffer free to be recycled.
        fn.saved = {out.saved()};
        record(out, {id_}, std::move(fn));
    }
    return out;
}

Tensor Tensor::pow_scalar(float e) const {
    Tensor out = new_uninit(dims_);
    launch(KernelClass::Elementwise, 8.0 * size_, "ts_hip_pow_scalar",
           [&] { return ts_hip_pow_scalar(dev(), e, out.dev_mut(), size_, S()); });
    if (requires_grad_ && is_grad_enabled()) {
        GradFn fn{GradFn::Kind::PowScalar};
        fn.scalar = e;
        fn.saved = {saved()};
        record(out, {id_}, std::move(fn));
    }
    return out;
}

Tensor Tensor::matmul(const Tensor &o) const {
    if (dims_.size() != 2 || o.dims_.size() != 2)
        throw Error("matmul: the device path implements 2D @ 2D; got " + dims_str(dims_) + " @ " +
                    dims_str(o.dims_));
    const size_t m = dims_[0], k = dims_[1], n = o.dims_[1];
    if (k != o.dims_[0])  // ops/matmul/mod.rs:577-583
        throw Error("Inner dimensions must match: " + std::to_string(k) + " vs " +
                    std::to_string(o.dims_[0]));
    Tensor out = new_uninit({m, n});
    launch(KernelClass::Gemm, 2.0 * m * n * k, "ts_hip_gemm", [&] {
        return ts_hip_gemm(0, 0, m, n, k, dev(), k, o.dev(), n, out.dev_mut(), n, S());
    });
    if ((requires_grad_ || o.requires_grad_) && is_grad_enabled()) {
        GradFn fn{GradFn::Kind::MatMul};
        fn.saved = {saved(), o.saved()};
        fn.req_left = requires_grad_;
        fn.req_right = o.requires_grad_;
        record(out, {id_, o.id_}, std::move(fn));  // matmul/mod.rs:303-306: always both
    }
    return out;
}

Tensor Tensor::sum() const {
    Tensor out = new_uninit({1});
    const size_t ws = ts_hip_sum_workspace_floats(size_);
    Allocation work(ws);
    launch(KernelClass::Reduction, 4.0 * size_ + 4.0, "ts_hip_sum",
           [&] { return ts_hip_sum(dev(), size_, out.dev_mut(), work.ptr, ws, S()); });
    if (requires_grad_) {  // reductions/sum.rs:131-138 (no is_grad_enabled check)
        GradFn fn{GradFn::Kind::ReduceSum};
        fn.input_shape = dims_;
        record(out, {id_}, std::move(fn));
    }
    return out;
}

Tensor Tensor::mean() const {
    Tensor out = new_uninit({1});
    const size_t ws = ts_hip_sum_workspace_floats(size_);
    Allocation work(ws);
    launch(KernelClass::Reduction, 4.0 * size_ + 4.0, "ts_hip_mean",
           [&] { return ts_hip_mean(dev(), size_, out.dev_mut(), work.ptr, ws, S()); });
    if (requires_grad_) {  // reductions/mean.rs:97-106
        GradFn fn{GradFn::Kind::ReduceMean};
        fn.input_shape = dims_;
        fn.numel = size_;
        record(out, {id_}, std::move(fn));
    }
    return out;
}

// ---- host access ------------------------------------------------------------------------

void Tensor::copy_to_host(float *out, size_t len) const {
    if (len != size_)
        throw Error("copy_to_host: buffer of " + std::to_string(len) + " floats for a tensor of " +
                    std::to_string(size_));
    if (size_) check(ts_hip_memcpy_async(out, dev(), size_, 1, S()), "ts_hip_memcpy_async");
    Runtime::get().sync();
}

std::vector<float> Tensor::data() const {
    std::vector<float> h(size_);
    copy_to_host(h.data(), size_);
    return h;
}

float Tensor::value() const {
    if (size_ != 1)  // utils.rs:1251-1260
        throw Error("value() can only be called on tensors with exactly one element, got " +
                    std::to_string(size_));
    float v = 0.0f;
    copy_to_host(&v, 1);
    return v;
}

// ---- backward formulas ---------------------------------------------------------------------

std::vector<std::optional<Tensor>> GradFn::apply(const Tensor &go) const {
    using K = Kind;
    std::vector<std::optional<Tensor>> r;
    const size_t n = go.size();
    switch (kind) {
        case K::Add: {  // grad_fn/ops/add.rs:4-28
            if (!has_shapes) { r.emplace_back(go.alias()); r.emplace_back(go.alias()); }
            else { r.emplace_back(reduce_to(go, shape_a)); r.emplace_back(reduce_to(go, shape_b)); }
            break;
        }
        case K::Sub: {  // grad_fn/ops/sub.rs:4-33
            if (!has_shapes) { r.emplace_back(go.alias()); r.emplace_back(neg_of(go)); }
            else {
                r.emplace_back(reduce_to(go, shape_a));
                r.emplace_back(neg_of(reduce_to(go, shape_b)));
            }
            break;
        }
        case K::Mul: {  // grad_fn/ops/mul.rs:4-49
            const SavedTensor &a = saved[0], &b = saved[1];
            if (!has_shapes) {
                Tensor ga = Tensor::new_uninit(go.dims()), gb = Tensor::new_uninit(go.dims());
                launch(KernelClass::Elementwise, 20.0 * n, "ts_hip_mul_backward", [&] {
                    return ts_hip_mul_backward(go.dev(), a.ptr(), b.ptr(), ga.dev_mut(),
                                               gb.dev_mut(), n, S());
                });
                r.emplace_back(std::move(ga));
                r.emplace_back(std::move(gb));
            } else {
                r.emplace_back(reduce_to(with_bcast(go, b, 2), shape_a));
                r.emplace_back(reduce_to(with_bcast(go, a, 2), shape_b));
            }
            break;
        }
        case K::Div: {  // grad_fn/ops/div.rs:4-49
            const SavedTensor &a = saved[0], &b = saved[1];
            if (!has_shapes) {
                Tensor ga = Tensor::new_uninit(go.dims()), gb = Tensor::new_uninit(go.dims());
                launch(KernelClass::Elementwise, 20.0 * n, "ts_hip_div_backward", [&] {
                    return ts_hip_div_backward(go.dev(), a.ptr(), b.ptr(), ga.dev_mut(),
                                               gb.dev_mut(), n, tail8(n), tail32(n),
                                               Runtime::get().zero_index(), S());
                });
                r.emplace_back(std::move(ga));
                r.emplace_back(std::move(gb));
            } else {
                Tensor ga_full = with_bcast(go, b, 3);                  // go / b
                Tensor neg_grad = with_bcast(go, a, 2);                 // go * a
                Tensor b_sq = same_shape(b.ptr(), b.ptr(), b.dims, 2);  // b * b
                Tensor gb_full = with_bcast(neg_grad, b_sq.saved(), 3);
                Tensor gb_neg = neg_of(gb_full);
                r.emplace_back(reduce_to(ga_full, shape_a));
                r.emplace_back(reduce_to(gb_neg, shape_b));
            }
            break;
        }
        case K::AddScalar:
        case K::SubScalar:
            r.emplace_back(go.alias());
            break;
        case K::MulScalar:
        case K::DivScalar: {
            Tensor g = Tensor::new_uninit(go.dims());
            launch(KernelClass::Elementwise, 8.0 * n, "scalar grad", [&] {
                return kind == K::MulScalar ? ts_hip_mul_scalar(go.dev(), scalar, g.dev_mut(), n, S())
                                            : ts_hip_div_scalar(go.dev(), scalar, g.dev_mut(), n, S());
            });
            r.emplace_back(std::move(g));
            break;
        }
        case K::Relu: {  // grad_fn/ops/relu.rs:4-17 (saved[0] is the relu output)
            Tensor g = Tensor::new_uninit(go.dims());
            launch(KernelClass::Elementwise, 12.0 * n, "ts_hip_relu_backward", [&] {
                return ts_hip_relu_backward(saved[0].ptr(), go.dev(), g.dev_mut(), n, S());
            });
            r.emplace_back(std::move(g));
            break;
        }
        case K::PowScalar: {  // grad_fn/ops/pow.rs:5-27
            Tensor g = Tensor::new_uninit(go.dims());
            launch(KernelClass::Elementwise, 12.0 * n, "ts_hip_pow_backward", [&] {
                return ts_hip_pow_backward(saved[0].ptr(), go.dev(), g.dev_mut(), n, scalar, S());
            });
            r.emplace_back(std::move(g));
            break;
        }
        case K::MatMul: {  // grad_fn/ops/matmul.rs:68-80, transposes folded into the loads
            const SavedTensor &a = saved[0], &b = saved[1];
            const size_t M = a.dims[0], Kd = a.dims[1], N = b.dims[1];
            if (req_left) {  // go[M,N] . b[Kd,N]^T -> [M,Kd]
                Tensor gl = Tensor::new_uninit({M, Kd});
                launch(KernelClass::Gemm, 2.0 * M * N * Kd, "ts_hip_gemm(dX)", [&] {
                    return ts_hip_gemm(0, 1, M, Kd, N, go.dev(), N, b.ptr(), N, gl.dev_mut(), Kd, S());
                });
                r.emplace_back(std::move(gl));
            } else {
                r.emplace_back(std::nullopt);
            }
            if (req_right) {  // a[M,Kd]^T . go[M,N] -> [Kd,N]
                Tensor gr = Tensor::new_uninit({Kd, N});
                launch(KernelClass::Gemm, 2.0 * M * N * Kd, "ts_hip_gemm(dW)", [&] {
                    return ts_hip_gemm(1, 0, Kd, N, M, a.ptr(), Kd, go.dev(), N, gr.dev_mut(), N, S());
                });
                r.emplace_back(std::move(gr));
            } else {
                r.emplace_back(std::nullopt);
            }
            break;
        }
        case K::ReduceSum: {  // grad_fn/reductions/sum.rs:4-16
            Tensor g = Tensor::new_uninit(input_shape);
            launch(KernelClass::Elementwise, 4.0 * g.size(), "sum grad", [&] {
                return go.size() == 1 ? ts_hip_fill_from_device(g.dev_mut(), go.dev(), 1.0f, 0, g.size(), S())
                                      : ts_hip_fill(g.dev_mut(), 1.0f, g.size(), S());
            });
            r.emplace_back(std::move(g));
            break;
        }
        case K::ReduceMean: {  // grad_fn/reductions/mean.rs:4-30
            const float base = numel > 0 ? 1.0f / static_cast<float>(numel) : 0.0f;
            Tensor g = Tensor::new_uninit(input_shape);
            launch(KernelClass::Elementwise, 4.0 * g.size(), "mean grad", [&] {
                return go.size() == 1 ? ts_hip_fill_from_device(g.dev_mut(), go.dev(), base, 1, g.size(), S())
                                      : ts_hip_fill(g.dev_mut(), base, g.size(), S());
            });
            r.emplace_back(std::move(g));
            break;
        }
    }
    return r;
}

}  // namespace ts
