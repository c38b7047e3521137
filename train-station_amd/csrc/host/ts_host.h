// Host side of the MI355X backend: train-station's Tensor / gradtrack /
// Adam API restated in C++ over the C-ABI of include/ts_hip.h.
//
// This library plays the part of train-station's Rust host code
// (train-station/src/tensor, gradtrack, optimizers) for callers without a
// Rust toolchain; it calls the device only through ts_hip.h, exactly as the
// Rust crate would through its FFI block.  Names, argument meaning and error
// behaviour follow the reference:
//   Tensor::{new, zeros, ones, from_slice, with_requires_grad, add_tensor,
//            sub_tensor, mul_tensor, div_tensor, *_scalar, relu, pow_scalar,
//            matmul, sum, mean, backward, grad_by_value, zero_grad, data,
//            value}   (tensor/core/utils.rs, tensor/ops/*, tensor/reductions/*)
//   GradEngine backward worklist                  (gradtrack/engine.rs:962-1047)
//   Adam::{new, with_config, with_learning_rate, add_parameter(s), step,
//          zero_grad}                             (optimizers/adam/mod.rs)
// Reference panics become ts::Error exceptions.
#pragma once

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

#include "ts_serial.h"

namespace ts {

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// ---- runtime ----------------------------------------------------------------

// Throws ts::Error("<what>: <message>") for a non-zero ts_hip status.
void check(int status, const char *what);

// Library state shared by every tensor of the process: the device stream all
// work is queued on, and the device word where division kernels record the
// first zero divisor (reported at the next synchronisation, see sync()).
class Runtime {
  public:
    static Runtime &get();
    void *stream() const { return stream_; }
    unsigned long long *zero_index() const { return zero_index_; }
    // Waits for queued work; throws the reference's division-by-zero panic
    // message if a division kernel recorded a zero divisor.
    void sync();

  private:
    Runtime();
    void *stream_ = nullptr;
    unsigned long long *zero_index_ = nullptr;
};

// Size-bucketed caching allocator for device buffers.  All work runs on the
// one library stream, so a block released after its last use was queued can
// be handed to later work without waiting.
class DevicePool {
  public:
    static DevicePool &get();
    float *acquire(size_t n_floats, size_t *rounded);
    void release(float *p, size_t rounded);
    void empty_cache();
    size_t live_bytes() const { return live_; }
    size_t cached_bytes() const { return cached_; }

    // Step recording (StepRecorder): while a recording is open, every block
    // acquired or used (note_use) is pinned to it; a pinned block released by
    // its owner is parked instead of reused, until every recording that
    // pinned it has been freed (unpin), so a replay never finds its buffers
    // handed to other work.
    void pin_begin(std::vector<float *> *sink);
    void pin_end();
    void note_use(float *p) {
        if (pinning_.load(std::memory_order_relaxed)) pin_locked(p);
    }
    void unpin(const std::vector<float *> &blocks);

  private:
    void pin(float *p);         // pool mutex held
    void pin_locked(float *p);  // takes the pool mutex
    std::atomic<bool> pinning_{false};
    std::unordered_map<size_t, std::vector<float *>> free_;
    size_t live_ = 0, cached_ = 0;
    std::unordered_map<float *, int> pins_;       // block -> recordings pinning it
    std::unordered_map<float *, size_t> parked_;  // released while pinned -> rounded size
    std::vector<float *> *sink_ = nullptr;        // the open recording's pin list
    std::unordered_set<float *> sink_set_;
};

struct Allocation;

// A deferred producer of an allocation's contents: C = op(A) . op(B) with the
// epilogue of ts_hip_gemm_fused (row bias, relu, relu-backward mask), run when
// the contents are first needed.  matmul returns its product deferred; a
// following broadcast bias add, relu, or (in backward) relu's gradient of the
// dX product extends the producer instead of launching a pass of its own, so
// the chain runs as one kernel and intermediates nobody reads are never
// written.  Results are the bits of the unfused ops.
//
// Each product runs once.  A consumer extends a record by forking a copy of
// it; the product's own buffer and every fork belong to one ProductGroup.
// When a member is first needed and it is the group's only member still
// pending, the product runs fused into it (the usual chain: the bare product
// and the bias add's result are dropped, the relu output is read).  With
// other members pending, the product runs once, bare, into its own buffer (or
// a temporary when that was dropped), and every pending member becomes an
// epilogue-only record reading it (`src`): its bias / relu / mask run as the
// separate elementwise kernels, whose bits are the fused epilogue's.
struct ProductGroup {
    std::weak_ptr<Allocation> bare;                  // the product's own buffer
    std::vector<std::weak_ptr<Allocation>> members;  // it and every fork
};

// A weight-gradient product held beside its matmul backward's deferred dX
// product (grad_fn/ops/matmul.rs:68-80 computes both; here for a layer with
// few outputs, whose dW takes the narrow kernel and dX the one-k-tile kernel,
// both latency-bound): when the dX product runs, the two are issued in one
// launch group (ts_hip_launch_group_begin / _end) and run as one launch.
// When one of its outputs (dW, the bias gradient, a loss summed in its
// launch) is read first, or an input is about to be written in place, it
// runs by itself.  Same bits either way.
struct SiblingLaunch {
    std::function<void()> run;                    // the product's launcher, through launch()
    std::vector<std::shared_ptr<Allocation>> inputs;  // fetched before the group forms
    bool done = false;
    std::vector<std::weak_ptr<Allocation>> outputs;
};

struct PendingGemm {
    int ta = 0, tb = 0;
    size_t M = 0, N = 0, K = 0, lda = 0, ldb = 0;
    std::shared_ptr<Allocation> A, B, bias, mask;
    // after the bias: minus a same-shape buffer (the MSE's prediction minus
    // target, ts_hip_gemm_fused_sub; products on the narrow kernel only)
    std::shared_ptr<Allocation> sub;
    std::shared_ptr<Allocation> src;  // epilogue-only: the produced [M, N] buffer the epilogue reads
    bool relu = false;
    std::shared_ptr<ProductGroup> group;
    std::shared_ptr<SiblingLaunch> sibling;  // run in the same launch group as this product
    bool bare() const { return !src && !bias && !sub && !mask && !relu; }
};

// One division checked for zero divisors (the reference's panic in
// div_tensor, ops/div.rs:383-416) recorded in a deferred program: done once a
// pass has computed the division, and so checked it.  A program that is
// copied into a larger one shares its checks, so the check is made once,
// by whichever pass computes the division first.
struct DivCheck {
    bool done = false;
};

// A deferred elementwise value: a chain of same-shape elementwise ops (and
// their backward formulas) recorded as a small program over leaf buffers and
// run by ts_hip_map when the value is first needed.  An op whose operands are
// such values extends their programs instead of launching, so a chain runs as
// one pass that reads each leaf once and writes only what is read later.
// Every node is one op of ts_hip.h's map set, in the reference's fp32 order,
// so each value has the bits of the op-by-op sequence.
struct MapNode {
    static constexpr uint8_t kLeaf = 255;
    uint8_t code = kLeaf;  // TS_HIP_MAP_* or kLeaf
    uint8_t flags = 0;     // TS_HIP_MAP_CHECKED on a division checked for zero
    int16_t a = -1, b = -1;  // operand nodes (earlier ones); a leaf: its index in leaves
    float imm = 0.0f;
    // the allocation this node's value was deferred for, if any: when a
    // program computes it anyway and the allocation is still pending and held
    // elsewhere, the same pass stores it
    std::weak_ptr<Allocation> origin;
    // a checked division: the checks it stands for (several when equal
    // divisions were merged into one node)
    std::vector<std::shared_ptr<DivCheck>> checks;
};

struct PendingMap {
    size_t n = 0;  // elements
    std::vector<std::shared_ptr<Allocation>> leaves;
    uint32_t scalar = 0;  // bit k: leaf k is one value used for every element
    // bit k: leaf k is the constant values[k] (no buffer; leaves[k] is null)
    uint32_t consts = 0;
    std::vector<float> values;  // per leaf
    std::vector<MapNode> nodes;  // in evaluation order
    int root = -1;
    // the whole program is one constant (a deferred fill): its value, or null
    const float *constant() const {
        return (leaves.size() == 1 && consts == 1u && nodes.size() == 1 && root == 0) ? &values[0] : nullptr;
    }
};

// A deferred column sum out[n] = sum over r of src[r][n] of a [rows, cols]
// buffer: the bias gradient, reduce_to [rows, cols] -> [cols].  It runs as
// ts_hip_sum_dim0 when first read, unless the weight-gradient product that
// reads the same rows runs first: that product writes it too
// (ts_hip_gemm_colsum), so the rows are read once for both.  Same bits either
// way.
struct PendingColsum {
    std::shared_ptr<Allocation> src;
    size_t rows = 0, cols = 0;
};

// A deferred transposed copy: the contents are src (dims) with axes d0 and d1
// swapped, written by ts_hip_transpose when first read.  A product reads a
// transposed matrix through its trans flag instead (the copy is never made),
// and transposing it back gives src itself.  `view`: the result of
// Tensor::transpose / t(), which, like the reference's strided view
// (transform/transpose.rs:183-186), reads src as src is when it is read (no
// reader link, so an in-place write of src is not held back for it); not a
// view: contiguous()'s copy, which keeps src's values at the call (a reader
// of src, run before src is written in place).
struct PendingTranspose {
    std::shared_ptr<Allocation> src;
    std::vector<size_t> dims;  // src's
    size_t d0 = 0, d1 = 1;
    bool view = true;
};

// A deferred sum or mean of a deferred elementwise value or product x
// (reductions/sum.rs:80-141, mean.rs:48-109): out[0] = sum(x), divided by
// (float)n for the mean, with the bits of ts_hip_sum / ts_hip_mean over x's
// values.  The first pass that reads x's inputs anyway adds x up as its
// reduction (backward of the loss usually is that pass), and a weight-gradient
// product that reads x as its right operand can add it up in its own launch
// (ts_hip_gemm_colsum_bsum); otherwise it runs when out is read.
struct PendingReduce {
    std::shared_ptr<Allocation> x;
    size_t n = 0;
    bool mean = false;
};

// Device variant of tensor/core/allocation.rs:43-187: owns one pooled device
// buffer; shared (Arc-like) by tensors, saved graph operands and gradients.
struct Allocation : std::enable_shared_from_this<Allocation> {
    explicit Allocation(size_t n_floats);
    ~Allocation();
    Allocation(const Allocation &) = delete;
    Allocation &operator=(const Allocation &) = delete;
    // The device buffer, after running a pending producer.
    float *get();
    // The device buffer as it is (for the producer itself and the pool).
    float *raw() const { return ptr_; }
    // Before this buffer is written in place: runs every still-pending
    // producer that reads it, so they see the old contents.
    void before_write();
    std::shared_ptr<PendingGemm> pending;
    std::shared_ptr<PendingMap> map;                 // deferred elementwise value
    std::shared_ptr<PendingColsum> colsum;           // deferred column sum
    std::shared_ptr<PendingTranspose> transpose;     // deferred transposed copy
    std::shared_ptr<PendingReduce> reduce;           // deferred sum / mean
    std::shared_ptr<SiblingLaunch> sibling;          // written by a held weight-gradient product
    bool deferred() const { return pending || map || colsum || transpose || reduce || sibling; }
    std::vector<std::weak_ptr<Allocation>> readers;  // pending allocations reading this one
    size_t n = 0, rounded = 0;
    // held by this thread's list of deferred programs with a checked
    // division not yet computed (run_division_checks), one reference more
    // than its users hold
    bool check_hold = false;

  private:
    float *ptr_ = nullptr;
};

// Runs a's pending producer (tensor.cpp).
void materialize(Allocation &a);
// Runs a's deferred elementwise program (tensor.cpp).
void materialize_map(Allocation &a);
// Runs a's deferred column sum (tensor.cpp).
void materialize_colsum(Allocation &a);
// Runs a's deferred transposed copy (tensor.cpp).
void materialize_transpose(Allocation &a);
// Runs a's deferred sum / mean (tensor.cpp).
void materialize_reduce(Allocation &a);
// Runs the held product that writes a, by itself (tensor.cpp).
void run_sibling(Allocation &a);
// A matrix operand as a product reads it: a 2-D transposed view or copy not
// yet written is its source with the trans flag set (tensor.cpp).
struct MatOperand {
    std::shared_ptr<Allocation> buf;
    int trans = 0;
};
MatOperand mat_operand(const std::shared_ptr<Allocation> &a);
// Runs the deferred elementwise programs of several allocations, merged into
// as few passes as the program limits allow (tensor.cpp).
void materialize_maps(const std::vector<std::shared_ptr<Allocation>> &allocs);
// Runs every deferred program of this thread that holds a checked division
// no pass has computed yet, whether or not its value is still held, so a
// zero divisor is reported by the next synchronisation even when the
// quotient is never read (Runtime::sync calls it first).  Only divisions
// with a tail are tracked: the check covers the elements past the last
// whole 32-element block, as the reference's does (ops/div.rs:378-417).
void run_division_checks();
// Makes `out` pending on p and records it as a reader of p's inputs.
void set_pending(const std::shared_ptr<Allocation> &out, std::shared_ptr<PendingGemm> p);
// A new deferred product C = op(A) . op(B) for `out`, the first member of
// its group.
std::shared_ptr<PendingGemm> new_product(const std::shared_ptr<Allocation> &out);
// A copy of src's pending record for `out` to extend with an epilogue, joined
// to src's product group; nullptr when src has no pending record.
std::shared_ptr<PendingGemm> fork_pending(const std::shared_ptr<Allocation> &src, const std::shared_ptr<Allocation> &out);
// Fusion switch (on by default): off, every op launches its own kernels.
void set_fusion(bool on);
bool fusion_enabled();

// ---- profiling ----------------------------------------------------------------

// Optional per-launch timing with device events on the library stream,
// grouped by kernel class, with each launch's algorithmic work (FLOPs for
// GEMMs, bytes for the bandwidth-bound kernels).
enum class KernelClass : int { Gemm = 0, Elementwise = 1, Reduction = 2, Adam = 3, kCount = 4 };

struct ClassStats {
    double ms = 0.0;
    double work = 0.0;  // FLOPs (Gemm) or bytes (others)
    uint64_t launches = 0;
};

class Profiler {
  public:
    static Profiler &get();
    void enable(bool on);
    bool enabled() const { return enabled_; }
    // Classes timed (bit k for KernelClass k; all by default).  Launches of
    // other classes record no events, so timing one class perturbs the rest
    // of the stream least.
    void set_classes(unsigned mask) { classes_ = mask; }
    void begin(KernelClass k);
    void end(KernelClass k, double work);
    void abort();  // the launch failed: drop its window
    // Synchronises and folds every recorded launch into the totals.
    void collect();
    ClassStats stats(KernelClass k) const { return totals_[static_cast<int>(k)]; }
    void reset();

  private:
    // A run of kernels timed by one pair of events carried in their dispatches
    // (ts_hip_timing_begin/end); kernels == 0: the events were never recorded.
    struct Segment {
        void *start = nullptr, *stop = nullptr;
        int kernels = -1;  // -1 while the window is open
    };
    using Segments = std::vector<Segment>;
    struct Pending {
        Segments segments;
        KernelClass k;
        double work;
    };
    struct Frame {
        bool timed;         // its class is selected: its segments are recorded
        Segments segments;  // while timed
    };
    void *event();
    void open_segment(Segments &segs);
    void close_segment(Segments &segs);
    void pause_enclosing();
    void resume_enclosing();
    bool enabled_ = false;
    unsigned classes_ = ~0u;
    std::vector<Frame> open_;  // launches in progress, innermost last
    std::vector<Pending> pending_;
    std::vector<void *> spare_;
    ClassStats totals_[static_cast<int>(KernelClass::kCount)];
};

// Runs one launcher (a call returning a ts_hip status), timed by the profiler
// when it is enabled; a failed status throws with `what` in the message.
// Operands should be fetched before the call (a deferred operand that runs
// inside the window is charged to its own class all the same).
// While a launch group forms (a dX product and its held sibling), the
// launchers' GEMM calls are issued into the group with no profiler window of
// their own: the group's one launch is timed once, with their work summed.
struct LaunchCollector {
    double work = 0.0;
};
LaunchCollector *&launch_collector();

template <class F>
void launch(KernelClass k, double work, const char *what, F &&f) {
    if (LaunchCollector *c = launch_collector(); c && k == KernelClass::Gemm) {
        check(f(), what);
        c->work += work;
        return;
    }
    Profiler &P = Profiler::get();
    P.begin(k);
    try {
        check(f(), what);
    } catch (...) {
        P.abort();
        throw;
    }
    P.end(k, work);
}

// ---- tensors --------------------------------------------------------------------

class Tensor;

struct SavedTensor {
    std::shared_ptr<Allocation> alloc;
    std::vector<size_t> dims;
    const float *ptr() const { return alloc ? alloc->get() : nullptr; }
};

// GradFn variants on the training-step path (gradtrack/grad_fn/mod.rs:127-450).
struct GradFn {
    enum class Kind {
        Add, Sub, Mul, Div, AddScalar, SubScalar, MulScalar, DivScalar,
        Relu, PowScalar, MatMul, ReduceSum, ReduceMean,
        Exp, Log, Sqrt, Tanh, Sigmoid, LeakyRelu, Softmax, ReduceSumDims, ReduceMeanDims,
        Transpose, Contiguous
    };
    explicit GradFn(Kind k) : kind(k) {}
    Kind kind;
    bool has_shapes = false;           // original_shapes: Some((a, b))
    std::vector<size_t> shape_a, shape_b;
    float scalar = 0.0f;               // scalar operand or exponent
    std::vector<SavedTensor> saved;    // saved operands, shared not copied
    bool req_left = false, req_right = false;
    std::vector<size_t> input_shape;   // reductions
    size_t numel = 0;
    std::vector<size_t> reduce_dims;   // sum_dims / mean_dims: sorted, deduplicated
    bool keepdim = false;
    size_t axis = 0;                   // softmax
    size_t dim0 = 0, dim1 = 0;         // transpose: the axes swapped

    // GradFn::apply (grad_fn/mod.rs:490-789): gradients by operand position.
    std::vector<std::optional<Tensor>> apply(const Tensor &grad_output) const;
};

class Tensor {
  public:
    Tensor() = default;
    Tensor(Tensor &&) = default;
    Tensor &operator=(Tensor &&) = default;
    Tensor(const Tensor &) = delete;
    Tensor &operator=(const Tensor &) = delete;

    // construction (tensor/core/utils.rs:120-171, init/basic.rs, init/data.rs)
    static Tensor new_uninit(std::vector<size_t> dims);
    static Tensor zeros(std::vector<size_t> dims);
    static Tensor ones(std::vector<size_t> dims);
    static Tensor filled(std::vector<size_t> dims, float v);
    // filled(dims, v), deferred with fusion on: the value becomes a constant
    // of the elementwise program that reads it (the gradient seed of
    // backward(None)), and is written only if something else reads it.
    static Tensor constant(std::vector<size_t> dims, float v);
    static Tensor from_slice(const float *data, size_t len, std::vector<size_t> dims);
    // Tensor::randn (init/random.rs:231-235): XorShiftRng values generated on
    // the device; without a seed, one derived from the clock (random.rs:492-497)
    static Tensor randn(std::vector<size_t> dims, const uint64_t *seed);
    // fill_randn (random.rs:270-299), in place
    void fill_randn(const uint64_t *seed);

    // Checkpoint in the reference's formats (StructSerializable for Tensor,
    // tensor/core/serialization.rs:179-288; serialization/core/traits.rs)
    std::vector<uint8_t> to_binary() const;
    static Tensor from_binary(const uint8_t *data, size_t len);
    std::string to_json() const;
    static Tensor from_json(const std::string &json);
    void save_binary(const std::string &path) const;
    void save_json(const std::string &path) const;
    static Tensor load_binary(const std::string &path);
    static Tensor load_json(const std::string &path);

    // Tensor::clone: new buffer with the same values, new id, no grad
    Tensor clone() const;
    // Handle on the same buffer with a new id (graph-internal sharing).
    Tensor alias() const;
    // Handle on the same buffer with the same id: this tensor itself, as a
    // reference to it (&Tensor) would see it; carries no gradient.
    Tensor view() const;

    size_t id() const { return id_; }
    const std::vector<size_t> &dims() const { return dims_; }
    size_t size() const { return size_; }
    const float *dev() const { return alloc_ ? alloc_->get() : nullptr; }
    const std::shared_ptr<Allocation> &allocation() const { return alloc_; }
    float *dev_mut() { return alloc_ ? alloc_->get() : nullptr; }
    SavedTensor saved() const { return SavedTensor{alloc_, dims_}; }
    static Tensor from_saved(const SavedTensor &s);

    // gradient API (tensor/core/utils.rs:412-790)
    bool requires_grad() const { return requires_grad_; }
    Tensor &with_requires_grad() { requires_grad_ = true; return *this; }
    void set_requires_grad(bool r);
    void backward(const Tensor *grad_output = nullptr);
    std::optional<Tensor> grad_by_value() const;
    // Tensor::grad (utils.rs:491-506): the gradient stored on the tensor
    // itself, or nullptr -- also when only the graph's map holds one, as there.
    const Tensor *grad_direct() const { return grad_.get(); }
    // The gradient Adam reads: self.grad, else the graph's map entry; no copy.
    const Tensor *grad_ref() const;
    void set_grad(Tensor g);
    void zero_grad() { grad_.reset(); }
    void accumulate_grad(Tensor g);

    // recorded ops
    Tensor add_tensor(const Tensor &o) const;
    Tensor sub_tensor(const Tensor &o) const;
    Tensor mul_tensor(const Tensor &o) const;
    Tensor div_tensor(const Tensor &o) const;
    Tensor add_scalar(float s) const;
    Tensor sub_scalar(float s) const;
    Tensor mul_scalar(float s) const;
    Tensor div_scalar(float s) const;
    Tensor relu() const;
    Tensor pow_scalar(float e) const;
    Tensor matmul(const Tensor &o) const;
    Tensor sum() const;
    Tensor mean() const;
    // tensor/ops/{exp,log,sqrt,tanh,sigmoid,leaky_relu,softmax}.rs
    Tensor exp() const;
    Tensor log() const;
    Tensor sqrt() const;
    Tensor tanh() const;
    Tensor sigmoid() const;
    Tensor leaky_relu(float negative_slope) const;
    Tensor softmax(size_t dim) const;
    // reductions/sum.rs:225-306, reductions/mean.rs:186-230
    Tensor sum_dims(const std::vector<size_t> &dims, bool keepdim) const;
    Tensor mean_dims(const std::vector<size_t> &dims, bool keepdim) const;
    // transform/transpose.rs:156-291, contiguous.rs:123-157: a transposed
    // view (deferred copy, see PendingTranspose), t() = the last two axes;
    // contiguous() of a view is its copy, of anything else a clone; both
    // record their GradFn whenever the input requires grad (no
    // is_grad_enabled check, as there)
    Tensor transpose(size_t dim0, size_t dim1) const;
    Tensor t() const;
    Tensor contiguous() const;
    bool is_contiguous() const;
    // init/basic.rs:304-326: every element set to value, in place
    void fill(float value);

    // host access (synchronises)
    std::vector<float> data() const;
    void copy_to_host(float *out, size_t len) const;
    float value() const;

  private:
    friend struct GradFn;
    Tensor binary(const Tensor &o, GradFn::Kind kind) const;
    Tensor scalar_op(float s, GradFn::Kind kind) const;
    template <class F>
    Tensor unary(GradFn::Kind kind, const char *what, bool save_output, float slope, F &&launcher) const;
    void record(Tensor &out, std::vector<size_t> input_ids, GradFn fn) const;

    std::shared_ptr<Allocation> alloc_;
    std::vector<size_t> dims_;
    size_t size_ = 0;
    size_t id_ = 0;
    bool requires_grad_ = false;
    // a transposed view of a contiguous tensor (transform/transpose.rs:
    // 182-186): is_contiguous() is false, as for the reference's strided view
    bool strided_ = false;
    std::shared_ptr<Tensor> grad_;
};

// x with axes d0 != d1 swapped, deferred (no recording): a deferred bare
// matrix product becomes the product of its swapped operands; a pending view
// transposed back, a deferred copy of its source; anything else a
// PendingTranspose of x (a view when `view`).
Tensor transposed_value(const Tensor &x, size_t d0, size_t d1, bool view);

size_t next_tensor_id();

// ---- gradtrack -------------------------------------------------------------------

bool is_grad_enabled();             // no_grad_track.rs:155-160
void push_grad_enabled(bool on);    // NoGradTrack::new / with_no_grad (no_grad_track.rs:96-104, :229-235)
void pop_grad_enabled();            // NoGradTrack's Drop (no_grad_track.rs:117-127)
void set_grad_enabled(bool on);     // no_grad_track.rs:188-199: replaces the innermost state
void clear_gradients();             // engine.rs:812-816
// existing + g (engine.rs:514-524), deferred into the gradients' pass when fusion is on
Tensor add_gradients(const Tensor &existing, const Tensor &g);
bool gradients_pending();           // the gradient map holds at least one gradient
void register_operation(size_t output_id, std::vector<size_t> input_ids, GradFn fn);
const Tensor *accumulated_gradient(size_t id);
void engine_backward(Tensor &root, const Tensor *grad_output);
// true while engine_backward runs on this thread: its passes store only the
// values they run for (the forward values they recompute are past their last
// graph use)
bool in_backward();

// ---- optimizer -----------------------------------------------------------------------

struct AdamConfig {
    float learning_rate = 1e-3f;
    float beta1 = 0.9f;
    float beta2 = 0.999f;
    float eps = 1e-8f;
    float weight_decay = 0.0f;
    bool amsgrad = false;
};

// AdamConfig on its own (StructSerializable, adam/serialization.rs:40-62)
std::vector<uint8_t> adam_config_to_binary(const struct AdamConfig &c);
std::string adam_config_to_json(const struct AdamConfig &c);
struct AdamConfig adam_config_from_binary(const uint8_t *data, size_t len);
struct AdamConfig adam_config_from_json(const std::string &json);

// Rust's Debug form of a shape, "[2, 3]"
std::string dims_str(const std::vector<size_t> &d);

// Step counters of one optimizer: its global step count and, per parameter,
// the steps that replays of recorded steps ran (or a recording took back)
// that the parameter's state has not absorbed yet.  Shared by the optimizer
// and every step graph that recorded one of its steps, so a replay reads the
// count the optimizer has at that moment, whatever ran in between.
struct AdamLedger {
    uint64_t step_count = 0;                          // adam/mod.rs:1037, replays included
    std::unordered_map<size_t, int64_t> param_delta;  // parameter id -> steps to add to its State
};

class Adam {
  public:
    Adam() = default;
    Adam(Adam &&) = default;
    Adam &operator=(Adam &&) = default;
    Adam(const Adam &) = delete;
    Adam &operator=(const Adam &) = delete;
    static Adam with_config(AdamConfig c);
    static Adam with_learning_rate(float lr);
    void add_parameter(const Tensor &p);
    void add_parameters(const std::vector<const Tensor *> &ps);
    // Optimizer::step (adam/mod.rs:1036-1044); warns and skips params without grads.
    void step(const std::vector<Tensor *> &params);
    // Optimizer::zero_grad (adam/mod.rs:1061-1068)
    void zero_grad(const std::vector<Tensor *> &params);
    float learning_rate() const { return config_.learning_rate; }
    void set_learning_rate(float lr) { config_.learning_rate = lr; }
    const AdamConfig &config() const { return config_; }
    uint64_t step_count() const { return ledger_->step_count; }
    size_t parameter_count() const { return states_.size(); }
    // m / v of a linked parameter (device), for checkpoint and tests.
    const float *state_m(size_t param_id) const;
    const float *state_v(size_t param_id) const;

    // Checkpoint (optimizers/adam/serialization.rs:140-235).  A loaded
    // optimizer holds the saved states under the saved parameter ids until
    // relink_parameters maps them, by insertion position, onto live tensors
    // (adam/mod.rs:396-454).
    std::vector<uint8_t> to_binary() const;
    static Adam from_binary(const uint8_t *data, size_t len);
    std::string to_json() const;
    static Adam from_json(const std::string &json);
    void save_binary(const std::string &path) const;
    void save_json(const std::string &path) const;
    static Adam load_binary(const std::string &path);
    static Adam load_json(const std::string &path);
    void relink_parameters(const std::vector<const Tensor *> &params);
    size_t saved_parameter_count() const { return states_.size(); }
    // per-parameter step counter (ParameterState::step), 0 if not linked
    uint64_t parameter_step(size_t param_id) const;

  private:
    struct State {
        std::shared_ptr<Allocation> m, v, v_hat_max;
        std::vector<size_t> dims;
        size_t n = 0;
        uint64_t step = 0;
    };
    // Adds the ledger's per-parameter deltas to the states.
    void settle() const;
    ser::Fields to_fields(bool binary) const;
    static Adam from_fields(const ser::Fields &f);
    AdamConfig config_;
    mutable std::unordered_map<size_t, State> states_;
    std::vector<size_t> insertion_order_;
    std::shared_ptr<AdamLedger> ledger_ = std::make_shared<AdamLedger>();
};

// ---- step recording ----------------------------------------------------------------

// One recorded step: a HIP graph of the library stream's work between
// StepRecorder::begin and end, the blocks it pinned, and per recorded
// Adam::step a table of bias corrections, which each recorded Adam launch
// indexes by device tickets of its own (ts_hip_adam_step_multi_ticket: the
// r-th launch since the tickets were cleared reads entry r, so a replay needs
// no counter-advancing launch).  A recording itself runs nothing, so it leaves
// every step counter as it was; each replay then counts as many steps as it
// ran.
struct StepGraph {
    ~StepGraph();
    // Runs the recorded work `times` times in stream order.
    void replay(size_t times);
    void *exec = nullptr;
    std::vector<float *> pins;
    std::vector<std::shared_ptr<Allocation>> tickets;  // per recorded Adam launch, one unsigned per wave
    struct AdamUse {
        std::shared_ptr<Allocation> table;  // kReplayChunk [cf1, cf2] pairs
        float beta1 = 0, beta2 = 0;
        std::shared_ptr<AdamLedger> ledger;
        size_t order = 0;       // recorded steps of the same optimizer before this one
        size_t per_replay = 0;  // recorded steps of that optimizer in this graph
        std::vector<size_t> params;  // the parameters this step updated
    };
    std::vector<AdamUse> adams;
    uint64_t executed = 0;  // replays run so far
};

class StepRecorder {
  public:
    static constexpr size_t kReplayChunk = 1024;  // replays per bias-correction table fill
    static StepRecorder &get();
    bool open() const { return graph_ != nullptr; }
    // Refuses to start while the gradient map holds gradients: a recorded
    // accumulation would add that fixed buffer again on every replay.
    void begin();
    StepGraph *end();
    void abort();
    // Called by Adam::step while recording, before it counts the step: the
    // table its launches read; `use` names the step for adam_param, which
    // records each parameter as soon as it is stepped.
    struct AdamSlot {
        const float *table;
        size_t use;
    };
    AdamSlot adam_step(float beta1, float beta2, const std::shared_ptr<AdamLedger> &ledger);
    // The tickets of one recorded Adam launch of `waves` waves (cleared
    // before each run of replays).
    unsigned *adam_tickets(size_t waves);
    void adam_param(size_t use, size_t param_id);

  private:
    // The counts the recorded Adam steps added while recording, taken back.
    static void take_back(StepGraph &g);
    std::unique_ptr<StepGraph> graph_;
};

// Host <-> device copies cannot be recorded (a replay would copy from or to
// host memory that no longer holds the data): refused while recording.
inline void refuse_while_recording(const char *what) {
    if (StepRecorder::get().open())
        throw Error(std::string(what) + ": a step being recorded cannot upload or read device data; "
                                        "create inputs before the recording and read results after a replay");
}

}  // namespace ts
