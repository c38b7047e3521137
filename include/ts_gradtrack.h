/*
 * ts_gradtrack.h -- C handle API of the host-side mirror of train-station's
 * Tensor / gradtrack / Adam (libts_gradtrack.so), for callers that are not
 * C++ (Python ctypes tests and bench, or a foreign host).  Each entry names
 * the reference method it mirrors.  The library reaches the device only
 * through include/ts_hip.h.
 *
 * Errors: calls returning a pointer return NULL, calls returning int return
 * -1; ts_last_error() then holds the message (the reference panics with the
 * same text).  Handles are owned by the caller and released with
 * ts_tensor_free / ts_adam_free.
 */
#ifndef TS_GRADTRACK_H
#define TS_GRADTRACK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ts_tensor ts_tensor;
typedef struct ts_adam ts_adam;
typedef struct ts_step_graph ts_step_graph;

const char *ts_last_error(void);

/* Tensor::new (tensor/core/utils.rs:120-171), uninitialised */
ts_tensor *ts_tensor_new(const size_t *dims, size_t rank);
/* Tensor::zeros / ones (init/basic.rs:136-180) */
ts_tensor *ts_tensor_zeros(const size_t *dims, size_t rank);
ts_tensor *ts_tensor_ones(const size_t *dims, size_t rank);
/* Tensor::from_slice (init/data.rs:227-247) */
ts_tensor *ts_tensor_from_slice(const float *data, size_t len, const size_t *dims, size_t rank);
/* Tensor::randn(dims, seed) / fill_randn (init/random.rs:231-299): values of
 * the reference's XorShiftRng + Box-Muller, generated on the device.  With
 * has_seed == 0 the seed comes from the clock, as XorShiftRng::new_from_time
 * (random.rs:492-497) does. */
ts_tensor *ts_tensor_randn(const size_t *dims, size_t rank, uint64_t seed, int has_seed);
int ts_tensor_fill_randn(ts_tensor *t, uint64_t seed, int has_seed);
/* Tensor::clone (core/mod.rs:344-378): new buffer, new id, no grad */
ts_tensor *ts_tensor_clone(const ts_tensor *t);
void ts_tensor_free(ts_tensor *t);

uint64_t ts_tensor_id(const ts_tensor *t);
size_t ts_tensor_rank(const ts_tensor *t);
size_t ts_tensor_dims(const ts_tensor *t, size_t *dims_out, size_t cap);
size_t ts_tensor_size(const ts_tensor *t);
const float *ts_tensor_device_ptr(const ts_tensor *t);

/* with_requires_grad / set_requires_grad / requires_grad (utils.rs:412-450) */
int ts_tensor_with_requires_grad(ts_tensor *t);
int ts_tensor_set_requires_grad(ts_tensor *t, int requires_grad);
int ts_tensor_requires_grad(const ts_tensor *t);

/* recorded ops (tensor/ops/{add,sub,mul,div,relu,pow}.rs, ops/matmul/mod.rs,
 * tensor/reductions/{sum,mean}.rs).  The binary ops broadcast NumPy-style
 * (ops/broadcasting.rs:299-478), up to rank 8. */
ts_tensor *ts_tensor_add_tensor(const ts_tensor *a, const ts_tensor *b);
ts_tensor *ts_tensor_sub_tensor(const ts_tensor *a, const ts_tensor *b);
ts_tensor *ts_tensor_mul_tensor(const ts_tensor *a, const ts_tensor *b);
ts_tensor *ts_tensor_div_tensor(const ts_tensor *a, const ts_tensor *b);
ts_tensor *ts_tensor_add_scalar(const ts_tensor *a, float s);
ts_tensor *ts_tensor_sub_scalar(const ts_tensor *a, float s);
ts_tensor *ts_tensor_mul_scalar(const ts_tensor *a, float s);
ts_tensor *ts_tensor_div_scalar(const ts_tensor *a, float s);
ts_tensor *ts_tensor_relu(const ts_tensor *a);
ts_tensor *ts_tensor_pow_scalar(const ts_tensor *a, float exponent);
ts_tensor *ts_tensor_matmul(const ts_tensor *a, const ts_tensor *b);
ts_tensor *ts_tensor_sum(const ts_tensor *a);
ts_tensor *ts_tensor_mean(const ts_tensor *a);
/* tensor/ops/{exp,log,sqrt,tanh,sigmoid,leaky_relu,softmax}.rs; exp / log /
 * tanh (and sigmoid's exp) are correctly rounded where the reference uses the
 * host libm */
ts_tensor *ts_tensor_exp(const ts_tensor *a);
ts_tensor *ts_tensor_log(const ts_tensor *a);
ts_tensor *ts_tensor_sqrt(const ts_tensor *a);
ts_tensor *ts_tensor_tanh(const ts_tensor *a);
ts_tensor *ts_tensor_sigmoid(const ts_tensor *a);
ts_tensor *ts_tensor_leaky_relu(const ts_tensor *a, float negative_slope);
ts_tensor *ts_tensor_softmax(const ts_tensor *a, size_t dim);
/* sum_dims / mean_dims (reductions/sum.rs:225-306, mean.rs:186-230) */
ts_tensor *ts_tensor_sum_dims(const ts_tensor *a, const size_t *dims, size_t ndims, int keepdim);
ts_tensor *ts_tensor_mean_dims(const ts_tensor *a, const size_t *dims, size_t ndims, int keepdim);

/* transpose(dim0, dim1) / t() (transform/transpose.rs:156-208, :283-291): a
 * transposed view, recorded (Transpose GradFn, grad_fn/mod.rs:243-249, :575)
 * whenever the input requires grad.  The view's values are copied only when
 * something reads them; a 2-D view given to matmul is read by the product
 * with its transpose flag instead (forward and backward), never copied.
 * contiguous() (transform/contiguous.rs:123-157): a view's copy, anything
 * else's clone (Contiguous GradFn: identity).  is_contiguous(): 0 for a
 * transposed view of a contiguous tensor.  Panics as the reference: "dim0 2
 * out of bounds for tensor with rank 2", "Matrix transpose requires at least
 * 2 dimensions, got 1". */
ts_tensor *ts_tensor_transpose(const ts_tensor *a, size_t dim0, size_t dim1);
ts_tensor *ts_tensor_t(const ts_tensor *a);
ts_tensor *ts_tensor_contiguous(const ts_tensor *a);
int ts_tensor_is_contiguous(const ts_tensor *a);
/* Tensor::fill (init/basic.rs:304-326): every element set to value, in place
 * (through a view not yet copied, into its source, which it shares) */
int ts_tensor_fill(ts_tensor *t, float value);

/* Tensor::backward(Option<Tensor>) (utils.rs:634-636); grad_output may be NULL */
int ts_tensor_backward(ts_tensor *t, const ts_tensor *grad_output);
/* Tensor::grad (utils.rs:491-506): the gradient stored on the tensor itself
 * (set_grad, or the backward root's own accumulation), as a handle on the
 * same buffer and id (no copy; free the handle, the gradient stays); NULL
 * with ts_last_error() "" when there is none -- also when only the graph's
 * gradient map holds one, as in the reference. */
ts_tensor *ts_tensor_grad(const ts_tensor *t);
/* grad_by_value (utils.rs:525-534): a copy, or NULL with ts_last_error() ""
 * when there is no gradient */
ts_tensor *ts_tensor_grad_by_value(const ts_tensor *t);
/* set_grad / zero_grad (utils.rs:766-790) */
int ts_tensor_set_grad(ts_tensor *t, const ts_tensor *grad);
int ts_tensor_zero_grad(ts_tensor *t);
/* data() / value(): device -> host, synchronises (utils.rs:1251-1260) */
int ts_tensor_data(const ts_tensor *t, float *out, size_t len);
int ts_tensor_value(const ts_tensor *t, float *out);

/* gradtrack (engine.rs:812-816, no_grad_track.rs:80-235) */
void ts_clear_gradients(void);
void ts_no_grad_push(void);
void ts_no_grad_pop(void);
int ts_is_grad_enabled(void);
/* set_grad_enabled (no_grad_track.rs:188-199): replaces the innermost state */
void ts_set_grad_enabled(int enabled);

/* Adam (optimizers/adam/mod.rs:227-320, :1036-1068) */
ts_adam *ts_adam_new(void);
ts_adam *ts_adam_with_config(float learning_rate, float beta1, float beta2, float eps,
                             float weight_decay, int amsgrad);
ts_adam *ts_adam_with_learning_rate(float learning_rate);
void ts_adam_free(ts_adam *opt);
int ts_adam_add_parameter(ts_adam *opt, const ts_tensor *param);
int ts_adam_step(ts_adam *opt, ts_tensor *const *params, size_t count);
int ts_adam_zero_grad(ts_adam *opt, ts_tensor *const *params, size_t count);
float ts_adam_learning_rate(const ts_adam *opt);
void ts_adam_set_learning_rate(ts_adam *opt, float lr);
uint64_t ts_adam_step_count(const ts_adam *opt);
/* copy a linked parameter's m or v (which 0 / 1) to the host */
int ts_adam_state(const ts_adam *opt, const ts_tensor *param, int which, float *out, size_t len);

/* ---- checkpoint / resume ------------------------------------------------------
 * The reference's formats (serialization/binary "TS_B" v1 and JSON) through
 * StructSerializable (serialization/core/traits.rs): to_binary / from_binary,
 * to_json / from_json, save_* / load_* on a path.  Buffers returned through
 * `data` are owned by the caller and released with ts_buffer_free; JSON text
 * is NUL-terminated and *len excludes the NUL. */
void ts_buffer_free(void *data);
/* Tensor (tensor/core/serialization.rs:179-288): data, shape, device,
 * requires_grad.  Loaded tensors are placed on the device. */
int ts_tensor_to_binary(const ts_tensor *t, uint8_t **data, size_t *len);
ts_tensor *ts_tensor_from_binary(const uint8_t *data, size_t len);
int ts_tensor_to_json(const ts_tensor *t, char **json, size_t *len);
ts_tensor *ts_tensor_from_json(const char *json, size_t len);
int ts_tensor_save_binary(const ts_tensor *t, const char *path);
int ts_tensor_save_json(const ts_tensor *t, const char *path);
ts_tensor *ts_tensor_load_binary(const char *path);
ts_tensor *ts_tensor_load_json(const char *path);
/* Adam (optimizers/adam/serialization.rs:140-235): config, per-parameter
 * m / v / v_hat_max / step, step_count, insertion_order.  A loaded optimizer
 * keeps the saved states under the saved parameter ids; relink them onto the
 * live parameters, in insertion order, with ts_adam_relink_parameters
 * (adam/mod.rs:396-454) before stepping. */
int ts_adam_to_binary(const ts_adam *opt, uint8_t **data, size_t *len);
ts_adam *ts_adam_from_binary(const uint8_t *data, size_t len);
int ts_adam_to_json(const ts_adam *opt, char **json, size_t *len);
ts_adam *ts_adam_from_json(const char *json, size_t len);
int ts_adam_save_binary(const ts_adam *opt, const char *path);
int ts_adam_save_json(const ts_adam *opt, const char *path);
ts_adam *ts_adam_load_binary(const char *path);
ts_adam *ts_adam_load_json(const char *path);
int ts_adam_relink_parameters(ts_adam *opt, const ts_tensor *const *params, size_t count);
/* Adam::saved_parameter_count (adam/serialization.rs:226-228) */
size_t ts_adam_saved_parameter_count(const ts_adam *opt);
/* ParameterState::step of a linked parameter (0 if not linked) */
uint64_t ts_adam_parameter_step(const ts_adam *opt, const ts_tensor *param);
/* the optimizer's AdamConfig (learning_rate, beta1, beta2, eps, weight_decay)
 * and amsgrad flag */
int ts_adam_config(const ts_adam *opt, float *values5, int *amsgrad);
/* AdamConfig on its own (adam/serialization.rs:40-62) */
int ts_adam_config_to_binary(const float *values5, int amsgrad, uint8_t **data, size_t *len);
int ts_adam_config_from_binary(const uint8_t *data, size_t len, float *values5, int *amsgrad);
int ts_adam_config_to_json(const float *values5, int amsgrad, char **json, size_t *len);
int ts_adam_config_from_json(const char *json, size_t len, float *values5, int *amsgrad);

/* runtime: wait for queued work (reports a recorded division by zero) */
int ts_synchronize(void);

/* Fusion of recorded ops into the producing product (no counterpart in the
 * reference): with it on (the default), a 2-D matmul's product is deferred
 * until its result is first read, a following add_tensor of a row vector and
 * a relu are applied in that product's store, and in backward relu's gradient
 * of the dX product is applied in its store (ts_hip_gemm_fused).  Results are
 * bit-identical either way; off, every op launches its own kernels.  Products
 * that read a tensor written in place (Adam::step, fill_randn) run before the
 * write; a caller writing through ts_tensor_device_ptr should read the
 * tensors that depend on it first, or switch fusion off. */
void ts_fusion_enable(int on);
int ts_fusion_enabled(void);

/* Step graphs (no counterpart in the reference, whose steps run eagerly on
 * the CPU): the library stream's work between ts_step_graph_begin and
 * ts_step_graph_end (typically a forward, ts_tensor_backward, ts_adam_step and
 * ts_adam_zero_grad) is recorded as a HIP graph, not run -- and not counted:
 * the optimizer's counters are the same after the recording as before it.
 * Each replay runs all of it as one graph launch, and each recorded
 * ts_adam_step in it takes the bias corrections of the step count that
 * follows the optimizer's count at that moment (eager steps, other graphs and
 * earlier replays included), so any interleaving of replays and eager steps
 * gives the bits of the same steps run eagerly, and the counters advance with
 * the replays.
 * Rules:
 *  - begin refuses while the gradient map holds gradients (a recorded
 *    accumulation would add that fixed buffer again on every replay): start
 *    the recording after zero_grad and end the recorded step with zero_grad;
 *  - inside the recording nothing may wait for or read the device
 *    (ts_tensor_value / data, ts_synchronize) or upload host data
 *    (ts_tensor_from_slice): create inputs before, read results after a replay;
 *  - every buffer the recorded work touches stays reserved until the graph is
 *    freed (tensors dropped meanwhile are not reused), and a replay reads the
 *    current contents of the inputs it recorded: refill them in place
 *    (ts_tensor_device_ptr + copies) to feed new data;
 *  - link parameters to the optimizer (ts_adam_add_parameter) before the
 *    recording;
 *  - record an AMSGrad step only after the optimizer's first step; the
 *    learning rate and other settings are the recorded ones;
 *  - the profiler must be off while recording.
 * On an error inside the recording, call ts_step_graph_abort. */
int ts_step_graph_begin(void);
ts_step_graph *ts_step_graph_end(void);
void ts_step_graph_abort(void);
int ts_step_graph_recording(void);
int ts_step_graph_replay(ts_step_graph *g, size_t times);
void ts_step_graph_free(ts_step_graph *g);
/* library stream (for timing events on the stream the kernels run on) */
void *ts_stream(void);
/* device pool statistics and cache release */
size_t ts_pool_live_bytes(void);
size_t ts_pool_cached_bytes(void);
void ts_pool_empty_cache(void);

/* kernel timing with device events: class 0 GEMM (work = FLOP), 1 elementwise,
 * 2 reduction, 3 Adam (work = algorithmic bytes) */
void ts_profile_enable(int on);
/* Classes timed while profiling: bit k for class k (0 GEMM, 1 elementwise,
 * 2 reduction, 3 Adam); all by default.  Launches of the other classes record
 * no events and perturb the stream less. */
void ts_profile_classes(unsigned mask);
void ts_profile_reset(void);
int ts_profile_read(int kernel_class, double *ms, double *work, uint64_t *launches);

#ifdef __cplusplus
}
#endif
#endif /* TS_GRADTRACK_H */
