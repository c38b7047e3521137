/*
 * ts_hip.h -- C-ABI of the MI355X (gfx950) backend for train-station's
 * gradtrack training step.
 *
 * This is the drop-in replacement for the `extern "C"` block that
 * train-station binds behind its `cuda` feature
 * (train-station/src/cuda/mod.rs:139-208, implemented today by the host-only
 * stub train-station/src/cuda/cuda_wrapper.cpp:19-94).  Conventions kept from
 * that block:
 *   - buffer sizes are ELEMENT counts of f32 (cuda/memory.rs:62-76);
 *   - a NULL stream means the device's default stream (cuda/kernels.rs:37);
 *   - memcpy kinds are 0 = host->device, 1 = device->host, 2 = device->device.
 * Changed on purpose: every call returns an int status (0 = success, a HIP
 * error code, or one of the TS_HIP_E* codes below) instead of a bool, so the
 * caller can panic with a message from ts_hip_error_string().
 *
 * All tensor pointers are device pointers to contiguous row-major f32 data.
 * Launchers are asynchronous on `stream`.  They allocate nothing, with two
 * exceptions: ts_hip_gemm (and ts_hip_matmul, which calls it) takes a split-K
 * temporary from the stream-ordered allocator for few output tiles with a
 * long K, and ts_hip_gemm_fused / ts_hip_gemm_colsum (and their _xf forms)
 * given a NULL workspace take it from the same allocator.  With the caller's
 * workspace they allocate nothing, and ts_hip_gemm_noalloc (fixed device
 * array) computes ts_hip_gemm's products without allocating.
 * No torch or HIP types appear in these signatures.
 */
#ifndef TS_HIP_H
#define TS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TS_HIP_OK 0
#define TS_HIP_EINVAL 100001      /* bad argument (shape, NULL pointer, kind) */
#define TS_HIP_ENODEVICE 100002   /* no gfx950 device visible */
#define TS_HIP_EWORKSPACE 100003  /* workspace smaller than *_workspace_floats() */
#define TS_HIP_ESCRATCH 100004    /* problem needs more scratch than ts_hip_gemm_noalloc holds */

/* ---- runtime -------------------------------------------------------------- */

/* cuda_ffi_initialize (cuda/mod.rs:141): selects device 0, checks it is gfx950 */
int ts_hip_initialize(void);
/* cuda_ffi_cleanup (cuda/mod.rs:144) */
void ts_hip_cleanup(void);
/* get_cuda_device_count (cuda/mod.rs:147) */
int ts_hip_get_device_count(int *count);
/* set_cuda_device (cuda/mod.rs:150) */
int ts_hip_set_device(int device_id);
/* get_current_cuda_device (cuda/mod.rs:154) */
int ts_hip_get_device(int *device_id);
/* cuda_malloc (cuda/mod.rs:157): *ptr receives room for n_floats f32 values */
int ts_hip_malloc(float **ptr, size_t n_floats);
/* cuda_free (cuda/mod.rs:160) */
int ts_hip_free(float *ptr);
/* cuda_memcpy (cuda/mod.rs:163): synchronous copy of n_floats values */
int ts_hip_memcpy(float *dst, const float *src, size_t n_floats, int kind);
/* hipMemcpyAsync wrapper (no counterpart in the stub; required by the
 * device Allocation of tensor/core/allocation.rs:43-187) */
int ts_hip_memcpy_async(float *dst, const float *src, size_t n_floats, int kind, void *stream);
/* the same for a byte count (checkpoint records are 5 bytes per element) */
int ts_hip_memcpy_bytes(void *dst, const void *src, size_t bytes, int kind, void *stream);
/* Code objects: load a caller's gfx950 code object (hipModuleLoadData),
 * look a kernel up by name and launch it (hipModuleLaunchKernel; kernel_params
 * is an array of pointers to the arguments, as there).  This library's own
 * kernels are linked into it and need none of this; the entries complete the
 * runtime surface a host binding needs for kernels of its own (no
 * counterpart in the reference's CUDA stub, cuda/mod.rs:139-208). */
int ts_hip_module_load_data(const void *image, void **module);
int ts_hip_module_unload(void *module);
int ts_hip_module_get_function(void *module, const char *name, void **function);
int ts_hip_module_launch(void *function, unsigned grid_x, unsigned grid_y, unsigned grid_z, unsigned block_x,
                         unsigned block_y, unsigned block_z, unsigned lds_bytes, void *stream,
                         void **kernel_params);
/* pinned host memory for asynchronous device->host copies */
int ts_hip_host_malloc(void **ptr, size_t bytes);
int ts_hip_host_free(void *ptr);
/* create_cuda_stream / destroy_cuda_stream (cuda/mod.rs:166, 169); streams
 * are created non-blocking at the default priority */
int ts_hip_stream_create(void **stream);
int ts_hip_stream_destroy(void *stream);
int ts_hip_stream_synchronize(void *stream);
int ts_hip_device_synchronize(void);
/* events for timing on a stream (no counterpart in the reference) */
int ts_hip_event_create(void **event);
int ts_hip_event_destroy(void *event);
int ts_hip_event_record(void *event, void *stream);
int ts_hip_event_synchronize(void *event);
int ts_hip_event_elapsed_ms(float *ms, void *start, void *stop);
/* Kernel-attached timing (no counterpart in the reference): between begin and
 * end, every kernel this library launches from the calling thread carries the
 * two events in its own dispatch -- `start` takes the first kernel's start
 * time, `stop` each kernel's end time -- so ts_hip_event_elapsed_ms(start,
 * stop) spans the kernels alone, without the queue time of a separately
 * recorded event.  end stores how many kernels were stamped (0: the events
 * were never recorded and must not be read).  One window per thread; begin
 * while one is open replaces it. */
int ts_hip_timing_begin(void *start, void *stop);
int ts_hip_timing_end(int *kernels);
/* HIP graphs (no counterpart in the reference): work issued on `stream`
 * between begin and end is recorded, not run (relaxed capture mode: the
 * caller's other HIP calls stay legal, stream synchronisation does not), then
 * instantiated into *graph_exec; ts_hip_graph_launch runs it on a stream.  A
 * recorded launch keeps the pointers and arguments it was given. */
int ts_hip_stream_begin_capture(void *stream);
int ts_hip_stream_end_capture(void *stream, void **graph_exec);
int ts_hip_stream_is_capturing(void *stream, int *capturing);
int ts_hip_graph_launch(void *graph_exec, void *stream);
int ts_hip_graph_destroy(void *graph_exec);
/* message for a status returned by any ts_hip_* call */
const char *ts_hip_error_string(int status);
/* free / total device memory in bytes */
int ts_hip_mem_info(size_t *free_bytes, size_t *total_bytes);

/* ---- elementwise forward (bit-exact with the reference) -------------------- */

/* launch_add_kernel (cuda/mod.rs:172); ops/add.rs:276-379: out = a + b */
int ts_hip_add(const float *a, const float *b, float *out, size_t n, void *stream);
/* launch_sub_kernel (cuda/mod.rs:181); ops/sub.rs:311: out = a - b */
int ts_hip_sub(const float *a, const float *b, float *out, size_t n, void *stream);
/* launch_mul_kernel (cuda/mod.rs:190); ops/mul.rs:289-409: out = a * b */
int ts_hip_mul(const float *a, const float *b, float *out, size_t n, void *stream);
/* ops/div.rs:291-418: out = a / b (IEEE division).  The reference panics on a
 * zero divisor at indices i >= zero_check_start (32*floor(n/32) there).  If
 * zero_index is not NULL it must point to a device uint64 holding UINT64_MAX;
 * the kernel lowers it to the smallest such index (atomic min). */
int ts_hip_div(const float *a, const float *b, float *out, size_t n,
               size_t zero_check_start, unsigned long long *zero_index, void *stream);
/* ops/{add,sub,mul,div}.rs scalar variants: out = x op s */
int ts_hip_add_scalar(const float *x, float s, float *out, size_t n, void *stream);
int ts_hip_sub_scalar(const float *x, float s, float *out, size_t n, void *stream);
int ts_hip_mul_scalar(const float *x, float s, float *out, size_t n, void *stream);
int ts_hip_div_scalar(const float *x, float s, float *out, size_t n, void *stream);
/* core/utils.rs:802-871 negate_inplace: out = 0 - x for i < tail_start,
 * -x after (tail_start = 8*floor(n/8) reproduces the reference). out may be x. */
int ts_hip_neg(const float *x, float *out, size_t n, size_t tail_start, void *stream);
/* ops/relu.rs:117-273: out = x > 0 ? x : +0 */
int ts_hip_relu(const float *x, float *out, size_t n, void *stream);
/* ops/pow.rs:79-236 pow_scalar: e == 2 -> x*x, e == 0.5 -> sqrt(x), else powf */
int ts_hip_pow_scalar(const float *x, float e, float *out, size_t n, void *stream);
/* ops/add.rs:106-146 with ops/broadcasting.rs:299-478, the row broadcast
 * [rows,cols] + [cols]: out[r][c] = x[r][c] + bias[c] (bias[c] + x[r][c] when
 * bias_first), without materialising the broadcast bias. */
int ts_hip_bias_add(const float *x, const float *bias, float *out, size_t rows, size_t cols,
                    int bias_first, void *stream);
/* Row broadcast for the other binary ops (ops/{sub,mul,div}.rs broadcast
 * paths): op 0 add, 1 sub, 2 mul, 3 div.  out[r][c] = x[r][c] op v[c], or
 * v[c] op x[r][c] when vec_first.  For div, zero_index as in ts_hip_div over
 * the flat [rows*cols] index from zero_check_start on. */
int ts_hip_row_broadcast(int op, const float *x, const float *v, float *out, size_t rows,
                         size_t cols, int vec_first, size_t zero_check_start,
                         unsigned long long *zero_index, void *stream);
/* init/basic.rs:136-326 zeros/ones/fill: out[i] = value */
int ts_hip_fill(float *out, float value, size_t n, void *stream);
/* Tensor::randn / fill_randn with Some(seed) (init/random.rs:231-299,
 * XorShiftRng :453-615): out[i] = Box-Muller of draws 2i+1 and 2i+2 of
 * xorshift64(13,7,17) from `seed`, generated on the device.  ln and cos are
 * correctly rounded (the reference takes them from the host libm's logf /
 * cosf).  n == 0 is a no-op; n must not exceed 2^62. */
int ts_hip_randn(float *out, size_t n, uint64_t seed, void *stream);

/* Checkpoint encoding of a Tensor's data as the reference's binary format
 * stores a Vec<f32> (serialization/core/impls.rs:278-288 makes it an Array
 * of F32 values; binary/structs.rs:193-196 writes each as the type tag 10 and
 * the f32 bits little-endian): dst receives 5*n bytes, record i =
 * [10][bits of src[i], LE].  src 16-byte aligned, dst 4-byte aligned. */
int ts_hip_encode_f32_records(const float *src, size_t n, void *dst, void *stream);
/* The inverse (binary/structs.rs:395-398 reads tag 10 + f32).  When
 * bad_index is not NULL, the index of the first record whose tag is not 10 is
 * folded into *bad_index with a minimum (the caller sets it to ~0 first).
 * src 4-byte aligned, dst 16-byte aligned. */
int ts_hip_decode_f32_records(const void *src, size_t n, float *dst, unsigned long long *bad_index,
                              void *stream);
/* Fill from a device scalar without a host round trip (the upstream gradient
 * of a scalar loss): out[i] = src[0] (grad_fn/reductions/sum.rs:4-16), or
 * multiplier * src[0] when use_multiplier (grad_fn/reductions/mean.rs:4-30). */
int ts_hip_fill_from_device(float *out, const float *src, float multiplier, int use_multiplier,
                            size_t n, void *stream);
/* Tensor::clone for contiguous data (core/mod.rs:344-355) */
int ts_hip_copy(const float *src, float *dst, size_t n, void *stream);

/* ---- other recorded ops (tensor/ops/{exp,log,sqrt,tanh,sigmoid,leaky_relu,
 * softmax}.rs) ------------------------------------------------------------- */

/* out = exp(x), ln(x), tanh(x): correctly rounded (the reference calls the
 * host libm's expf / logf / tanhf, which agree except in the last place on a
 * small share of inputs) */
int ts_hip_exp(const float *x, float *out, size_t n, void *stream);
int ts_hip_log(const float *x, float *out, size_t n, void *stream);
int ts_hip_tanh(const float *x, float *out, size_t n, void *stream);
/* out = sqrt(x), correctly rounded as in the reference (bit-exact) */
int ts_hip_sqrt(const float *x, float *out, size_t n, void *stream);
/* sigmoid.rs:9-21: x >= 0 ? 1 / (1 + exp(-x)) : exp(x) / (1 + exp(x)) */
int ts_hip_sigmoid(const float *x, float *out, size_t n, void *stream);
/* leaky_relu.rs: x > 0 ? x : negative_slope * x (bit-exact) */
int ts_hip_leaky_relu(const float *x, float negative_slope, float *out, size_t n, void *stream);
/* softmax along an axis of a tensor viewed as [outer, reduce, inner]
 * (softmax.rs:4-60): per slice max, exp(x - max), sequential fp32 sum,
 * times 1/sum.  reduce must be > 0 when outer*inner > 0. */
int ts_hip_softmax(const float *x, float *y, size_t outer, size_t reduce, size_t inner, void *stream);

/* ---- broadcasting and axis sums (ops/broadcasting.rs:299-478,
 * reductions/{sum,mean}.rs sum_dims / mean_dims, grad_fn/utils.rs:23-60) ---- */

#define TS_HIP_MAX_RANK 8
/* out (out_dims) = src (src_dims) broadcast NumPy-style: source axes align to
 * the right, axes of size 1 (or missing) repeat; times scale when use_scale.
 * Dims arrays are host memory; ranks up to TS_HIP_MAX_RANK. */
int ts_hip_broadcast_copy(const float *src, const size_t *src_dims, size_t src_rank, float *out,
                          const size_t *out_dims, size_t out_rank, float scale, int use_scale,
                          void *stream);
/* transform/transpose.rs:156-208 and contiguous.rs:123-157 (the reference's
 * strided view, materialised): out = src (dims, rank) with axes d0 and d1
 * swapped, both row-major; d0 == d1 copies.  A matrix operand of a product
 * is never transposed this way: the GEMM entries read it transposed. */
int ts_hip_transpose(const float *src, const size_t *dims, size_t rank, size_t d0, size_t d1, float *out,
                     void *stream);
/* Sum of x (dims, rank) over the axes whose bit is set in reduce_mask, into
 * out laid out with those axes of size 1 (keepdim); f64 accumulation in a
 * fixed order, rounded once, then times scale (fp32) when use_scale. */
int ts_hip_reduce_sum(const float *x, const size_t *dims, size_t rank, unsigned reduce_mask, float *out,
                      float scale, int use_scale, void *stream);

/* ---- elementwise backward -------------------------------------------------- */

/* grad_fn/ops/relu.rs:4-17: gi = x > 0 ? go : 0.  A saved relu OUTPUT may be
 * passed as x: relu(x) > 0 exactly when x > 0. */
int ts_hip_relu_backward(const float *x, const float *go, float *gi, size_t n, void *stream);
/* grad_fn/ops/pow.rs:5-27: gi = go * (e * powf(x, e - 1)) (0 when e == 0) */
int ts_hip_pow_backward(const float *x, const float *go, float *gi, size_t n, float e,
                        void *stream);
/* grad_fn/ops/mul.rs:4-49 same-shape case in one pass: ga = go*b, gb = go*a.
 * Either output may be NULL. */
int ts_hip_mul_backward(const float *go, const float *a, const float *b, float *ga, float *gb,
                        size_t n, void *stream);
/* grad_fn/ops/div.rs:4-49 same-shape case in one pass:
 *   ga = go / b;   gb = neg((go * a) / (b * b))   (neg as in ts_hip_neg)
 * zero_index as in ts_hip_div, covering both divisions of the reference
 * (divisor b, then b*b) from zero_check_start on.  Either output may be NULL. */
int ts_hip_div_backward(const float *go, const float *a, const float *b, float *ga, float *gb,
                        size_t n, size_t tail_start, size_t zero_check_start,
                        unsigned long long *zero_index, void *stream);

/* grad_fn/ops/log.rs: go * (1 / x), from the saved input x */
int ts_hip_log_backward(const float *x, const float *go, float *gi, size_t n, void *stream);
/* grad_fn/ops/sqrt.rs: go * ((1 / y) * 0.5), from the saved output y */
int ts_hip_sqrt_backward(const float *y, const float *go, float *gi, size_t n, void *stream);
/* grad_fn/ops/tanh.rs: go * (1 - y*y), from the saved output y */
int ts_hip_tanh_backward(const float *y, const float *go, float *gi, size_t n, void *stream);
/* grad_fn/ops/sigmoid.rs: go * y * (1 - y), from the saved output y */
int ts_hip_sigmoid_backward(const float *y, const float *go, float *gi, size_t n, void *stream);
/* grad_fn/ops/leaky_relu.rs: x > 0 ? go : negative_slope * go */
int ts_hip_leaky_relu_backward(const float *x, const float *go, float *gi, size_t n, float negative_slope,
                               void *stream);
/* grad_fn/ops/softmax.rs:4-38: per slice dot = sequential sum of go*y, then
 * gi = y * (go - dot).  (exp's backward is ts_hip_mul(go, y).) */
int ts_hip_softmax_backward(const float *y, const float *go, float *gi, size_t outer, size_t reduce,
                            size_t inner, void *stream);

/* ---- fused elementwise programs (no counterpart in the reference, which runs
 * every op as its own pass) ---------------------------------------------------
 * One pass evaluates a short program of the elementwise ops above over up to
 * TS_HIP_MAP_MAX_INPUTS inputs of n elements (or one value used for every
 * element: bit k of scalar_inputs reads inputs[k][0]; bit k of const_inputs
 * takes const_values[k], and inputs[k] is not read) and stores up to
 * TS_HIP_MAP_MAX_OUTPUTS of its values.  The pass has TS_HIP_MAP_REGS
 * registers per element: registers 0 .. n_inputs-1 start with the inputs; op k
 * reads registers a and b and writes register d (any register, an input's or
 * an earlier op's included: the op reads its operands first), so a program of
 * up to TS_HIP_MAP_MAX_OPS ops fits the file when its values' lifetimes do
 * (every register read must have been written, by the inputs or an earlier
 * op).  Outputs and the summed register are read after the last op.  Each op's
 * formula and fp32 operation order is that of the separate
 * kernel of the same op, so every stored value has the bits the op-by-op
 * sequence gives:
 *   ADD a+b, SUB a-b, MUL a*b, DIV a/b (with flags & TS_HIP_MAP_CHECKED the
 *   divisor is checked as ts_hip_div does, from zero_check_start on, into
 *   zero_index), NEG (0-a before tail_start, -a after: ts_hip_neg), RELU,
 *   RELU_BWD (a > 0 ? b : +0: ts_hip_relu_backward with a the saved value, b
 *   the gradient), ADD_S / SUB_S / MUL_S / DIV_S (a op imm), SQUARE (a*a).
 * A constant input is the value ts_hip_fill would write into a buffer read in
 * its place.  With sum_out != NULL, register reduce_reg is also added up into
 * sum_out[0] (divided by (float)n when mean) with the bits ts_hip_sum /
 * ts_hip_mean give over a 16-byte-aligned buffer holding those values (the
 * pass groups by four whatever its outputs' alignment; ts_hip_sum over an
 * unaligned buffer adds element by element); the workspace is
 * ts_hip_map_workspace_floats(n) floats, 8-byte aligned. */
#define TS_HIP_MAP_MAX_INPUTS 5
#define TS_HIP_MAP_MAX_OPS 24
#define TS_HIP_MAP_MAX_OUTPUTS 4
#define TS_HIP_MAP_REGS 16
#define TS_HIP_MAP_CHECKED 1
enum {
    TS_HIP_MAP_ADD = 0, TS_HIP_MAP_SUB = 1, TS_HIP_MAP_MUL = 2, TS_HIP_MAP_DIV = 3, TS_HIP_MAP_NEG = 4,
    TS_HIP_MAP_RELU = 5, TS_HIP_MAP_RELU_BWD = 6, TS_HIP_MAP_ADD_S = 7, TS_HIP_MAP_SUB_S = 8,
    TS_HIP_MAP_MUL_S = 9, TS_HIP_MAP_DIV_S = 10, TS_HIP_MAP_SQUARE = 11
};
typedef struct ts_hip_map_op {
    uint8_t code, a, b, flags;
    float imm;
    uint8_t d; /* destination register */
} ts_hip_map_op;
typedef struct ts_hip_map_program {
    const float *inputs[TS_HIP_MAP_MAX_INPUTS];
    uint32_t scalar_inputs, n_inputs, n_ops, n_outputs;
    ts_hip_map_op ops[TS_HIP_MAP_MAX_OPS];
    float *outputs[TS_HIP_MAP_MAX_OUTPUTS];
    uint8_t output_regs[TS_HIP_MAP_MAX_OUTPUTS];
    int32_t reduce_reg;
    uint32_t const_inputs;
    float const_values[TS_HIP_MAP_MAX_INPUTS];
} ts_hip_map_program;
size_t ts_hip_map_workspace_floats(size_t n);
int ts_hip_map(const ts_hip_map_program *prog, size_t n, size_t tail_start, size_t zero_check_start,
               unsigned long long *zero_index, float *sum_out, int mean, float *workspace, size_t workspace_floats,
               void *stream);
/* Compiled programs (no counterpart in the reference).  ts_hip_map runs a
 * program whose operands are all 16-byte aligned as a kernel compiled at run
 * time for its shape -- its ops, registers, inputs read per element, stored
 * values and reduction; not the pointers, constants or immediates -- with the
 * interpreter's loop and fp32 operations written out as straight-line code
 * (hipRTC, the library's numerics flags), so with the same bits; compiled
 * kernels are cached for the process, per device.  mode 0: never; 1: from a
 * shape's second use (the default); 2: from its first.  Returns the previous
 * mode, or -1 for a bad one.  A shape whose compilation fails runs
 * interpreted, counted in *failed, with the compiler's log in
 * ts_hip_map_jit_log(). */
int ts_hip_map_jit_mode(int mode);
int ts_hip_map_jit_stats(size_t *compiled, size_t *failed);
const char *ts_hip_map_jit_log(void);
/* The source compiled for a program with its operands aligned (reduce: with
 * its sum), NUL-terminated into buf (at most cap bytes); returns its length
 * + 1, or 0 for a malformed program. */
size_t ts_hip_map_jit_source(const ts_hip_map_program *prog, int reduce, char *buf, size_t cap);

/* ---- reductions ------------------------------------------------------------- */

/* Workspace (device floats) needed by ts_hip_sum / ts_hip_mean for n inputs. */
size_t ts_hip_sum_workspace_floats(size_t n);
/* reductions/sum.rs:80-141: out[0] = sum(x).  Deterministic two-pass tree with
 * f64 partials (not the reference's sequential fp32 order; within 1e-4). */
int ts_hip_sum(const float *x, size_t n, float *out, float *workspace, size_t workspace_floats,
               void *stream);
/* reductions/mean.rs:48-109: out[0] = sum(x) / (float)n */
int ts_hip_mean(const float *x, size_t n, float *out, float *workspace, size_t workspace_floats,
                void *stream);
/* Workspace (device floats) needed by ts_hip_sum_dim0 for [rows,cols]: one
 * f64 sum per 64-row chunk and column, 2 * ceil(rows/64) * cols floats, so it
 * grows with the row count (32 MiB for [2^24, 16]). */
size_t ts_hip_sum_dim0_workspace_floats(size_t rows, size_t cols);
/* reductions/sum.rs:225-306 sum_dims(&[0]) on [rows,cols] -> [cols]; the
 * bias-gradient column reduction of grad_fn/utils.rs:23-60.  Fixed order:
 * chunks of 64 rows, each added row by row in f64 from +0; groups of 8
 * consecutive chunk sums, each added in chunk order in f64 from +0; the group
 * sums added in group order in f64 from +0; rounded to fp32 once (not the
 * reference's fp32 row order; within 1e-4 of it, within f64 rounding of the
 * exact sum).  The last sum is one dependent add per group of 512 rows. */
int ts_hip_sum_dim0(const float *x, size_t rows, size_t cols, float *out, float *workspace,
                    size_t workspace_floats, void *stream);

/* ---- contractions (fp32 MFMA) ------------------------------------------------ */

/* launch_matmul_kernel (cuda/mod.rs:199): row-major C[m,n] = A[m,k] . B[k,n] */
int ts_hip_matmul(const float *a, const float *b, float *c, size_t m, size_t n, size_t k,
                  void *stream);
/* General form used by matmul forward and backward (ops/matmul/mod.rs:572-611,
 * grad_fn/ops/matmul.rs:68-80) with the transposes folded into the operand
 * loads instead of the reference's t().contiguous() copies:
 *   C[M,N] = op(A)[M,K] . op(B)[K,N]
 *   trans_a == 0: A(i,k) = A[i*lda + k]   (A stored [M][lda])
 *   trans_a == 1: A(i,k) = A[k*lda + i]   (A stored [K][lda], i.e. A^T view)
 *   trans_b == 0: B(k,j) = B[k*ldb + j]   (B stored [K][ldb])
 *   trans_b == 1: B(k,j) = B[j*ldb + k]   (B stored [N][ldb], i.e. B^T view)
 *   C(i,j) = C[i*ldc + j]
 * fp32 inputs, fp32 MFMA accumulation (v_mfma_f32_16x16x4_f32 when M and N
 * are multiples of 256, K of 32 and the grid has a 256x256 tile per CU; else
 * v_mfma_f32_32x32x2_f32: the two add k in different groupings, so a product's
 * last bits depend on which it takes; every entry point below takes the same
 * one for the same shape, layout and alignment).  M, N, K and
 * the leading dimensions must be below 2^31 (TS_HIP_EINVAL otherwise).  For
 * few output tiles with a long K (e.g. M = 32, K = 784) the call splits K and
 * takes a temporary of up to 16*M*N floats from the stream-ordered allocator
 * (hipMallocAsync / hipFreeAsync on `stream`); where that allocator is
 * unavailable it runs unsplit. */
int ts_hip_gemm(int trans_a, int trans_b, size_t M, size_t N, size_t K, const float *A,
                size_t lda, const float *B, size_t ldb, float *C, size_t ldc, void *stream);

/* ts_hip_gemm without any allocation.  No counterpart in the reference: for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments,
 * kernels and results (bit for bit) as ts_hip_gemm; a split product's
 * temporary comes from a fixed device array of 2^21 floats (8 MiB) that each
 * device holds for the life of the process, which every split this device
 * can choose fits (a product needing more returns TS_HIP_ESCRATCH).  The
 * array is shared by all calls on a device: calls that overlap on one device
 * (on several streams) race and must be serialised by the caller. */
int ts_hip_gemm_noalloc(int trans_a, int trans_b, size_t M, size_t N, size_t K, const float *A,
                        size_t lda, const float *B, size_t ldb, float *C, size_t ldc, void *stream);

/* Floats of workspace a split product needs (the temporary ts_hip_gemm takes
 * from the stream-ordered allocator for few output tiles with a long K):
 * 0 when the product M x N x K is not split. */
size_t ts_hip_gemm_workspace_floats(size_t M, size_t N, size_t K);

/* The same product with the elementwise ops that follow it fused into the
 * store (no counterpart in the reference, which runs them as separate passes:
 * matmul then add_tensor with a broadcast row bias, ops/add.rs:276-379, then
 * relu, ops/relu.rs:77-273; or the product then relu's backward,
 * grad_fn/ops/relu.rs:4-17).  Per output element, in this order:
 *   v = op(A) . op(B) as ts_hip_gemm computes it;
 *   bias != NULL:  v = v + bias[j]              (bias: N floats)
 *   relu != 0:     v = v > 0 ? v : +0
 *   mask != NULL:  v = mask[i*ldc + j] > 0 ? v : +0   (mask laid out as C)
 *   C[i*ldc + j] = v
 * Bit-identical to ts_hip_gemm followed by ts_hip_bias_add, ts_hip_relu and
 * ts_hip_relu_backward(mask, C, C).  A split product (see
 * ts_hip_gemm_workspace_floats) uses `workspace` (device, at least that many
 * floats; TS_HIP_EWORKSPACE if fewer) as its temporary, so the call allocates
 * nothing and can be recorded into a HIP graph; with workspace == NULL it
 * allocates as ts_hip_gemm does. */
int ts_hip_gemm_fused(int trans_a, int trans_b, size_t M, size_t N, size_t K, const float *A, size_t lda,
                      const float *B, size_t ldb, const float *bias, int relu, const float *mask, float *C,
                      size_t ldc, float *workspace, size_t workspace_floats, void *stream);

/* ts_hip_gemm_fused with a subtraction in the epilogue (no counterpart in
 * the reference, whose MSE subtracts the target in a pass of its own:
 * feedforward_network.rs:478-479 through ops/sub.rs's sub_tensor of
 * same-shape tensors).  Per output element, after the bias:
 *   v = v - sub[i*ldc + j]   (sub laid out as C)
 * then relu and mask as in ts_hip_gemm_fused: the bits of ts_hip_gemm_fused
 * (bias only) followed by ts_hip_sub, then the rest.  Only for products that
 * ts_hip_gemm_takes_sub accepts (the one-pass narrow kernel: at most 16
 * output columns, or few output tiles and a long K); TS_HIP_EINVAL otherwise.
 * Allocates nothing. */
int ts_hip_gemm_takes_sub(int trans_a, int trans_b, size_t M, size_t N, size_t K);
int ts_hip_gemm_fused_sub(int trans_a, int trans_b, size_t M, size_t N, size_t K, const float *A, size_t lda,
                          const float *B, size_t ldb, const float *bias, const float *sub, int relu,
                          const float *mask, float *C, size_t ldc, void *stream);

/* The weight gradient of a linear layer together with its bias gradient (no
 * counterpart in the reference, which reduces the bias gradient in a pass of
 * its own: grad_fn/ops/add.rs:4-28 through reduce_gradient_to_shape,
 * grad_fn/utils.rs:23-60, i.e. sum_dims(&[0]) of reductions/sum.rs:225-306):
 *   C[M,N] = op(A)[M,K] . B[K,N]   as ts_hip_gemm(trans_a, 0, ...) computes it
 *   colsum[n] = sum over k of B[k*ldb + n]   with the bits of ts_hip_sum_dim0
 * With trans_a == 1 (dW = X^T . dY) the product's own launch adds B's
 * columns: from the B tiles it stages (large aligned products, then a short
 * combine pass), from workgroups appended to its grid (register-staged tiles),
 * or from the rows its first workgroup holds (N <= 16); other shapes take a
 * column-sum pass after the product.  M == 0 gives the column sums alone.
 * Workspace as ts_hip_gemm_colsum_workspace_floats (8-byte aligned; NULL:
 * taken from the stream-ordered allocator, whose error is returned when it
 * cannot give it: hipErrorOutOfMemory for a full device). */
size_t ts_hip_gemm_colsum_workspace_floats(int trans_a, size_t M, size_t N, size_t K);
int ts_hip_gemm_colsum(int trans_a, size_t M, size_t N, size_t K, const float *A, size_t lda, const float *B,
                       size_t ldb, float *C, size_t ldc, float *colsum, float *workspace, size_t workspace_floats,
                       void *stream);

/* Operand transforms (no counterpart in the reference, which stores the
 * elementwise op's result and then multiplies it: e.g. relu's backward,
 * grad_fn/ops/relu.rs:4-17, or the MSE's gradient, grad_fn/ops/pow.rs:5-27,
 * before the matmul backward of grad_fn/ops/matmul.rs:68-80).  A
 * ts_hip_operand_xf is applied to each element of its operand as the product
 * loads it: n_ops ops in order, each x = op(x, imm[i]) as one fp32 operation
 * with the bits of the elementwise kernel of that op:
 *   ADD_S x+imm, SUB_S x-imm, MUL_S x*imm, DIV_S x/imm, RSUB_S imm-x,
 *   RDIV_S imm/x, RELU (x > 0 ? x : +0), RELU_BWD_S (x > 0 ? imm : +0: relu's
 *   backward with a gradient of imm everywhere), SQUARE (x*x).
 * The chain must map +0 to +0 (the zeros that pad a k tile stay zeros);
 * TS_HIP_EINVAL otherwise.  The product, its epilogue and its column sums
 * then have the bits of the same call on an operand holding the transformed
 * values.  Only the kernels of products that ts_hip_gemm_takes_xf accepts
 * apply transforms (register-staged tiles, few-column and one-k-tile
 * kernels: products with fewer than one 256x256 tile per compute unit and
 * no split of K); the _xf calls refuse the rest with TS_HIP_EINVAL.  xa / xb
 * NULL: no transform of that operand. */
#define TS_HIP_XF_MAX_OPS 4
enum {
    TS_HIP_XF_ADD_S = 0, TS_HIP_XF_SUB_S = 1, TS_HIP_XF_MUL_S = 2, TS_HIP_XF_DIV_S = 3, TS_HIP_XF_RSUB_S = 4,
    TS_HIP_XF_RDIV_S = 5, TS_HIP_XF_RELU = 6, TS_HIP_XF_RELU_BWD_S = 7, TS_HIP_XF_SQUARE = 8
};
typedef struct ts_hip_operand_xf {
    uint32_t n_ops;
    uint8_t code[TS_HIP_XF_MAX_OPS];
    float imm[TS_HIP_XF_MAX_OPS];
} ts_hip_operand_xf;
int ts_hip_gemm_takes_xf(int trans_a, int trans_b, size_t M, size_t N, size_t K, int colsum);
int ts_hip_gemm_fused_xf(int trans_a, int trans_b, size_t M, size_t N, size_t K, const float *A, size_t lda,
                         const ts_hip_operand_xf *xa, const float *B, size_t ldb, const ts_hip_operand_xf *xb,
                         const float *bias, int relu, const float *mask, float *C, size_t ldc, float *workspace,
                         size_t workspace_floats, void *stream);
int ts_hip_gemm_colsum_xf(int trans_a, size_t M, size_t N, size_t K, const float *A, size_t lda,
                          const ts_hip_operand_xf *xa, const float *B, size_t ldb, const ts_hip_operand_xf *xb,
                          float *C, size_t ldc, float *colsum, float *workspace, size_t workspace_floats,
                          void *stream);

/* ts_hip_gemm_colsum_xf with ldb == N that also adds up B as stored, each
 * value put through xs first (NULL: none; the ops and fp32 semantics of
 * ts_hip_operand_xf), in the same launch (no counterpart in the reference,
 * which sums the loss in a pass of its own, reductions/sum.rs:80-141 and
 * reductions/mean.rs:48-109, before its backward reads the same values: the
 * README step's relu(x W + b).sum(), README.md:71-79, whose weight gradient
 * reads relu's output through relu's backward, or an MSE's mean of d * d,
 * feedforward_network.rs:478-479, whose last weight gradient reads d):
 *   bsum[0] = the sum of xs(B)'s K*N values, divided by (float)(K*N) when
 *   mean, with the bits of ts_hip_sum / ts_hip_mean over those values,
 * from one workgroup appended to the product's grid.  Only where
 * ts_hip_gemm_takes_bsum accepts (trans_a == 1; the products whose column
 * sums come from the product's own launch with no workspace -- the
 * register-staged tiles, or the narrow kernel at its widest workgroups,
 * K >= 1024; K*N <= 16384), with B 16-byte aligned; TS_HIP_EINVAL otherwise.
 * Allocates nothing. */
int ts_hip_gemm_takes_bsum(int trans_a, size_t M, size_t N, size_t K);
int ts_hip_gemm_colsum_bsum(int trans_a, size_t M, size_t N, size_t K, const float *A, size_t lda,
                            const ts_hip_operand_xf *xa, const float *B, const ts_hip_operand_xf *xb, float *C,
                            size_t ldc, float *colsum, const ts_hip_operand_xf *xs, float *bsum, int mean,
                            void *stream);

/* Launch groups (no counterpart in the reference, whose matmul backward,
 * grad_fn/ops/matmul.rs:68-80, runs its two products one after the other).
 * Between ts_hip_launch_group_begin(stream) and ts_hip_launch_group_end(stream)
 * the calling thread's products on `stream` that take the narrow kernel (few
 * output columns: ts_hip_gemm_takes_sub, or the column-sum / bsum forms there)
 * or the one-k-tile kernel (K <= 16) are held, at most two; any other work on
 * the stream -- another launch, a copy, an event, a synchronisation -- runs
 * them first, in the order they were issued.  At the end one of each runs as
 * one launch, their workgroups side by side, when the pair is one the library
 * builds (an MLP backward's dW with its bias gradient and, at its widest
 * workgroups, K >= 1024, its dX with relu's backward mask); otherwise what is
 * held is launched as issued.  Same results either way.  The products of a
 * group must not read each other's outputs (the caller's contract: a matmul
 * backward's dX and dW read only the forward's values and the incoming
 * gradient).  Entry points called inside a group return TS_HIP_OK for a held
 * launch; errors of the launch come from _end.  One group per thread at a
 * time: _begin inside an open group and _end on another stream are
 * TS_HIP_EINVAL.  Allocates nothing. */
int ts_hip_launch_group_begin(void *stream);
int ts_hip_launch_group_end(void *stream);

/* Batched C[b] = op(A[b]) . op(B[b]) (matmul/mod.rs:634-760 batched_matmul and
 * the batched backward of grad_fn/ops/matmul.rs:150-219) on the same MFMA
 * tiles: a batch grid of batch_rank axes (<= 6) with sizes batch_dims; the A /
 * B matrices of batch coordinate c start at sum_k c_k * a_batch_strides[k]
 * (resp. b_...) elements -- 0 on an axis the operand broadcasts -- and the C
 * matrices are c_batch_stride elements apart, in row-major batch order. */
int ts_hip_gemm_batched(int trans_a, int trans_b, size_t M, size_t N, size_t K, const float *A, size_t lda,
                        const float *B, size_t ldb, float *C, size_t ldc, size_t batch_rank,
                        const size_t *batch_dims, const size_t *a_batch_strides, const size_t *b_batch_strides,
                        size_t c_batch_stride, void *stream);
/* Vector cases (matmul/mod.rs:332-632): trans 0: y[r] = sum_c A[r][c] x[c]
 * (matrix . vector); trans 1: y[c] = sum_r x[r] A[r][c] (vector . matrix, and
 * the backward of matrix . vector).  A is [rows, cols] row-major (lda == cols
 * for trans 1); f64 accumulation.  trans 1 needs the workspace of
 * ts_hip_gemv_workspace_floats (8-byte aligned). */
size_t ts_hip_gemv_workspace_floats(int trans, size_t rows, size_t cols);
int ts_hip_gemv(int trans, size_t rows, size_t cols, const float *A, size_t lda, const float *x, float *y,
                float *workspace, size_t workspace_floats, void *stream);
/* 1-D . 1-D (matmul/mod.rs:310-350 dot_product_1d): out[0] = sum a[i]*b[i],
 * f64 accumulation; workspace as ts_hip_sum_workspace_floats(n) */
int ts_hip_dot(const float *a, const float *b, size_t n, float *out, float *workspace, size_t workspace_floats,
               void *stream);
/* out[i][j] = a[i] * b[j] (grad_fn/ops/matmul.rs compute_outer_product, fp32) */
int ts_hip_outer(const float *a, size_t m, const float *b, size_t n, float *out, void *stream);

/* ---- optimizer ------------------------------------------------------------------ */

/* optimizers/adam/mod.rs:485-1007, one parameter, fused into one pass that
 * reads p, g, m, v once and writes p, m, v once.  step_count is the
 * optimizer's global count after its increment (:1036-1044); the bias
 * corrections are computed on the host exactly as :524-531 (f64 powf, cast to
 * f32, 1.0f/bc).  Per element, in the reference's fp32 order:
 *   m = b1*m + (1-b1)*g
 *   v = b2*v + (1-b2)*(g*g)       i <  tail_start (AVX2 body)
 *   v = b2*v + ((1-b2)*g)*g       i >= tail_start (scalar tail)
 *   p = p - (lr*(m*cf1)) / (sqrt(v*cf2) + eps)
 * tail_start = 8*floor(n/8) reproduces the reference.  weight_decay > 0
 * first forms g + weight_decay*p (adam/mod.rs:511-518).  AMSGrad
 * (:534-541): when v_hat_max is not NULL it is set to v*cf2 on the
 * parameter's first step (amsgrad_first != 0), else to
 * (v_hat_max > v*cf2 ? v_hat_max : v*cf2), and the update uses it. */
int ts_hip_adam_step(float *p, const float *g, float *m, float *v, float *v_hat_max, size_t n,
                     float lr, float beta1, float beta2, float eps, float weight_decay,
                     uint64_t step_count, size_t tail_start, int amsgrad_first, void *stream);

/* One parameter of a multi-tensor Adam launch (fields as in ts_hip_adam_step;
 * the tail rule is the reference's, tail_start = 8*floor(n/8)). */
typedef struct ts_hip_adam_param {
    float *p;
    const float *g;
    float *m;
    float *v;
    float *v_hat_max; /* NULL unless AMSGrad */
    size_t n;
    int amsgrad_first;
} ts_hip_adam_param;

#define TS_HIP_ADAM_MAX_PARAMS 16

/* Optimizer::step over up to TS_HIP_ADAM_MAX_PARAMS parameters in one launch
 * (adam/mod.rs:1036-1044 steps them one after another; they are independent,
 * so one launch gives the same bits).  Larger counts: call once per group of
 * 16 with the same step_count. */
int ts_hip_adam_step_multi(const ts_hip_adam_param *params, size_t count, float lr, float beta1,
                           float beta2, float eps, float weight_decay, uint64_t step_count,
                           void *stream);

/* The same step with its bias corrections read on the device: pair s = *slot
 * of `bias_corrections` (device memory, [cf1, cf2] pairs as
 * ts_hip_adam_bias_corrections computes them), so one recorded step replays at
 * later step counts (no counterpart in the reference, which steps eagerly). */
int ts_hip_adam_step_multi_table(const ts_hip_adam_param *params, size_t count, float lr, float beta1,
                                 float beta2, float eps, float weight_decay, const float *bias_corrections,
                                 const unsigned *slot, void *stream);
/* The same with self-advancing replay counters (no counterpart in the
 * reference): tickets holds one uint32 per wave of the launch
 * (ts_hip_adam_multi_waves of the same list; device memory, 4-byte aligned,
 * zero before the first launch); wave w adds 1 to tickets[w] and uses pair
 * s = its value before the add, so the r-th launch since the tickets were
 * cleared uses pair r with no counter-advancing launch of its own.  Launches
 * that share tickets must run one after another (one stream) with the same
 * parameter sizes and alignments. */
size_t ts_hip_adam_multi_waves(const ts_hip_adam_param *params, size_t count);
int ts_hip_adam_step_multi_ticket(const ts_hip_adam_param *params, size_t count, float lr, float beta1,
                                  float beta2, float eps, float weight_decay, const float *bias_corrections,
                                  unsigned *tickets, void *stream);
/* Host: the bias corrections of steps first_step .. first_step + count - 1 as
 * ts_hip_adam_step_multi computes them (adam/mod.rs:524-531, bias_correct
 * :790-833): out[2i] = 1 / (1 - beta1^t), out[2i+1] = 1 / (1 - beta2^t), the
 * power in f64, the rest in f32. */
int ts_hip_adam_bias_corrections(float beta1, float beta2, uint64_t first_step, size_t count, float *out);
/* *slot += 1, in stream order (the replay counter of a recorded step) */
int ts_hip_slot_advance(unsigned *slot, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* TS_HIP_H */
