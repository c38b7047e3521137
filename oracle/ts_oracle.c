/*
 * ts_oracle.c -- CPU restatement of train-station's gradtrack hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker or as the reported CPU baseline.  The product path never calls it.
 *
 * Every function restates the arithmetic of one reference function in the
 * same fp32 operation order (IEEE binary32, round-to-nearest-even, no FMA
 * contraction: the file is compiled with -ffp-contract=off).  Citations are
 * paths under train-station/src/ of the reference.
 *
 * Pinning (how each function is checked independently of this file):
 *   elementwise (add/sub/mul/div/scalar/relu/pow2/bias_add): bit-exact against
 *       torch CPU fp32 on random and special values, plus the reference's own
 *       known answers (relu.rs:281, pow.rs:547, add.rs:893);
 *   neg: IEEE special values of the two formulas (0-x on the 8-wide body,
 *       -x on the tail), utils.rs:847-870;
 *   relu_bwd / pow_bwd / mul / div backward: torch autograd (float64) on the
 *       same graphs, plus matmul/mod.rs:1145-1195 known answers;
 *   sum / mean / sum_dim0: reference known answers (sum.rs:314-420,
 *       mean.rs:238-320), math.fsum error bounds and an engineered vector
 *       whose value depends on the 4-wide grouping of sum.rs:94-105;
 *   gemm_f64: reference matmul known answers, brute force on tiny shapes,
 *       torch float64 matmul on all three operand layouts;
 *   adam_step: torch.optim.Adam (float64) on the reference's own LibTorch
 *       validation cases incl. weight decay and AMSGrad (ltv/src/validation/optimizers/adam.rs:65-160) and
 *       on 100 random steps; closed form for constant gradients.
 *   parity unpinned: the exact bits of the bias-correction scalars depend on
 *       the host libm's f64 pow, as in the reference (adam/mod.rs:526-531).
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

/* ---- elementwise forward ------------------------------------------------ */

/* ops/add.rs:276-379 : out[i] = a[i] + b[i] (AVX2 body and tail identical) */
EXPORT void o_add(const float *a, const float *b, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

/* ops/sub.rs:311-... : out[i] = a[i] - b[i] */
EXPORT void o_sub(const float *a, const float *b, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = a[i] - b[i];
}

/* ops/mul.rs:289-409 : out[i] = a[i] * b[i] */
EXPORT void o_mul(const float *a, const float *b, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = a[i] * b[i];
}

/* ops/div.rs:291-418 : out[i] = a[i] / b[i].  The reference panics on a zero
 * divisor only outside the 32-wide unrolled body, i.e. at i >= 32*floor(n/32)
 * (div.rs:378-417).  Returns the first such index, or -1. */
EXPORT long long o_div(const float *a, const float *b, float *out, size_t n) {
    size_t checked = (n / 32) * 32;
    for (size_t i = checked; i < n; ++i)
        if (b[i] == 0.0f) return (long long)i;
    for (size_t i = 0; i < n; ++i) out[i] = a[i] / b[i];
    return -1;
}

/* ops/{add,sub,mul,div}.rs scalar variants: x op s */
EXPORT void o_add_scalar(const float *x, float s, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = x[i] + s;
}
EXPORT void o_sub_scalar(const float *x, float s, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = x[i] - s;
}
EXPORT void o_mul_scalar(const float *x, float s, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = x[i] * s;
}
EXPORT void o_div_scalar(const float *x, float s, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = x[i] / s;
}

/* core/utils.rs:802-871 negate_inplace: 0.0 - x on the 8-wide AVX2 body
 * (i < 8*floor(n/8)), -x on the scalar tail.  The two differ in the sign of
 * a zero result. */
EXPORT void o_neg(const float *x, float *out, size_t n) {
    size_t body = (n / 8) * 8;
    for (size_t i = 0; i < body; ++i) out[i] = 0.0f - x[i];
    for (size_t i = body; i < n; ++i) out[i] = -x[i];
}

/* ops/relu.rs:117-273 : x > 0 ? x : +0.0 (max_ps(x, 0) gives the same bits,
 * including +0 for -0 and NaN inputs) */
EXPORT void o_relu(const float *x, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = x[i] > 0.0f ? x[i] : 0.0f;
}

/* ops/pow.rs:192-236 : exponent 2.0 is x * x */
EXPORT void o_pow2(const float *x, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = x[i] * x[i];
}

/* ops/add.rs:106-146 + ops/broadcasting.rs:299-478: [rows,cols] + [cols] is
 * computed after materialising the bias to [rows,cols], so each element is
 * x[r][c] + bias[c].  bias_first selects [cols] + [rows,cols]. */
EXPORT void o_bias_add(const float *x, const float *bias, float *out,
                       size_t rows, size_t cols, int bias_first) {
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; ++c)
            out[r * cols + c] = bias_first ? bias[c] + x[r * cols + c]
                                           : x[r * cols + c] + bias[c];
}

/* init/basic.rs fill */
EXPORT void o_fill(float *out, float v, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = v;
}

/* ---- elementwise backward ----------------------------------------------- */

/* gradtrack/grad_fn/ops/relu.rs:4-17 : x > 0 ? go : 0.0 */
EXPORT void o_relu_bwd(const float *x, const float *go, float *gi, size_t n) {
    for (size_t i = 0; i < n; ++i) gi[i] = x[i] > 0.0f ? go[i] : 0.0f;
}

/* gradtrack/grad_fn/ops/pow.rs:5-27 : go * (e * powf(x, e - 1)), 0 if e == 0.
 * For e == 2 powf(x, 1) == x exactly. */
EXPORT void o_pow_bwd(const float *x, const float *go, float *gi, size_t n, float e) {
    for (size_t i = 0; i < n; ++i) {
        float local = (e == 0.0f) ? 0.0f : e * powf(x[i], e - 1.0f);
        gi[i] = go[i] * local;
    }
}

/* ---- reductions --------------------------------------------------------- */

/* reductions/sum.rs:80-141 : one fp32 accumulator, acc += ((x0+x1)+x2)+x3
 * per group of four, then the remainder one element at a time. */
EXPORT float o_sum(const float *x, size_t n) {
    float acc = 0.0f;
    size_t i = 0;
    for (; i + 4 <= n; i += 4) acc += x[i] + x[i + 1] + x[i + 2] + x[i + 3];
    for (; i < n; ++i) acc += x[i];
    return acc;
}

/* reductions/mean.rs:48-109 : the same sum, then / (n as f32) */
EXPORT float o_mean(const float *x, size_t n) {
    if (n == 0) return 0.0f;
    return o_sum(x, n) / (float)n;
}

/* f64 reference value of the sum (loss parity is checked against it) */
EXPORT double o_sum_f64(const float *x, size_t n) {
    double acc = 0.0;
    for (size_t i = 0; i < n; ++i) acc += (double)x[i];
    return acc;
}

/* reductions/sum.rs:225-306 sum_dims(&[0]) on [rows,cols]: zero-initialised
 * output, elements visited in row-major order, out[c] += x[r][c]. */
EXPORT void o_sum_dim0(const float *x, size_t rows, size_t cols, float *out) {
    for (size_t c = 0; c < cols; ++c) out[c] = 0.0f;
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; ++c) out[c] += x[r * cols + c];
}

/* f64 column sums (bias-gradient parity is checked against these) */
EXPORT void o_sum_dim0_f64(const float *x, size_t rows, size_t cols, double *out) {
    for (size_t c = 0; c < cols; ++c) out[c] = 0.0;
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; ++c) out[c] += (double)x[r * cols + c];
}

/* ---- contractions -------------------------------------------------------- */

/* Textbook GEMM with f64 accumulation:  C[M,N] = op(A)[M,K] . op(B)[K,N].
 * ta == 0: A[i][k] = A[i*lda + k];  ta == 1: A[i][k] = A[k*lda + i].
 * tb == 0: B[k][j] = B[k*ldb + j];  tb == 1: B[k][j] = B[j*ldb + k].
 * This is the matmul oracle (ops/matmul/mod.rs:572-611 computes the same
 * product; its blocked kernel is wrong for blocks narrower than k or n,
 * kernels.rs:1092-1133, so its bits are not reproduced). */
EXPORT void o_gemm_f64(int ta, int tb, size_t M, size_t N, size_t K,
                       const float *A, size_t lda, const float *B, size_t ldb,
                       double *C) {
    for (size_t i = 0; i < M; ++i)
        for (size_t j = 0; j < N; ++j) C[i * N + j] = 0.0;
    for (size_t i = 0; i < M; ++i) {
        for (size_t k = 0; k < K; ++k) {
            double a = ta ? (double)A[k * lda + i] : (double)A[i * lda + k];
            if (a == 0.0) continue;
            double *crow = C + i * N;
            if (!tb) {
                const float *brow = B + k * ldb;
                for (size_t j = 0; j < N; ++j) crow[j] += a * (double)brow[j];
            } else {
                for (size_t j = 0; j < N; ++j) crow[j] += a * (double)B[j * ldb + k];
            }
        }
    }
}

/* fp32 GEMM with the reference SIMD-column arithmetic (kernels.rs:254-706):
 * c[i][j] = fma(a[i][p], b[p][j], c[i][j]) for p = 0..K-1 in order.  Cache
 * blocked over k and j only, which does not change any element's operation
 * order.  Used as the single-core CPU baseline of the contractions; operands
 * with ta/tb set are first copied to row-major, as matmul/mod.rs:586-595 does
 * with contiguous() on transposed views. */
static void gemm_f32_rowmajor(size_t M, size_t N, size_t K, const float *A,
                              const float *B, float *C) {
    const size_t KB = 256, JB = 512;
    for (size_t i = 0; i < M * N; ++i) C[i] = 0.0f;
    for (size_t k0 = 0; k0 < K; k0 += KB) {
        size_t k1 = k0 + KB < K ? k0 + KB : K;
        for (size_t j0 = 0; j0 < N; j0 += JB) {
            size_t j1 = j0 + JB < N ? j0 + JB : N;
            for (size_t i = 0; i < M; ++i) {
                float *crow = C + i * N;
                for (size_t k = k0; k < k1; ++k) {
                    const float a = A[i * K + k];
                    const float *brow = B + k * N;
                    for (size_t j = j0; j < j1; ++j) crow[j] = fmaf(a, brow[j], crow[j]);
                }
            }
        }
    }
}

EXPORT void o_gemm_f32(int ta, int tb, size_t M, size_t N, size_t K,
                       const float *A, size_t lda, const float *B, size_t ldb,
                       float *C, float *scratch_a, float *scratch_b) {
    const float *Ar = A, *Br = B;
    if (ta || lda != K) {
        for (size_t i = 0; i < M; ++i)
            for (size_t k = 0; k < K; ++k)
                scratch_a[i * K + k] = ta ? A[k * lda + i] : A[i * lda + k];
        Ar = scratch_a;
    }
    if (tb || ldb != N) {
        for (size_t k = 0; k < K; ++k)
            for (size_t j = 0; j < N; ++j)
                scratch_b[k * N + j] = tb ? B[j * ldb + k] : B[k * ldb + j];
        Br = scratch_b;
    }
    gemm_f32_rowmajor(M, N, K, Ar, Br, C);
}

/* ---- optimizer ----------------------------------------------------------- */

/* Bias-correction factor exactly as optimizers/adam/mod.rs:524-531 and
 * bias_correct (:790-833): bc = (1 - (beta as f64).powf(t as f32 as f64)) as
 * f32; factor = 1.0f / bc. */
EXPORT float o_adam_correction_factor(float beta, uint64_t step_count) {
    float t = (float)step_count;
    double bc = 1.0 - pow((double)beta, (double)t);
    return 1.0f / (float)bc;
}

/* One Adam::step for one parameter (optimizers/adam/mod.rs:485-1007), with
 * step_count the optimizer's global count after its increment (:1036-1044).
 * The five reference passes are fused per element; each element still sees
 * the reference's operation order:
 *   g' = g + wd*p         only when wd > 0 (:511-518, :567-620)
 *   m = b1*m + c1*g'
 *   v = b2*v + c2*(g'*g') on the 8-wide body, (c2*g')*g' on the tail (:736-773)
 *   mh = m*cf1; vh = v*cf2
 *   AMSGrad (vmax != NULL, :534-541): vmax = first ? vh : max(vmax, vh); vh = vmax
 *   p = p - (lr*mh)/(sqrt(vh)+eps)
 * with c1 = 1-b1 and c2 = 1-b2 in fp32. */
EXPORT void o_adam_step(float *p, const float *g, float *m, float *v, float *vmax, size_t n,
                        float lr, float b1, float b2, float eps, float wd, uint64_t step_count,
                        int amsgrad_first) {
    const float c1 = 1.0f - b1, c2 = 1.0f - b2;
    const float cf1 = o_adam_correction_factor(b1, step_count);
    const float cf2 = o_adam_correction_factor(b2, step_count);
    const size_t body = (n / 8) * 8;
    for (size_t i = 0; i < n; ++i) {
        float gi = g[i];
        if (wd > 0.0f) gi = gi + wd * p[i];
        float mi = b1 * m[i] + c1 * gi;
        float vi = (i < body) ? b2 * v[i] + c2 * (gi * gi) : b2 * v[i] + (c2 * gi) * gi;
        m[i] = mi;
        v[i] = vi;
        float mh = mi * cf1;
        float vh = vi * cf2;
        if (vmax) {
            float old = amsgrad_first ? vh : vmax[i];
            vh = old > vh ? old : vh;
            vmax[i] = vh;
        }
        float den = sqrtf(vh) + eps;
        p[i] = p[i] - (lr * mh) / den;
    }
}
