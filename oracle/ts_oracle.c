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
 *   randn: xorshift64 against Marsaglia's published test vector (seed
 *       88172645463325252 -> 8748534153485358512) and step-by-step advance;
 *       seed 0 gives the closed-form constant sqrt(2 ln 2) * cos(pi) for
 *       every element; mode 1 (f64 log / cos rounded once) is checked
 *       correctly rounded on all 2^23 inputs against long double.
 *   exp / log / cos / tanh (mode 2, glibc 2.35's evaluations restated):
 *       against the host libm on every f32 input (cos below 120), 0
 *       differences; mode 0 calls the host libm, as the reference does.
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

/* ---- random initialisation -------------------------------------------------- */

/* XorShiftRng::next_u64 (tensor/init/random.rs:524-529): Marsaglia's
 * xorshift64 with the shift triple (13, 7, 17). */
static uint64_t xs_next(uint64_t *s) {
    uint64_t x = *s;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *s = x;
    return x;
}

EXPORT uint64_t o_xorshift_next(uint64_t s) { return xs_next(&s); }

/* State after k steps from s, one step at a time (the brute-force check of
 * the device's jump-ahead). */
EXPORT uint64_t o_xorshift_advance(uint64_t s, uint64_t k) {
    while (k--) xs_next(&s);
    return s;
}

/* next_f32 (random.rs:557-564): the low 23 bits of the draw become the
 * mantissa of a float with biased exponent 126, a value in [0.5, 1). */
static float xs_unit(uint64_t *s) {
    uint32_t bits = (uint32_t)(xs_next(s) & 0x7FFFFFu) | (126u << 23);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* ---- glibc 2.35's f32 exp / log / cos / tanh, restated (mode 2) ----------
 *
 * The reference takes these from the host libm (Rust's f32::exp / ln / cos /
 * tanh call expf / logf / cosf / tanhf); the pinned libm is glibc 2.35 (the
 * image's, Ubuntu 2.35-0ubuntu3).  Its algorithms are published:
 *   expf, logf, cosf: Arm optimized-routines (MIT / Apache-2.0), shipped as
 *     glibc's sysdeps/ieee754/flt-32/e_expf.c, e_logf.c, s_cosf.c with the
 *     tables of e_exp2f_data.c, e_logf_data.c, s_sincosf_data.c; on an x86-64
 *     CPU with FMA glibc selects the builds compiled with FMA (multiarch
 *     e_expf-fma, e_logf-fma, s_cosf-fma), in which every product whose only
 *     uses are additions is fused;
 *   tanhf (with expm1f): fdlibm's s_tanhf.c / s_expm1f.c (Sun Microsystems,
 *     "permission to use, copy, modify, and distribute this software is
 *     freely granted, provided that this notice is preserved"), compiled
 *     for plain x86-64, in f32 with no fused operations.
 * Each function below restates that evaluation step by step in this file's
 * own code, with the published constants (the exp table is 2^(i/32)
 * rounded to double, computed here).  Pinned: o_glibc_restated_diff counts
 * inputs where a restatement differs from the host libm; on every one of
 * the 2^32 f32 inputs (|x| < 120 for cos, the only range used) the count is
 * 0 on this image with FMA (tests/test_ops_oracle.py runs strided and dense
 * sweeps).  Without FMA glibc's expf differs from this on 2 inputs of 2^32
 * and cosf on 22 below 120. */
static uint64_t d_bits(double x) { uint64_t u; memcpy(&u, &x, 8); return u; }
static double d_of(uint64_t u) { double x; memcpy(&x, &u, 8); return x; }
static uint32_t f_bits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static float f_of(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* expf: x = (k + r)/32 * ln2 with integer k (ties to even through the
 * 1.5*2^52 shift) and |r| <= 1/2; exp(x) = 2^(k/32) * 2^(r/32), the first a
 * table entry with k/32's integer part added to its exponent, the second a
 * degree-3 polynomial, all in double, rounded to f32 once. */
static uint64_t gl_exp_tab[32];
static int gl_exp_ready;
static void gl_exp_init(void) {
    for (int i = 0; i < 32; ++i) /* 2^(i/32) rounded to double, less i/32 in the exponent field */
        gl_exp_tab[i] = d_bits((double)exp2l((long double)i / 32)) - ((uint64_t)i << 52) / 32;
    gl_exp_ready = 1;
}
static float gl_expf(float x) {
    if (!gl_exp_ready) gl_exp_init();
    const double InvLn2N = 0x1.71547652b82fep+0 * 32, SHIFT = 0x1.8p+52;
    const double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 C2 = 0x1.62e42ff0c52d6p-1 / 32;
    const uint32_t abstop = (f_bits(x) >> 20) & 0x7ff;
    if (abstop >= 0x42b) { /* |x| >= 88, inf, nan */
        if (f_bits(x) == f_bits(-INFINITY)) return 0.0f;
        if (abstop >= 0x7f8) return x + x;
        if (x > 0x1.62e42ep6f) return INFINITY;
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double xd = (double)x;
    double kd = fma(InvLn2N, xd, SHIFT);
    const uint64_t ki = d_bits(kd);
    kd -= SHIFT;
    const double r = fma(InvLn2N, xd, -kd);
    const double s = d_of(gl_exp_tab[ki % 32] + (ki << 47));
    const double z = fma(C0, r, C1), r2 = r * r;
    double y = fma(C2, r, 1.0);
    y = fma(z, r2, y);
    return (float)(y * s);
}

/* logf: x = 2^k z with z in [0x3f330000, 2 * that) as bits; z's subinterval
 * (16 of them) gives c ~ its centre: log(x) = log1p(z/c - 1) + log(c) + k ln2,
 * log1p by a degree-4 polynomial, in double, rounded once. */
static const double gl_log_invc[16] = {
    0x1.661ec79f8f3bep+0, 0x1.571ed4aaf883dp+0, 0x1.49539f0f010bp+0,  0x1.3c995b0b80385p+0,
    0x1.30d190c8864a5p+0, 0x1.25e227b0b8eap+0,  0x1.1bb4a4a1a343fp+0, 0x1.12358f08ae5bap+0,
    0x1.0953f419900a7p+0, 0x1p+0,               0x1.e608cfd9a47acp-1, 0x1.ca4b31f026aap-1,
    0x1.b2036576afce6p-1, 0x1.9c2d163a1aa2dp-1, 0x1.886e6037841edp-1, 0x1.767dcf5534862p-1};
static const double gl_log_logc[16] = {
    -0x1.57bf7808caadep-2, -0x1.2bef0a7c06ddbp-2, -0x1.01eae7f513a67p-2, -0x1.b31d8a68224e9p-3,
    -0x1.6574f0ac07758p-3, -0x1.1aa2bc79c81p-3,  -0x1.a4e76ce8c0e5ep-4, -0x1.1973c5a611cccp-4,
    -0x1.252f438e10c1ep-5, 0x0p+0,               0x1.aa5aa5df25984p-5,  0x1.c5e53aa362eb4p-4,
    0x1.526e57720db08p-3,  0x1.bc2860d22477p-3,   0x1.1058bc8a07ee1p-2,  0x1.4043057b6ee09p-2};
static float gl_logf(float x) {
    const double A0 = -0x1.00ea348b88334p-2, A1 = 0x1.5575b0be00b6ap-2, A2 = -0x1.ffffef20a4123p-2,
                 Ln2 = 0x1.62e42fefa39efp-1;
    uint32_t ix = f_bits(x);
    if (ix == 0x3f800000) return 0.0f;
    if (ix - 0x00800000 >= 0x7f800000 - 0x00800000) { /* zero, subnormal, negative, inf, nan */
        if (ix * 2 == 0) return -INFINITY;
        if (ix == 0x7f800000) return x;
        if ((ix & 0x80000000) || ix * 2 >= 0xff000000) return NAN;
        ix = f_bits(x * 0x1p23f); /* normalise a subnormal */
        ix -= 23u << 23;
    }
    const uint32_t tmp = ix - 0x3f330000;
    const int i = (int)((tmp >> 19) % 16);
    const int32_t k = (int32_t)tmp >> 23;
    const double z = (double)f_of(ix - (tmp & 0xff800000u));
    const double r = fma(z, gl_log_invc[i], -1.0);
    const double y0 = fma((double)k, Ln2, gl_log_logc[i]);
    const double r2 = r * r;
    double y = fma(A1, r, A2);
    y = fma(A0, r2, y);
    y = fma(y, r2, y0 + r);
    return (float)y;
}

/* cosf for |x| < 120: below pi/4 the even polynomial directly; else x less
 * n * pi/2 (n from the 2/pi * 2^24 scaled product, rounded), the sign and
 * the sin or cos polynomial by n's low bits; in double, rounded once. */
typedef struct { double sign[4], hpi_inv, hpi, c0, c1, c2, c3, c4, s1, s2, s3; } gl_sincos_t;
static const gl_sincos_t gl_sincos[2] = {
    {{1.0, -1.0, -1.0, 1.0}, 0x1.45F306DC9C883p+23, 0x1.921FB54442D18p0, 0x1p0, -0x1.ffffffd0c621cp-2,
     0x1.55553e1068f19p-5, -0x1.6c087e89a359dp-10, 0x1.99343027bf8c3p-16, -0x1.555545995a603p-3,
     0x1.1107605230bc4p-7, -0x1.994eb3774cf24p-13},
    {{1.0, -1.0, -1.0, 1.0}, 0x1.45F306DC9C883p+23, 0x1.921FB54442D18p0, -0x1p0, 0x1.ffffffd0c621cp-2,
     -0x1.55553e1068f19p-5, 0x1.6c087e89a359dp-10, -0x1.99343027bf8c3p-16, -0x1.555545995a603p-3,
     0x1.1107605230bc4p-7, -0x1.994eb3774cf24p-13}};
static float gl_sincos_poly(double x, double x2, const gl_sincos_t *p, int n) {
    if ((n & 1) == 0) { /* sin */
        const double x3 = x * x2, s1 = fma(x2, p->s3, p->s2), x7 = x3 * x2, s = fma(x3, p->s1, x);
        return (float)fma(x7, s1, s);
    }
    const double x4 = x2 * x2, c2 = fma(x2, p->c4, p->c3), c1 = fma(x2, p->c1, p->c0), x6 = x4 * x2,
                 c = fma(x4, p->c2, c1);
    return (float)fma(x6, c2, c);
}
static float gl_cosf(float y) { /* |y| < 120 */
    const uint32_t top = (f_bits(y) >> 20) & 0x7ff;
    const gl_sincos_t *p = &gl_sincos[0];
    double x = (double)y;
    if (top < ((f_bits(0x1.921FB6p-1f) >> 20) & 0x7ff)) { /* |y| < pi/4 */
        if (top < ((f_bits(0x1p-12f) >> 20) & 0x7ff)) return 1.0f;
        return gl_sincos_poly(x, x * x, p, 1);
    }
    const int n = (((int32_t)(x * p->hpi_inv)) + 0x800000) >> 24;
    x = fma(-(double)n, p->hpi, x);
    const double sgn = p->sign[n & 3];
    if (n & 2) p = &gl_sincos[1];
    return gl_sincos_poly(x * sgn, x * x, p, n ^ 1);
}

/* expm1f (fdlibm s_expm1f.c): x = k ln2 + r with |r| <= ln2/2 split into
 * hi - lo, expm1(r) from a rational form with a degree-5 polynomial in
 * r^2/2, then the exponent k applied; all in f32. */
static float gl_expm1f(float x) {
    const float one = 1.0f, huge = 1.0e+30f, tiny = 1.0e-30f, o_threshold = f_of(0x42b17180),
                ln2_hi = f_of(0x3f317180), ln2_lo = f_of(0x3717f7d1), invln2 = f_of(0x3fb8aa3b),
                Q1 = f_of(0xbd088889), Q2 = f_of(0x3ad00d01), Q3 = f_of(0xb8a670cd), Q4 = f_of(0x36867e54),
                Q5 = f_of(0xb457edbb);
    float y, hi, lo, c = 0.0f, t, e, hxs, hfx, r1;
    int32_t k;
    uint32_t hx = f_bits(x);
    const uint32_t xsb = hx & 0x80000000u;
    hx &= 0x7fffffff;
    if (hx >= 0x4195b844) { /* |x| >= 27 ln2 */
        if (hx >= 0x42b17218) {
            if (hx > 0x7f800000) return x + x;
            if (hx == 0x7f800000) return xsb == 0 ? x : -1.0f;
            if (x > o_threshold) return huge * huge;
        }
        if (xsb != 0 && x + tiny < 0.0f) return tiny - one;
    }
    if (hx > 0x3eb17218) { /* |x| > ln2/2 */
        if (hx < 0x3F851592) { /* and < 3 ln2/2 */
            if (xsb == 0) { hi = x - ln2_hi; lo = ln2_lo; k = 1; }
            else { hi = x + ln2_hi; lo = -ln2_lo; k = -1; }
        } else {
            k = (int32_t)(invln2 * x + (xsb == 0 ? 0.5f : -0.5f));
            t = (float)k;
            hi = x - t * ln2_hi;
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000) { /* |x| < 2^-25 */
        t = huge + x;
        return x - (t - (huge + x));
    } else {
        k = 0;
    }
    hfx = 0.5f * x;
    hxs = x * hfx;
    r1 = one + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    t = 3.0f - r1 * hfx;
    e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = x * (e - c) - c;
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) return x < -0.25f ? -2.0f * (e - (x + 0.5f)) : one + 2.0f * (x - e);
    if (k <= -2 || k > 56) {
        y = one - (e - x);
        if (k == 128) y = y * 2.0f * f_of(0x7f000000);
        else y = f_of(f_bits(y) + ((uint32_t)k << 23));
        return y - one;
    }
    if (k < 23) {
        t = f_of(0x3f800000 - (0x1000000u >> k)); /* 1 - 2^-k */
        y = t - (e - x);
    } else {
        t = f_of((uint32_t)(0x7f - k) << 23); /* 2^-k */
        y = x - (e + t);
        y += one;
    }
    return f_of(f_bits(y) + ((uint32_t)k << 23));
}

/* tanhf (fdlibm s_tanhf.c): 1 - 2/(expm1(2|x|) + 2) for |x| >= 1,
 * -t/(t + 2) with t = expm1(-2|x|) below, 1 past 22, the sign restored. */
static float gl_tanhf(float x) {
    const float one = 1.0f, two = 2.0f, tiny = 1.0e-30f;
    float t, z;
    const int32_t jx = (int32_t)f_bits(x), ix = jx & 0x7fffffff;
    if (ix >= 0x7f800000) return jx >= 0 ? one / x + one : one / x - one;
    if (ix < 0x41b00000) { /* |x| < 22 */
        if (ix == 0) return x;
        if (ix < 0x24000000) return x * (one + x); /* |x| < 2^-55 */
        if (ix >= 0x3f800000) {
            t = gl_expm1f(two * fabsf(x));
            z = one - two / (t + two);
        } else {
            t = gl_expm1f(-two * fabsf(x));
            z = -t / (t + two);
        }
    } else {
        z = one - tiny;
    }
    return jx >= 0 ? z : -z;
}

/* Inputs x = offset + k * stride (as f32 bit patterns) where the
 * restatement of op (0 exp, 1 log, 2 tanh, 3 cos below 120, 4 expm1)
 * differs from the host libm's (any two NaNs agree). */
EXPORT long o_glibc_restated_diff(int op, unsigned stride, unsigned offset) {
    long diff = 0;
    for (uint64_t u = offset; u < (1ull << 32); u += stride) {
        const float x = f_of((uint32_t)u);
        float a, b;
        switch (op) {
            case 0: a = expf(x); b = gl_expf(x); break;
            case 1: a = logf(x); b = gl_logf(x); break;
            case 2: a = tanhf(x); b = gl_tanhf(x); break;
            case 3: if (!(fabsf(x) < 120.0f)) continue; a = cosf(x); b = gl_cosf(x); break;
            default: a = expm1f(x); b = gl_expm1f(x); break;
        }
        if (f_bits(a) != f_bits(b) && !(isnan(a) && isnan(b))) ++diff;
    }
    return diff;
}

/* f32 natural log and cosine.  mode 0 calls the host libm's logf / cosf, as
 * Rust's f32::ln / f32::cos do; mode 1 evaluates in f64 and rounds once,
 * which is correctly rounded on every input next_normal can produce
 * (checked against long double by o_libm_cr_check); mode 2 is glibc 2.35's
 * evaluation restated (above), mode 0's bits without the host libm. */
static float ln_f32(float x, int mode) {
    return mode == 1 ? (float)log((double)x) : mode == 2 ? gl_logf(x) : logf(x);
}
static float cos_f32(float x, int mode) {
    return mode == 1 ? (float)cos((double)x) : mode == 2 ? gl_cosf(x) : cosf(x);
}

/* 2*PI in fp32: std::f32::consts::PI (0x40490FDB) doubled exactly. */
static const float kTwoPiF = 6.28318548202514648438f;

/* next_normal (random.rs:592-615): Box-Muller on two consecutive draws,
 *   u1 = next_f32, u2 = next_f32, u1 clamped into (0, 1),
 *   z  = sqrt(-2 * ln(u1)) * cos((2*PI) * u2)    all in fp32,
 *   z  = 0 if NaN or infinite. */
static float xs_normal(uint64_t *s, int mode) {
    float u1 = xs_unit(s);
    float u2 = xs_unit(s);
    if (u1 <= 0.0f) u1 = 1e-7f;
    else if (u1 >= 1.0f) u1 = 1.0f - 1e-7f;
    float r = sqrtf(-2.0f * ln_f32(u1, mode));
    float z = r * cos_f32(kTwoPiF * u2, mode);
    return (isnan(z) || isinf(z)) ? 0.0f : z;
}

/* Tensor::randn / fill_randn (random.rs:231-299, XorShiftRng::new :473-475): element i takes draws
 * 2i+1 and 2i+2 of XorShiftRng::new(seed), in order; both fill paths
 * (fill_randn_simd_avx2 :340-362, fill_randn_scalar :401-419) draw
 * sequentially, so the layout does not depend on the path taken. */
EXPORT void o_randn(float *out, size_t n, uint64_t seed, int mode) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; ++i) out[i] = xs_normal(&s, mode);
}

/* Exhaustive checks over the 2^23 values next_f32 can return.
 * which = 0: ln(u); which = 1: cos((2*PI) * u).
 * o_libm_cr_check counts inputs where the f64 evaluation rounded to f32
 * disagrees with the long-double evaluation rounded to f32 (0 means mode 1
 * is correctly rounded on the whole domain).  o_libm_glibc_diff counts
 * inputs where the host's logf / cosf differ from mode 1. */
static float unit_of(uint32_t m) {
    uint32_t bits = m | (126u << 23);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

EXPORT long o_libm_cr_check(int which) {
    long bad = 0;
    for (uint32_t m = 0; m < (1u << 23); ++m) {
        float u = unit_of(m);
        float x = which ? kTwoPiF * u : u;
        float a = which ? (float)cos((double)x) : (float)log((double)x);
        float b = which ? (float)cosl((long double)x) : (float)logl((long double)x);
        if (memcmp(&a, &b, 4) != 0) ++bad;
    }
    return bad;
}

EXPORT long o_libm_glibc_diff(int which) {
    long diff = 0;
    for (uint32_t m = 0; m < (1u << 23); ++m) {
        float u = unit_of(m);
        float a = which ? cos_f32(kTwoPiF * u, 0) : ln_f32(u, 0);
        float b = which ? cos_f32(kTwoPiF * u, 1) : ln_f32(u, 1);
        if (memcmp(&a, &b, 4) != 0) ++diff;
    }
    return diff;
}

/* ---- other recorded ops (tensor/ops/{exp,log,sqrt,tanh,sigmoid,leaky_relu,softmax}.rs) ---- */

/* f32 exp / ln / tanh: mode 0 is the host libm (expf, logf, tanhf), which
 * Rust's f32::exp / ln / tanh call; mode 1 evaluates in f64 and rounds once;
 * mode 2 is glibc 2.35's evaluation restated (above). */
static float f_exp(float x, int mode) { return mode == 1 ? (float)exp((double)x) : mode == 2 ? gl_expf(x) : expf(x); }
static float f_log(float x, int mode) { return mode == 1 ? (float)log((double)x) : mode == 2 ? gl_logf(x) : logf(x); }
static float f_tanh(float x, int mode) {
    return mode == 1 ? (float)tanh((double)x) : mode == 2 ? gl_tanhf(x) : tanhf(x);
}

/* op: 0 exp (exp.rs scalar loop), 1 log (log.rs), 2 sqrt (sqrt.rs; AVX2
 * sqrt_ps and f32::sqrt are both correctly rounded), 3 tanh (tanh.rs),
 * 4 sigmoid (sigmoid.rs:9-21: x >= 0 ? 1/(1+exp(-x)) : z/(1+z), z = exp(x)),
 * 5 leaky_relu (leaky_relu.rs: x > 0 ? x : slope*x) */
EXPORT void o_unary(int op, const float *x, float *y, size_t n, float slope, int mode) {
    for (size_t i = 0; i < n; ++i) {
        const float v = x[i];
        switch (op) {
            case 0: y[i] = f_exp(v, mode); break;
            case 1: y[i] = f_log(v, mode); break;
            case 2: y[i] = sqrtf(v); break;
            case 3: y[i] = f_tanh(v, mode); break;
            case 4:
                if (v >= 0.0f) {
                    const float z = f_exp(-v, mode);
                    y[i] = 1.0f / (1.0f + z);
                } else {
                    const float z = f_exp(v, mode);
                    y[i] = z / (1.0f + z);
                }
                break;
            default: y[i] = v > 0.0f ? v : slope * v; break;
        }
    }
}

/* Backward formulas (grad_fn/ops/{exp,log,sqrt,tanh,sigmoid,leaky_relu}.rs);
 * `saved` is the output y for exp / sqrt / tanh / sigmoid and the input x for
 * log / leaky_relu:
 *   exp: go*y; log: inv = 1/x, go*inv; sqrt: inv = 1/y, s = inv*0.5, go*s;
 *   tanh: go*(1 - y*y); sigmoid: go*y*(1 - y) (left to right);
 *   leaky_relu: x > 0 ? go : slope*go */
EXPORT void o_unary_bwd(int op, const float *saved, const float *go, float *gi, size_t n, float slope) {
    for (size_t i = 0; i < n; ++i) {
        const float s = saved[i], g = go[i];
        switch (op) {
            case 0: gi[i] = g * s; break;
            case 1: {
                const float inv = 1.0f / s;
                gi[i] = g * inv;
                break;
            }
            case 2: {
                const float inv = 1.0f / s;
                const float sc = inv * 0.5f;
                gi[i] = g * sc;
                break;
            }
            case 3: gi[i] = g * (1.0f - s * s); break;
            case 4: gi[i] = g * s * (1.0f - s); break;
            default: gi[i] = s > 0.0f ? g : slope * g; break;
        }
    }
}

/* softmax.rs:4-60 on [outer, reduce, inner]: per slice max, then exp(x - max)
 * with a sequential fp32 sum, then y *= 1/sum */
EXPORT void o_softmax(const float *x, float *y, size_t outer, size_t reduce, size_t inner, int mode) {
    for (size_t o = 0; o < outer; ++o)
        for (size_t i = 0; i < inner; ++i) {
            const size_t base = o * reduce * inner + i;
            float maxv = -INFINITY;
            for (size_t j = 0; j < reduce; ++j) {
                const float v = x[base + j * inner];
                if (v > maxv) maxv = v;
            }
            float sum = 0.0f;
            for (size_t j = 0; j < reduce; ++j) {
                const float e = f_exp(x[base + j * inner] - maxv, mode);
                y[base + j * inner] = e;
                sum += e;
            }
            const float inv = 1.0f / sum;
            for (size_t j = 0; j < reduce; ++j) y[base + j * inner] *= inv;
        }
}

/* grad_fn/ops/softmax.rs:4-38: dot = sequential fp32 sum of go*y over the
 * slice, gi = y * (go - dot) */
EXPORT void o_softmax_bwd(const float *y, const float *go, float *gi, size_t outer, size_t reduce,
                          size_t inner) {
    for (size_t o = 0; o < outer; ++o)
        for (size_t i = 0; i < inner; ++i) {
            const size_t base = o * reduce * inner + i;
            float dot = 0.0f;
            for (size_t j = 0; j < reduce; ++j) dot += go[base + j * inner] * y[base + j * inner];
            for (size_t j = 0; j < reduce; ++j)
                gi[base + j * inner] = y[base + j * inner] * (go[base + j * inner] - dot);
        }
}

/* sum_dims (reductions/sum.rs:254-287): every input element, in order, is
 * added in fp32 to the output element its kept coordinates select.  out is
 * in the keepdim layout (reduced axes of size 1) and starts at zero; out64
 * (optional) receives the same sums in f64. */
EXPORT void o_sum_dims(const float *x, const size_t *dims, size_t rank, unsigned mask, float *out,
                       double *out64) {
    size_t n = 1, n_out = 1;
    for (size_t k = 0; k < rank; ++k) {
        n *= dims[k];
        if (!((mask >> k) & 1u)) n_out *= dims[k];
    }
    for (size_t o = 0; o < n_out; ++o) {
        out[o] = 0.0f;
        if (out64) out64[o] = 0.0;
    }
    for (size_t lin = 0; lin < n; ++lin) {
        size_t rem = lin, o = 0, ostride = 1;
        for (size_t k = rank; k-- > 0;) {
            const size_t c = rem % dims[k];
            rem /= dims[k];
            if (!((mask >> k) & 1u)) {
                o += c * ostride;
                ostride *= dims[k];
            }
        }
        out[o] += x[lin];
        if (out64) out64[o] += (double)x[lin];
    }
}

/* Inputs (of the 2^32 bit patterns, every `stride`-th) where the f64 value
 * rounded once disagrees with the long-double value rounded once (op 0 exp,
 * 1 log, 3 tanh); o_unary_glibc_diff counts where the host libm's expf /
 * logf / tanhf differ from the f64 value rounded once. */
EXPORT long o_unary_cr_check(int op, unsigned stride) {
    long bad = 0;
    for (uint64_t b = 0; b < (1ull << 32); b += stride) {
        uint32_t bits = (uint32_t)b;
        float x;
        memcpy(&x, &bits, 4);
        if (isnan(x)) continue;
        float a, c;
        if (op == 0) { a = (float)exp((double)x); c = (float)expl((long double)x); }
        else if (op == 1) { a = (float)log((double)x); c = (float)logl((long double)x); }
        else { a = (float)tanh((double)x); c = (float)tanhl((long double)x); }
        if (memcmp(&a, &c, 4) != 0 && !(isnan(a) && isnan(c))) ++bad;
    }
    return bad;
}

EXPORT long o_unary_glibc_diff(int op, unsigned stride) {
    long diff = 0;
    for (uint64_t b = 0; b < (1ull << 32); b += stride) {
        uint32_t bits = (uint32_t)b;
        float x;
        memcpy(&x, &bits, 4);
        if (isnan(x)) continue;
        float a, c;
        if (op == 0) { a = expf(x); c = (float)exp((double)x); }
        else if (op == 1) { a = logf(x); c = (float)log((double)x); }
        else { a = tanhf(x); c = (float)tanh((double)x); }
        if (memcmp(&a, &c, 4) != 0 && !(isnan(a) && isnan(c))) ++diff;
    }
    return diff;
}
