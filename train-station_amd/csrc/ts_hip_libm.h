// f32 exp, log, cos and tanh with the bits of the host libm the reference
// calls (Rust's f32::exp / ln / cos / tanh call expf / logf / cosf / tanhf;
// the pinned libm is glibc 2.35).  glibc's algorithms are published:
//   expf, logf, cosf: Arm optimized-routines (MIT / Apache-2.0), glibc's
//     sysdeps/ieee754/flt-32/e_expf.c, e_logf.c, s_cosf.c with the tables of
//     e_exp2f_data.c, e_logf_data.c, s_sincosf_data.c, evaluated in double;
//     on an x86-64 CPU with FMA glibc runs the builds compiled with FMA, in
//     which every product whose only uses are additions is fused (fma below,
//     the rest rounded step by step: this library compiles with contraction
//     off);
//   tanhf with expm1f: fdlibm's s_tanhf.c / s_expm1f.c (Sun Microsystems,
//     "permission to use, copy, modify, and distribute this software is
//     freely granted, provided that this notice is preserved"), in f32 with
//     no fused operations and IEEE division.
// Each function restates that evaluation in this file's own code with the
// published constants (the exp table's entries are 2^(i/32) rounded to
// double, generated from that definition; oracle/ts_oracle.c computes them
// the same way and restates the same functions in C).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tship {
namespace libm {

__device__ __forceinline__ uint32_t fbits(float x) { return __float_as_uint(x); }
__device__ __forceinline__ float fof(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint64_t dbits(double x) { return static_cast<uint64_t>(__double_as_longlong(x)); }
__device__ __forceinline__ double dof(uint64_t u) { return __longlong_as_double(static_cast<long long>(u)); }

// exp: x = (k + r)/32 * ln2 with integer k (ties to even through the 1.5*2^52
// shift) and |r| <= 1/2; exp(x) = 2^(k/32) * 2^(r/32): a table entry with
// k/32's integer part added to its exponent field, and a degree-3 polynomial.
// Table entry i: the bits of 2^(i/32) rounded to double, less i/32 in the
// exponent field (so k's bits can be added whole).
__device__ __constant__ const uint64_t kExpTab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

__device__ __forceinline__ float expf_glibc(float x) {
    const double InvLn2N = 0x1.71547652b82fep+0 * 32, SHIFT = 0x1.8p+52;
    const double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 C2 = 0x1.62e42ff0c52d6p-1 / 32;
    const uint32_t abstop = (fbits(x) >> 20) & 0x7ff;
    if (abstop >= 0x42b) {  // |x| >= 88, inf, nan
        if (fbits(x) == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double xd = static_cast<double>(x);
    double kd = __builtin_fma(InvLn2N, xd, SHIFT);
    const uint64_t ki = dbits(kd);
    kd -= SHIFT;
    const double r = __builtin_fma(InvLn2N, xd, -kd);
    const double s = dof(kExpTab[ki % 32] + (ki << 47));
    const double z = __builtin_fma(C0, r, C1), r2 = r * r;
    double y = __builtin_fma(C2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    return static_cast<float>(y * s);
}

// log: x = 2^k z with z's bits in [0x3f330000, that + 2^23); z's subinterval
// (16) gives c near its centre: log(x) = log1p(z/c - 1) + log(c) + k ln2,
// log1p by a degree-4 polynomial.
__device__ __constant__ const double kLogInvc[16] = {
    0x1.661ec79f8f3bep+0, 0x1.571ed4aaf883dp+0, 0x1.49539f0f010bp+0,  0x1.3c995b0b80385p+0,
    0x1.30d190c8864a5p+0, 0x1.25e227b0b8eap+0,  0x1.1bb4a4a1a343fp+0, 0x1.12358f08ae5bap+0,
    0x1.0953f419900a7p+0, 0x1p+0,               0x1.e608cfd9a47acp-1, 0x1.ca4b31f026aap-1,
    0x1.b2036576afce6p-1, 0x1.9c2d163a1aa2dp-1, 0x1.886e6037841edp-1, 0x1.767dcf5534862p-1};
__device__ __constant__ const double kLogLogc[16] = {
    -0x1.57bf7808caadep-2, -0x1.2bef0a7c06ddbp-2, -0x1.01eae7f513a67p-2, -0x1.b31d8a68224e9p-3,
    -0x1.6574f0ac07758p-3, -0x1.1aa2bc79c81p-3,  -0x1.a4e76ce8c0e5ep-4, -0x1.1973c5a611cccp-4,
    -0x1.252f438e10c1ep-5, 0x0p+0,               0x1.aa5aa5df25984p-5,  0x1.c5e53aa362eb4p-4,
    0x1.526e57720db08p-3,  0x1.bc2860d22477p-3,   0x1.1058bc8a07ee1p-2,  0x1.4043057b6ee09p-2};

__device__ __forceinline__ float logf_glibc(float x) {
    const double A0 = -0x1.00ea348b88334p-2, A1 = 0x1.5575b0be00b6ap-2, A2 = -0x1.ffffef20a4123p-2,
                 Ln2 = 0x1.62e42fefa39efp-1;
    uint32_t ix = fbits(x);
    if (ix == 0x3f800000u) return 0.0f;
    if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u) {  // zero, subnormal, negative, inf, nan
        if (ix * 2 == 0) return -__builtin_inff();
        if (ix == 0x7f800000u) return x;
        if ((ix & 0x80000000u) || ix * 2 >= 0xff000000u) return __builtin_nanf("");
        ix = fbits(x * 0x1p23f);  // a subnormal, normalised
        ix -= 23u << 23;
    }
    const uint32_t tmp = ix - 0x3f330000u;
    const int i = static_cast<int>((tmp >> 19) % 16);
    const int32_t k = static_cast<int32_t>(tmp) >> 23;
    const double z = static_cast<double>(fof(ix - (tmp & 0xff800000u)));
    const double r = __builtin_fma(z, kLogInvc[i], -1.0);
    const double y0 = __builtin_fma(static_cast<double>(k), Ln2, kLogLogc[i]);
    const double r2 = r * r;
    double y = __builtin_fma(A1, r, A2);
    y = __builtin_fma(A0, r2, y);
    y = __builtin_fma(y, r2, y0 + r);
    return static_cast<float>(y);
}

// cos for |x| < 120 (the caller's range: randn's 2*pi*u, u in [0, 1)):
// below pi/4 the even polynomial directly; else x less n * pi/2 (n from the
// 2/pi * 2^24 scaled product), and by n's low bits the sign and the sine or
// cosine polynomial (the second coefficient set negates the cosine's).
struct SinCos {
    double sign[4], hpi_inv, hpi, c0, c1, c2, c3, c4, s1, s2, s3;
};
__device__ __constant__ const SinCos kSinCos[2] = {
    {{1.0, -1.0, -1.0, 1.0}, 0x1.45F306DC9C883p+23, 0x1.921FB54442D18p0, 0x1p0, -0x1.ffffffd0c621cp-2,
     0x1.55553e1068f19p-5, -0x1.6c087e89a359dp-10, 0x1.99343027bf8c3p-16, -0x1.555545995a603p-3,
     0x1.1107605230bc4p-7, -0x1.994eb3774cf24p-13},
    {{1.0, -1.0, -1.0, 1.0}, 0x1.45F306DC9C883p+23, 0x1.921FB54442D18p0, -0x1p0, 0x1.ffffffd0c621cp-2,
     -0x1.55553e1068f19p-5, 0x1.6c087e89a359dp-10, -0x1.99343027bf8c3p-16, -0x1.555545995a603p-3,
     0x1.1107605230bc4p-7, -0x1.994eb3774cf24p-13}};

__device__ __forceinline__ float sincos_poly(double x, double x2, const SinCos &p, int n) {
    if ((n & 1) == 0) {  // sine
        const double x3 = x * x2, s1 = __builtin_fma(x2, p.s3, p.s2), x7 = x3 * x2, s = __builtin_fma(x3, p.s1, x);
        return static_cast<float>(__builtin_fma(x7, s1, s));
    }
    const double x4 = x2 * x2, c2 = __builtin_fma(x2, p.c4, p.c3), c1 = __builtin_fma(x2, p.c1, p.c0),
                 x6 = x4 * x2, c = __builtin_fma(x4, p.c2, c1);
    return static_cast<float>(__builtin_fma(x6, c2, c));
}

__device__ __forceinline__ float cosf_glibc_small(float y) {
    const uint32_t top = (fbits(y) >> 20) & 0x7ff;
    double x = static_cast<double>(y);
    if (top < 0x3f4) {  // |y| < pi/4 (0x3f490fdb's top 12 bits)
        if (top < 0x398) return 1.0f;  // |y| < 2^-12
        return sincos_poly(x, x * x, kSinCos[0], 1);
    }
    const int n = (static_cast<int32_t>(x * kSinCos[0].hpi_inv) + 0x800000) >> 24;
    x = __builtin_fma(-static_cast<double>(n), kSinCos[0].hpi, x);
    const double sgn = kSinCos[0].sign[n & 3];
    return sincos_poly(x * sgn, x * x, kSinCos[(n & 2) ? 1 : 0], n ^ 1);
}

// expm1 (fdlibm): x = k ln2 + r, |r| <= ln2/2, r split as hi - lo;
// expm1(r) from a rational form with a degree-5 polynomial in r^2/2, then
// the exponent k applied; all in f32.
__device__ __forceinline__ float expm1f_fdlibm(float x) {
    const float one = 1.0f, huge = 1.0e+30f, tiny = 1.0e-30f, o_threshold = fof(0x42b17180u),
                ln2_hi = fof(0x3f317180u), ln2_lo = fof(0x3717f7d1u), invln2 = fof(0x3fb8aa3bu),
                Q1 = fof(0xbd088889u), Q2 = fof(0x3ad00d01u), Q3 = fof(0xb8a670cdu), Q4 = fof(0x36867e54u),
                Q5 = fof(0xb457edbbu);
    float y, hi, lo, c = 0.0f, t, e, hxs, hfx, r1;
    int32_t k;
    uint32_t hx = fbits(x);
    const uint32_t xsb = hx & 0x80000000u;
    hx &= 0x7fffffffu;
    if (hx >= 0x4195b844u) {  // |x| >= 27 ln2
        if (hx >= 0x42b17218u) {
            if (hx > 0x7f800000u) return x + x;
            if (hx == 0x7f800000u) return xsb == 0 ? x : -1.0f;
            if (x > o_threshold) return huge * huge;
        }
        if (xsb != 0 && x + tiny < 0.0f) return tiny - one;
    }
    if (hx > 0x3eb17218u) {      // |x| > ln2/2
        if (hx < 0x3F851592u) {  // and < 3 ln2/2
            if (xsb == 0) {
                hi = x - ln2_hi;
                lo = ln2_lo;
                k = 1;
            } else {
                hi = x + ln2_hi;
                lo = -ln2_lo;
                k = -1;
            }
        } else {
            k = static_cast<int32_t>(invln2 * x + (xsb == 0 ? 0.5f : -0.5f));
            t = static_cast<float>(k);
            hi = x - t * ln2_hi;
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000u) {  // |x| < 2^-25
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
        if (k == 128) y = y * 2.0f * fof(0x7f000000u);
        else y = fof(fbits(y) + (static_cast<uint32_t>(k) << 23));
        return y - one;
    }
    if (k < 23) {
        t = fof(0x3f800000u - (0x1000000u >> k));  // 1 - 2^-k
        y = t - (e - x);
    } else {
        t = fof(static_cast<uint32_t>(0x7f - k) << 23);  // 2^-k
        y = x - (e + t);
        y += one;
    }
    return fof(fbits(y) + (static_cast<uint32_t>(k) << 23));
}

// tanh (fdlibm): 1 - 2/(expm1(2|x|) + 2) for |x| >= 1, -t/(t + 2) with
// t = expm1(-2|x|) below, 1 past 22; the sign restored.
__device__ __forceinline__ float tanhf_fdlibm(float x) {
    const float one = 1.0f, two = 2.0f, tiny = 1.0e-30f;
    float t, z;
    const int32_t jx = static_cast<int32_t>(fbits(x)), ix = jx & 0x7fffffff;
    if (ix >= 0x7f800000) return jx >= 0 ? one / x + one : one / x - one;
    if (ix < 0x41b00000) {  // |x| < 22
        if (ix == 0) return x;
        if (ix < 0x24000000) return x * (one + x);  // |x| < 2^-55
        if (ix >= 0x3f800000) {
            t = expm1f_fdlibm(two * __builtin_fabsf(x));
            z = one - two / (t + two);
        } else {
            t = expm1f_fdlibm(-two * __builtin_fabsf(x));
            z = -t / (t + two);
        }
    } else {
        z = one - tiny;
    }
    return jx >= 0 ? z : -z;
}

}  // namespace libm
}  // namespace tship
