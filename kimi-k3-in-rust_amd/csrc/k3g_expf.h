/* k3g_expf.h - the engine's float expf, bit for bit, for device and host code.
 *
 * The engine's router and SiTU/SwiGLU call the C library's expf (src/core/k3_ops.c:105,
 * :446-458): glibc 2.35 on the x86-64 hosts it runs on. That expf is not correctly rounded
 * (its documented bound is 0.502 ulp), so a correctly rounded exp disagrees with it on about
 * one input in several thousand, and a router weight computed from such a score is then one
 * ulp off the engine's. This is the published algorithm glibc uses (ARM optimized-routines'
 * expf, Szabolcs Nagy 2017; glibc sysdeps/ieee754/flt-32/e_expf.c with its exp2f table):
 *
 *   x / ln2 * 32 = k + r, k = round-to-nearest-even integer, |r| <= 1/2
 *   expf(x) = (float)(2^(k/32) * p(r)),  p(r) = (C0 r + C1) r^2 + (C2 r + 1)
 *
 * in double, with 2^(i/32) from a 32-entry table (the nearest double to 2^(i/32), minus
 * i << 47 so that adding k << 47 places the exponent) and the minimax coefficients
 * C0..C2 of 2^(r/32). The additions that follow a multiplication are fused
 * (fma), as glibc's FMA build computes them: that build is the one x86-64 glibc selects on
 * every CPU with FMA, and it equals the system expf of this machine on all 2^32 inputs
 * (tests/host/expf_audit.c). The build without FMA differs from it on two inputs.
 * The table entries are checked against 2^(i/32) computed to 60 digits by the same test.
 *
 * Special inputs as glibc: -inf -> 0, +inf and NaN -> x + x, x > 88.72 -> +inf,
 * x < -103.97 -> +0. */
#ifndef K3G_EXPF_H
#define K3G_EXPF_H

#include <stdint.h>

#if defined(__HIPCC__)
#define K3X_FN __host__ __device__ __forceinline__
#else
#include <math.h>
#include <string.h>
#define K3X_FN static inline
#endif

#define K3X_EXPF_N 32

K3X_FN double k3x_asdouble(uint64_t u)
{
#if defined(__HIPCC__)
    return __builtin_bit_cast(double, u);
#else
    double d;
    memcpy(&d, &u, sizeof d);
    return d;
#endif
}

K3X_FN uint64_t k3x_asuint64(double d)
{
#if defined(__HIPCC__)
    return __builtin_bit_cast(uint64_t, d);
#else
    uint64_t u;
    memcpy(&u, &d, sizeof u);
    return u;
#endif
}

K3X_FN uint32_t k3x_asuint(float f)
{
#if defined(__HIPCC__)
    return __builtin_bit_cast(uint32_t, f);
#else
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    return u;
#endif
}

/* nearest double to 2^(i/32), minus i << 47 */
K3X_FN uint64_t k3x_exp2_tab(int i)
{
    static const uint64_t tab[32] = {
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full,
        0x3fef9301d0125b51ull, 0x3fef72b83c7d517bull, 0x3fef54873168b9aaull,
        0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, 0x3fef06fe0a31b715ull,
        0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull,
        0x3feea47eb03a5585ull, 0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull,
        0x3feea11473eb0187ull, 0x3feea589994cce13ull, 0x3feeace5422aa0dbull,
        0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull,
        0x3fef3720dcef9069ull, 0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full,
        0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};
    return tab[i & 31];
}

K3X_FN float k3x_expf(float x)
{
    const uint32_t top = (k3x_asuint(x) >> 20) & 0x7ff;
    if (top >= 0x42b) {                               /* |x| >= 88, inf or NaN */
        if (k3x_asuint(x) == 0xff800000u) return 0.0f;
        if (top >= 0x7f8) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double N = (double)K3X_EXPF_N;
    const double inv = 0x1.71547652b82fep+0 * N;      /* 32 / ln 2 */
    const double shift = 0x1.8p+52;                   /* round-to-integer shift */
    const double c0 = 0x1.c6af84b912394p-5 / N / N / N;
    const double c1 = 0x1.ebfce50fac4f3p-3 / N / N;
    const double c2 = 0x1.62e42ff0c52d6p-1 / N;
    const double xd = (double)x;
    double kd = fma(inv, xd, shift);
    const uint64_t ki = k3x_asuint64(kd);
    kd -= shift;
    const double r = fma(inv, xd, -kd);
    const uint64_t t = k3x_exp2_tab((int)(ki % K3X_EXPF_N)) + (ki << (52 - 5));
    const double s = k3x_asdouble(t);
    const double z = fma(c0, r, c1);
    const double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    y = y * s;
    return (float)y;
}

#endif
