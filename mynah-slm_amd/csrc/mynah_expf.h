/* mynah_expf.h — expf with the exact bits of the reference's C library.
 *
 * The reference's f32 operators call expf from glibc (softmax,
 * src/kernels.c:207-220; the stable sigmoid, :193-205). The GPU's own expf
 * is accurate to about one ulp but rounds differently in many cases, which
 * moves whole logit vectors by ~1e-4 of the reference over a deep model.
 * This is glibc 2.35's method (the expf of Arm's optimized-routines):
 *   x * 32 / ln 2 = k + r with k integral (ties to even, through the
 *   1.5 * 2^52 shift) and |r| <= 1/2, taken in double as one fused
 *   multiply-add, then r = that product minus k as a second fused one;
 *   2^(k/32) from a 32-entry table of 2^(i/32) (the correctly rounded
 *   doubles, biased by -(i << 47) so that adding k << 47 places the
 *   exponent);
 *   2^(r/32) = (c0 r + c1) r^2 + (c2 r + 1), both linear terms and the
 *   outer sum as fused multiply-adds, with the method's published minimax
 *   coefficients;
 *   one final rounding of the double product to float; |x| >= 88 takes
 *   the special cases (-inf -> 0, NaN and +inf -> x + x, overflow -> +inf,
 *   x < -103.97 -> +0).
 * These are the fused forms of the x86-64 build that runs on FMA hosts.
 * tests/test_expf.py compares every float in (-110, 90) with the C
 * library's expf, bit for bit, on the CPU; the GPU tests do the same on the
 * device through mynah_hip_expf_dev.
 *
 * The header serves the device code (HIP) and the CPU pin (C11).
 *
 * SPDX-License-Identifier: MIT */
#ifndef MYNAH_EXPF_H
#define MYNAH_EXPF_H

#include <stdint.h>

#if defined(__HIPCC__)
#define MYNAH_EXPF_FN __device__ __forceinline__
#define MYNAH_EXPF_TAB __constant__
#define MYNAH_FMA64(a, b, c) __builtin_fma((a), (b), (c))
#else
#include <math.h>
#define MYNAH_EXPF_FN static inline
#define MYNAH_EXPF_TAB static const
#define MYNAH_FMA64(a, b, c) fma((a), (b), (c))
#endif

/* 2^(i/32) rounded to double, minus i << 47. */
MYNAH_EXPF_TAB uint64_t mynah_exp2_tab[32] = {
0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull
};

/* mynah_expf with the table read through `tab` (the 32 entries of
 * mynah_exp2_tab, e.g. a copy in GPU shared memory, whose reads do not wait
 * behind the wave's outstanding global loads). */
MYNAH_EXPF_FN float mynah_expf_t(float x, const uint64_t *tab) {
    uint32_t xb;
    __builtin_memcpy(&xb, &x, 4);
    const uint32_t abstop = (xb >> 20) & 0x7ffu;
    const double shift = 0x1.8p+52, inv_ln2_32 = 0x1.71547652b82fep+0 * 32.0;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = MYNAH_FMA64(inv_ln2_32, xd, shift);
    uint64_t ki;
    __builtin_memcpy(&ki, &kd, 8);
    kd -= shift;
    const double r = MYNAH_FMA64(inv_ln2_32, xd, -kd);
    const uint64_t t = tab[ki % 32u] + (ki << 47);
    double s;
    __builtin_memcpy(&s, &t, 8);
    const double z = MYNAH_FMA64(c0, r, c1), r2 = r * r;
    double y = MYNAH_FMA64(c2, r, 1.0);
    y = MYNAH_FMA64(z, r2, y);
    y = y * s;
    /* The special cases of |x| >= 88 or NaN, taken after the main path
     * (whose result they replace; its table index is in range whatever x
     * is), so that no lane branches: -inf -> 0 before NaN and +inf -> x + x,
     * before overflow -> +inf, before underflow -> +0. */
    float out = (float)y;
    if (abstop >= 0x42bu) {
        out = x < -0x1.9fe368p6f ? 0.0f : out;
        out = x > 0x1.62e42ep6f ? __builtin_inff() : out;
        out = abstop >= 0x7f8u ? x + x : out;
        out = xb == 0xff800000u ? 0.0f : out;
    }
    return out;
}

MYNAH_EXPF_FN float mynah_expf(float x) { return mynah_expf_t(x, mynah_exp2_tab); }

#endif
