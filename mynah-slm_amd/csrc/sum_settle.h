/* sum_settle.h — whether a double sum taken in a parallel order gives the
 * reference's f32 result, shared by the kernels (common.hip.h) and a host
 * build of the same test (oracle/settle_pin.c).
 *
 * The reference adds n non-negative terms, each exact in double, in index
 * order: the squares of RMSNorm (src/kernels.c:118-121) and the softmax's
 * exponentials (:213-218). Any order of such a sum lies within γ(n − 1) S
 * of the exact sum S, γ(k) = k u / (1 − k u), u = 2^-53 (Higham, Accuracy
 * and Stability of Numerical Algorithms, 2nd ed., §4.2: the bound holds for
 * every summation order), and so does the reference's. From a sum s in a
 * parallel order the reference's is s (1 + η) with |η| <= d = 2 γ / (1 − γ)
 * = 2 g / (1 − 2 g), g = (n − 1) u.
 *
 * The kernels use such a sum only through r = 1 / sum (softmax) or
 * r = 1 / sqrt(sum / n + eps) (RMSNorm), each operation correctly rounded,
 * and then the f32 rounding of r. Computed at s (1 + η) instead of s, r
 * moves by a factor within 1 ± (k d + 2 d²) of the real function (k = 1 for
 * the reciprocal; k = 1/2 for the inverse square root, whose argument
 * moves by at most the sum's relative change since eps > 0), and each
 * computed r is within 3 u of its real value (three roundings at most, the
 * first of an addition of two non-negative terms). So every r the
 * reference can compute lies within e r of this one, e = k d (1 + 2^-19)
 * + 12 u for n <= 2^20 (2^-19 covers 2 d² and 1 / (1 − 2 g) − 1). With r
 * in [2^E, 2^(E+1)) a double ulp is 2^(E−52) >= r 2^-53, so that distance
 * is at most T = e 2^53 ulps of r. The f32 rounding changes only at the
 * midpoints between f32 values, which in r's binade have low 29 mantissa
 * bits 2^28, the nearest ones outside it at least 2^27 ulps away (so for
 * T < 2^27, n <= 2^20, those never matter): when the low 29 bits of r are
 * more than T from 2^28, every r within T ulps rounds to the same f32, and
 * so does the reference's. Otherwise — about 2 T / 2^29 of the sums, 1 in
 * 10^5 for n = 2,560 — the kernel adds the terms again in index order
 * (seq_sumsq, seq_sum in common.hip.h); also for an r outside the normal
 * f32 range or not finite.
 *
 * mynah_sum_settled(hi, lo, n, k2): nonzero when it holds for r with bits
 * (hi << 32) | lo, a sum of n terms and k2 = 2 k (2 for the reciprocal, 1
 * for the inverse square root).
 *
 * SPDX-License-Identifier: MIT */
#ifndef MYNAH_SUM_SETTLE_H
#define MYNAH_SUM_SETTLE_H
#include <stdint.h>

#if defined(__HIPCC__)
#define MYNAH_SETTLE_FN static __host__ __device__ __forceinline__
#else
#define MYNAH_SETTLE_FN static inline
#endif

/* Branch-free (the kernels take one branch on the result): the distance of
 * the low 29 bits from 2^28 is the smaller of the two unsigned differences;
 * the exponent range and the sign are one unsigned compare of the top 12
 * bits (a set sign bit puts them past the range). */
MYNAH_SETTLE_FN int mynah_sum_settled(uint32_t hi, uint32_t lo, uint32_t n, uint32_t k2) {
    const uint32_t low = lo & 0x1fffffffu;
    const uint32_t a = low - (1u << 28), b = (1u << 28) - low;
    const uint32_t dist = a < b ? a : b;
    const uint32_t w = k2 * (n - (n > 0u ? 1u : 0u));
    const uint32_t t = w + (w >> 18) + 13u;
    const int range = (hi >> 20) - (1023u - 125u) <= 251u;
    return (n <= (1u << 20)) & range & (dist > t);
}

#endif
