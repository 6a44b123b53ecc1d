/* kernels.c — restatement of the as-built x86-64 reference kernels.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker, never the product.
 *
 * Numerics: compiled with -std=c11 -O2 -ffp-contract=off and no -march, like
 * the reference's ingot build (third_party/ingot/Makefile:8). Every product
 * and sum below is a separate IEEE f32 operation, in the reference's order.
 *
 * SPDX-License-Identifier: MIT */
#include "oracle.h"

#include <math.h>
#include <string.h>

#define QK 256

/* third_party/ingot/src/kernels.c:57-59 and 61-79 (kernel-local f16 decode:
 * exact, subnormals normalised, NaN payload passed through unquieted). */
static uint16_t le16(const unsigned char *p) {
    return (uint16_t)(p[0] | (p[1] << 8));
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 31u;
    uint32_t man = h & 1023u;
    uint32_t out;
    if (exp == 31u) {
        out = sign | 0x7f800000u | (man << 13);
    } else if (exp != 0u) {
        out = sign | ((exp + 112u) << 23) | (man << 13);
    } else if (man == 0u) {
        out = sign;
    } else {
        /* subnormal: shift the leading one up to bit 10, one exponent step
         * per shift, starting from the f16 subnormal exponent (-14). */
        int e = -14;
        while ((man & 1024u) == 0u) { man <<= 1; e--; }
        out = sign | ((uint32_t)(e + 127) << 23) | ((man & 1023u) << 13);
    }
    float f;
    memcpy(&f, &out, sizeof f);
    return f;
}

/* third_party/ingot/src/kernels.c:81-92: the 6-bit (scale, min) pair of
 * sub-block j from the 12-byte packed field. */
void orc_scale_min(const unsigned char *s, int j, unsigned char *sc, unsigned char *m) {
    if (j < 4) {
        *sc = s[j] & 63u;
        *m = s[j + 4] & 63u;
        return;
    }
    *sc = (unsigned char)((s[j + 4] & 15u) | ((s[j - 4] >> 6) << 4));
    *m = (unsigned char)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
}

/* third_party/ingot/src/dtype.c:37-83 for the five formats restated here. */
int orc_type_geometry(int type, uint64_t *block_elems, uint64_t *block_bytes) {
    switch (type) {
    case ORC_Q4_K: *block_elems = 256; *block_bytes = 144; return 0;
    case ORC_Q5_K: *block_elems = 256; *block_bytes = 176; return 0;
    case ORC_Q6_K: *block_elems = 256; *block_bytes = 210; return 0;
    case ORC_Q8_0: *block_elems = 32;  *block_bytes = 34;  return 0;
    case ORC_Q4_0: *block_elems = 32;  *block_bytes = 18;  return 0;
    default: return -1;
    }
}

int orc_has_kernel(int type) {
    uint64_t e, b;
    return orc_type_geometry(type, &e, &b) == 0;
}

/* ── Q4_K ─────────────────────────────────────────────────────────────────
 * Block: d f16 @0, dmin f16 @2, scales[12] @4, qs[128] @16. Group g = 0..3
 * reads qs[32g .. 32g+31]: low nibble -> weight 64g+i (sub-block 2g), high
 * nibble -> weight 64g+32+i (sub-block 2g+1). */

/* third_party/ingot/src/kernels.c:94-115 (dot_block): one running f32 sum,
 * the low-nibble term then the high-nibble term for each i. */
static float q4_k_block_dot(const unsigned char *blk, const float *x) {
    const float d = orc_f16_to_f32(le16(blk));
    const float dmin = orc_f16_to_f32(le16(blk + 2));
    const unsigned char *qs = blk + 16;
    float acc = 0.0f;
    for (int g = 0; g < 4; g++) {
        unsigned char sa, ma, sb, mb;
        orc_scale_min(blk + 4, 2 * g, &sa, &ma);
        orc_scale_min(blk + 4, 2 * g + 1, &sb, &mb);
        const float da = d * (float)sa, db = d * (float)sb;
        const float oa = dmin * (float)ma, ob = dmin * (float)mb;
        const float *xa = x + 64 * g, *xb = xa + 32;
        for (int i = 0; i < 32; i++) {
            const unsigned q = qs[32 * g + i];
            const float wa = da * (float)(q & 15u) - oa;
            acc = acc + wa * xa[i];
            const float wb = db * (float)(q >> 4) - ob;
            acc = acc + wb * xb[i];
        }
    }
    return acc;
}

/* third_party/ingot/src/kernels.c:117-136 (dequant_block). */
static void q4_k_block_decode(const unsigned char *blk, float *w) {
    const float d = orc_f16_to_f32(le16(blk));
    const float dmin = orc_f16_to_f32(le16(blk + 2));
    const unsigned char *qs = blk + 16;
    for (int g = 0; g < 4; g++) {
        unsigned char sa, ma, sb, mb;
        orc_scale_min(blk + 4, 2 * g, &sa, &ma);
        orc_scale_min(blk + 4, 2 * g + 1, &sb, &mb);
        const float da = d * (float)sa, db = d * (float)sb;
        const float oa = dmin * (float)ma, ob = dmin * (float)mb;
        for (int i = 0; i < 32; i++) {
            const unsigned q = qs[32 * g + i];
            w[64 * g + i] = da * (float)(q & 15u) - oa;
            w[64 * g + 32 + i] = db * (float)(q >> 4) - ob;
        }
    }
}

/* ── Q5_K ─────────────────────────────────────────────────────────────────
 * Block: d f16 @0, dmin f16 @2, scales[12] @4 (Q4_K's packing), qh[32] @16,
 * qs[128] @48. Group g = 0..3 reads qs[32g .. 32g+31]: low nibble plus 16 when
 * bit 2g of qh[i] is set -> weight 64g+i (sub-block 2g); high nibble plus 16
 * when bit 2g+1 of qh[i] is set -> weight 64g+32+i (sub-block 2g+1). */

/* third_party/ingot/src/kernels.c:1785-1810 (q5_dot_block, the lane of a
 * build without -march): one running f32 sum per super-block, the low term
 * then the high term for each i; weight (d*sc)*q - dmin*m. */
static float q5_k_block_dot(const unsigned char *blk, const float *x) {
    const float d = orc_f16_to_f32(le16(blk));
    const float dmin = orc_f16_to_f32(le16(blk + 2));
    const unsigned char *qh = blk + 16, *qs = blk + 48;
    float acc = 0.0f;
    for (int g = 0; g < 4; g++) {
        unsigned char sa, ma, sb, mb;
        orc_scale_min(blk + 4, 2 * g, &sa, &ma);
        orc_scale_min(blk + 4, 2 * g + 1, &sb, &mb);
        const float da = d * (float)sa, db = d * (float)sb;
        const float oa = dmin * (float)ma, ob = dmin * (float)mb;
        const float *xa = x + 64 * g, *xb = xa + 32;
        for (int i = 0; i < 32; i++) {
            const unsigned q = qs[32 * g + i], h = qh[i];
            const unsigned lo = (q & 15u) + (((h >> (2 * g)) & 1u) << 4);
            const unsigned hi = (q >> 4) + (((h >> (2 * g + 1)) & 1u) << 4);
            const float wa = da * (float)lo - oa;
            acc = acc + wa * xa[i];
            const float wb = db * (float)hi - ob;
            acc = acc + wb * xb[i];
        }
    }
    return acc;
}

/* third_party/ingot/src/kernels.c:1812-1833 (q5_dequant_block). */
static void q5_k_block_decode(const unsigned char *blk, float *w) {
    const float d = orc_f16_to_f32(le16(blk));
    const float dmin = orc_f16_to_f32(le16(blk + 2));
    const unsigned char *qh = blk + 16, *qs = blk + 48;
    for (int g = 0; g < 4; g++) {
        unsigned char sa, ma, sb, mb;
        orc_scale_min(blk + 4, 2 * g, &sa, &ma);
        orc_scale_min(blk + 4, 2 * g + 1, &sb, &mb);
        const float da = d * (float)sa, db = d * (float)sb;
        const float oa = dmin * (float)ma, ob = dmin * (float)mb;
        for (int i = 0; i < 32; i++) {
            const unsigned q = qs[32 * g + i], h = qh[i];
            w[64 * g + i] = da * (float)((q & 15u) + (((h >> (2 * g)) & 1u) << 4)) - oa;
            w[64 * g + 32 + i] = db * (float)((q >> 4) + (((h >> (2 * g + 1)) & 1u) << 4)) - ob;
        }
    }
}

/* ── Q4_0 ─────────────────────────────────────────────────────────────────
 * third_party/ingot/src/kernels.c:2353-2360 (q4_0_dequant_block) and
 * dequant.c:73-83 (dq_q4_0, the same values): d f16 @0, qs[16] @2; weight i
 * (i < 16) is d*((qs[i] & 15) - 8), weight 16+i is d*((qs[i] >> 4) - 8). */
static void q4_0_block_decode(const unsigned char *blk, float *w) {
    const float d = orc_f16_to_f32(le16(blk));
    const unsigned char *q = blk + 2;
    for (int i = 0; i < 16; i++) {
        w[i] = d * (float)((int)(q[i] & 15u) - 8);
        w[16 + i] = d * (float)((int)(q[i] >> 4) - 8);
    }
}

/* ── Q6_K ─────────────────────────────────────────────────────────────────
 * third_party/ingot/src/kernels.c:2176-2199 (q6_dequant_block). Block:
 * ql[128] @0, qh[64] @128, int8 scales[16] @192, d f16 @208. Half h covers
 * weights 128h..128h+127 from ql+64h, qh+32h, scales+8h; within a half,
 * quarter k = 0..3 takes its low 4 bits from ql[i + 32*(k&1)] (low nibble for
 * k < 2, high nibble for k >= 2) and its top 2 bits from qh[i] >> 2k; the
 * scale of weight e (in 0..255) is scales[e / 16]. Value d*sc*(q - 32), the
 * products taken left to right. */
static void q6_k_block_decode(const unsigned char *blk, float *w) {
    const float d = orc_f16_to_f32(le16(blk + 208));
    const signed char *sc = (const signed char *)(blk + 192);
    for (int h = 0; h < 2; h++) {
        const unsigned char *ql = blk + 64 * h, *qh = blk + 128 + 32 * h;
        for (int k = 0; k < 4; k++) {
            for (int i = 0; i < 32; i++) {
                const unsigned lo = (k < 2) ? (ql[i + 32 * (k & 1)] & 15u)
                                            : (ql[i + 32 * (k & 1)] >> 4);
                const unsigned hi = (qh[i] >> (2 * k)) & 3u;
                const int q = (int)(lo | (hi << 4)) - 32;
                const int e = 128 * h + 32 * k + i;
                w[e] = d * (float)sc[e / 16] * (float)q;
            }
        }
    }
}

/* ── Q8_0 ─────────────────────────────────────────────────────────────────
 * third_party/ingot/src/kernels.c:2518-2523: d f16 @0, int8 qs[32] @2,
 * value qs*d. */
static void q8_0_block_decode(const unsigned char *blk, float *w) {
    const float d = orc_f16_to_f32(le16(blk));
    const signed char *qs = (const signed char *)(blk + 2);
    for (int i = 0; i < 32; i++) w[i] = (float)qs[i] * d;
}

/* kernels.c:2635-2639: eight Q8_0 blocks as one 256-wide unit. */
static void q8_0_super_decode(const unsigned char *blk, float *w) {
    for (int b = 0; b < 8; b++) q8_0_block_decode(blk + 34 * b, w + 32 * b);
}

/* third_party/ingot/src/kernels.c:2037-2041 (qk_dot_scalar): sequential. */
static float seq_dot(const float *a, const float *b, size_t n) {
    float s = 0.0f;
    for (size_t i = 0; i < n; i++) s = s + a[i] * b[i];
    return s;
}

/* Shared geometry check (third_party/ingot/src/generic.c:50-62). */
static int row_bytes_of(int type, size_t rows, size_t cols, size_t *rb) {
    uint64_t e, b;
    if (rows == 0 || cols == 0 || orc_type_geometry(type, &e, &b) != 0) return -1;
    if (cols % e != 0) return -1;
    *rb = (size_t)(cols / e * b);
    if (rows > SIZE_MAX / *rb || rows > SIZE_MAX / cols) return -1;
    return 0;
}

/* The reference's matrix dequant goes through kquant_apply in 256-wide units
 * for Q4_K, Q6_K and Q8_0 (kernels.c:2096-2101, 2563-2567), so a Q8_0 row
 * that is not a whole number of 256-value units is refused (-1); Q5_K
 * (kernels.c:1941-1959) is whole super-blocks anyway, and Q4_0
 * (kernels.c:2500-2514) takes any multiple of 32. */
int orc_dequant_matrix(int type, const void *w, size_t rows, size_t cols, float *y) {
    size_t rb;
    if (w == NULL || y == NULL || row_bytes_of(type, rows, cols, &rb) != 0) return -1;
    if (type != ORC_Q4_0 && cols % QK != 0) return -1;
    const unsigned char *base = (const unsigned char *)w;
    for (size_t r = 0; r < rows; r++) {
        const unsigned char *row = base + r * rb;
        float *out = y + r * cols;
        if (type == ORC_Q4_K)
            for (size_t b = 0; b < cols / QK; b++) q4_k_block_decode(row + 144 * b, out + QK * b);
        else if (type == ORC_Q5_K)
            for (size_t b = 0; b < cols / QK; b++) q5_k_block_decode(row + 176 * b, out + QK * b);
        else if (type == ORC_Q4_0)
            for (size_t b = 0; b < cols / 32; b++) q4_0_block_decode(row + 18 * b, out + 32 * b);
        else if (type == ORC_Q6_K)
            for (size_t b = 0; b < cols / QK; b++) q6_k_block_decode(row + 210 * b, out + QK * b);
        else
            for (size_t b = 0; b < cols / 32; b++) q8_0_block_decode(row + 34 * b, out + 32 * b);
    }
    return 0;
}

/* matvec lanes of the as-built reference:
 *   Q4_K kernels.c:319-337: y[r] = sum over blocks (in order) of dot_block;
 *   Q5_K kernels.c:1835-1853: the same with q5_dot_block;
 *   Q6_K kernels.c:2096-2124 with 2305-2318: per block decode 256 values,
 *        then a sequential dot, added to the row sum;
 *   Q8_0 kernels.c:2525-2546: the same per 32-value block;
 *   Q4_0 kernels.c:2467-2484: ONE running sum over the whole row, no
 *        per-block partials. */
int orc_matvec(int type, const void *w, size_t rows, size_t cols,
               const float *x, float *y) {
    size_t rb;
    if (w == NULL || x == NULL || y == NULL || row_bytes_of(type, rows, cols, &rb) != 0)
        return -1;
    const unsigned char *base = (const unsigned char *)w;
    float tmp[QK];
    for (size_t r = 0; r < rows; r++) {
        const unsigned char *row = base + r * rb;
        float sum = 0.0f;
        if (type == ORC_Q4_K) {
            for (size_t b = 0; b < cols / QK; b++)
                sum = sum + q4_k_block_dot(row + 144 * b, x + QK * b);
        } else if (type == ORC_Q5_K) {
            for (size_t b = 0; b < cols / QK; b++)
                sum = sum + q5_k_block_dot(row + 176 * b, x + QK * b);
        } else if (type == ORC_Q4_0) {
            for (size_t b = 0; b < cols / 32; b++) {
                q4_0_block_decode(row + 18 * b, tmp);
                for (int i = 0; i < 32; i++) sum = sum + tmp[i] * x[32 * b + i];
            }
        } else if (type == ORC_Q6_K) {
            for (size_t b = 0; b < cols / QK; b++) {
                q6_k_block_decode(row + 210 * b, tmp);
                sum = sum + seq_dot(tmp, x + QK * b, QK);
            }
        } else {
            for (size_t b = 0; b < cols / 32; b++) {
                q8_0_block_decode(row + 34 * b, tmp);
                sum = sum + seq_dot(tmp, x + 32 * b, 32);
            }
        }
        y[r] = sum;
    }
    return 0;
}

/* Batched exact matmat (kernels.c:1030-1104 with the scalar branch of
 * qk_gemm_block, 1017-1026): for each (row, token) the accumulator starts at
 * zero and adds, per 256-wide super-block in order, the sequential dot of the
 * decoded 256 values with the token's slice. Token tiles and row strips only
 * change which (row, token) pairs are in flight, never this order.
 * tokens == 1 is the matvec (kernels.c:1726-1727, 2627-2648). Q5_K takes the
 * same core with its own decoder (kernels.c:2573-2595).
 *
 * Q4_0 has no batched kernel: ingot_matmat runs its generic path
 * (third_party/ingot/src/generic.c:76-93): each row decoded whole, then per
 * token one running sum over all cols in order — the matvec's chain. */
static void matmat_rows(int type, const unsigned char *base, size_t rb, size_t r0,
                        size_t r1, size_t rows, size_t cols, const float *x,
                        float *y, size_t tokens) {
    float dec[QK];
    if (type == ORC_Q4_0) {
        for (size_t r = r0; r < r1; r++) {
            const unsigned char *row = base + r * rb;
            for (size_t t = 0; t < tokens; t++) {
                float sum = 0.0f;
                for (size_t b = 0; b < cols / 32; b++) {
                    q4_0_block_decode(row + 18 * b, dec);
                    for (int i = 0; i < 32; i++) sum = sum + dec[i] * x[t * cols + 32 * b + i];
                }
                y[t * rows + r] = sum;
            }
        }
        return;
    }
    for (size_t r = r0; r < r1; r++) {
        const unsigned char *row = base + r * rb;
        for (size_t t = 0; t < tokens; t++) y[t * rows + r] = 0.0f;
        for (size_t b = 0; b < cols / QK; b++) {
            if (type == ORC_Q4_K) q4_k_block_decode(row + 144 * b, dec);
            else if (type == ORC_Q5_K) q5_k_block_decode(row + 176 * b, dec);
            else if (type == ORC_Q6_K) q6_k_block_decode(row + 210 * b, dec);
            else q8_0_super_decode(row + 272 * b, dec);
            for (size_t t = 0; t < tokens; t++)
                y[t * rows + r] = y[t * rows + r] + seq_dot(dec, x + t * cols + QK * b, QK);
        }
    }
}

static int matmat_check(int type, const void *w, size_t rows, size_t cols,
                        const float *x, const float *y, size_t tokens, size_t *rb) {
    if (w == NULL || x == NULL || y == NULL || tokens == 0) return -1;
    if (row_bytes_of(type, rows, cols, rb) != 0) return -1;
    /* the batched core works in 256-wide units; Q4_0's generic path does not */
    if (type != ORC_Q4_0 && cols % QK != 0) return -1;
    if (tokens > SIZE_MAX / rows) return -1;
    return 0;
}

int orc_matmat(int type, const void *w, size_t rows, size_t cols,
               const float *x, float *y, size_t tokens) {
    if (tokens == 1) return orc_matvec(type, w, rows, cols, x, y);
    size_t rb;
    if (matmat_check(type, w, rows, cols, x, y, tokens, &rb) != 0) return -1;
    matmat_rows(type, (const unsigned char *)w, rb, 0, rows, rows, cols, x, y, tokens);
    return 0;
}

/* ── the CPU-baseline threading ───────────────────────────────────────────── */
/* ── the AVX2 + FMA lanes (the secondary CPU baseline) ─────────────────────
 * What an ingot build with -mavx2 -mfma takes (INGOT_SDOT unset):
 *   Q4_K kernels.c:455-506 (q4_k_dot_block_avx2): eight lane accumulators;
 *        per 64-weight group and 8-weight step, lane j adds fma(low weight,
 *        x, acc[j]) then fma(high weight, x + 32, acc[j]); the weight is
 *        q * (d sc) - dmin m with both steps rounded (the reference builds
 *        with -std=c11, so no contraction); the eight lanes are then summed
 *        in order from 0, and the row sum adds the block sums in order;
 *   Q6_K kernels.c:2062-2081 (qk_dot_avx2) over the decoded block: four
 *        8-lane accumulators over steps of 32, the lanes (acc0 + acc1) +
 *        (acc2 + acc3), the 128-bit halves added, then (s0 + s2) + (s1 + s3);
 *   Q8_0 the same dot over each 32-value block.
 * Compiled for AVX2 + FMA (the loops over the eight lanes vectorise, fmaf is
 * one instruction) so the timing is an AVX2 build's; operation order per lane
 * is as written (no contraction, no reassociation). */
#define AVX2_LANES __attribute__((target("avx2,fma"), optimize("O3")))

AVX2_LANES static float q4_k_block_dot_avx2(const unsigned char *blk, const float *x) {
    const float d = orc_f16_to_f32(le16(blk));
    const float dmin = orc_f16_to_f32(le16(blk + 2));
    const unsigned char *qs = blk + 16;
    float acc[8] = {0};
    for (int g = 0; g < 4; g++) {
        unsigned char sa, ma, sb, mb;
        orc_scale_min(blk + 4, 2 * g, &sa, &ma);
        orc_scale_min(blk + 4, 2 * g + 1, &sb, &mb);
        const float d0 = d * (float)sa, d1 = d * (float)sb;
        const float m0 = dmin * (float)ma, m1 = dmin * (float)mb;
        for (int i = 0; i < 32; i += 8)
            for (int j = 0; j < 8; j++) {
                const unsigned q = qs[32 * g + i + j];
                const float lo = (float)(q & 15u) * d0 - m0;
                const float hi = (float)(q >> 4) * d1 - m1;
                acc[j] = fmaf(lo, x[64 * g + i + j], acc[j]);
                acc[j] = fmaf(hi, x[64 * g + i + j + 32], acc[j]);
            }
    }
    float sum = 0.0f;
    for (int j = 0; j < 8; j++) sum = sum + acc[j];
    return sum;
}

AVX2_LANES static float dot_avx2_order(const float *a, const float *b, size_t n) {
    float c[4][8] = {{0}};
    size_t i = 0;
    for (; i + 32 <= n; i += 32)
        for (int k = 0; k < 4; k++)
            for (int j = 0; j < 8; j++)
                c[k][j] = fmaf(a[i + 8 * k + j], b[i + 8 * k + j], c[k][j]);
    float acc[8], s[4];
    for (int j = 0; j < 8; j++) acc[j] = (c[0][j] + c[1][j]) + (c[2][j] + c[3][j]);
    for (int j = 0; j < 4; j++) s[j] = acc[j] + acc[j + 4];
    float sum = (s[0] + s[2]) + (s[1] + s[3]);
    for (; i < n; i++) sum = sum + a[i] * b[i];
    return sum;
}

AVX2_LANES static void matvec_avx2_rows(int type, const unsigned char *base, size_t rb,
                                        size_t rows, size_t cols, const float *x, float *y) {
    float tmp[QK];
    for (size_t r = 0; r < rows; r++) {
        const unsigned char *row = base + r * rb;
        float sum = 0.0f;
        if (type == ORC_Q4_K) {
            for (size_t b = 0; b < cols / QK; b++)
                sum = sum + q4_k_block_dot_avx2(row + 144 * b, x + QK * b);
        } else if (type == ORC_Q6_K) {
            for (size_t b = 0; b < cols / QK; b++) {
                q6_k_block_decode(row + 210 * b, tmp);
                sum = sum + dot_avx2_order(tmp, x + QK * b, QK);
            }
        } else {
            for (size_t b = 0; b < cols / 32; b++) {
                q8_0_block_decode(row + 34 * b, tmp);
                sum = sum + dot_avx2_order(tmp, x + 32 * b, 32);
            }
        }
        y[r] = sum;
    }
}

int orc_matvec_avx2(int type, const void *w, size_t rows, size_t cols,
                    const float *x, float *y) {
    size_t rb;
    if (!__builtin_cpu_supports("avx2") || !__builtin_cpu_supports("fma")) return -1;
    if (w == NULL || x == NULL || y == NULL || row_bytes_of(type, rows, cols, &rb) != 0 ||
        (type != ORC_Q4_K && type != ORC_Q6_K && type != ORC_Q8_0))
        return -1;
    matvec_avx2_rows(type, (const unsigned char *)w, rb, rows, cols, x, y);
    return 0;
}

void orc_pool_run(int n, void (*fn)(void *, int), void *ctx);

typedef int (*matvec_fn)(int, const void *, size_t, size_t, const float *, float *);

typedef struct {
    int type;
    const unsigned char *base;
    size_t rb, rows, cols, per;
    const float *x;
    float *y;
    int rc;
    matvec_fn mv;
} project_job;

static void project_chunk(void *ctx, int i) {
    project_job *j = (project_job *)ctx;
    const size_t first = (size_t)i * j->per;
    if (first >= j->rows) return;
    size_t n = j->per;
    if (first + n > j->rows) n = j->rows - first;
    if (j->mv(j->type, j->base + first * j->rb, n, j->cols, j->x, j->y + first) != 0)
        j->rc = -1;
}

/* src/arch_qwen3.c:52-83: 4*nth contiguous chunks of output rows, each an
 * independent matvec; serial when nth <= 1 or rows < 64. */
static int project_with(matvec_fn mv, int type, const void *w, size_t rows, size_t cols,
                        const float *x, float *y) {
    const int nth = orc_threads_count();
    size_t rb;
    if (nth <= 1 || rows < 64 || row_bytes_of(type, rows, cols, &rb) != 0)
        return mv(type, w, rows, cols, x, y);
    int chunks = nth * 4;
    if ((size_t)chunks > rows) chunks = (int)rows;
    project_job j = { type, (const unsigned char *)w, rb, rows, cols,
                      (rows + (size_t)chunks - 1) / (size_t)chunks, x, y, 0, mv };
    orc_pool_run(chunks, project_chunk, &j);
    return j.rc;
}

int orc_project(int type, const void *w, size_t rows, size_t cols,
                const float *x, float *y) {
    return project_with(orc_matvec, type, w, rows, cols, x, y);
}

int orc_project_avx2(int type, const void *w, size_t rows, size_t cols,
                     const float *x, float *y) {
    return project_with(orc_matvec_avx2, type, w, rows, cols, x, y);
}

typedef struct {
    int type;
    const unsigned char *base;
    size_t rb, rows, cols, tokens;
    const float *x;
    float *y;
} strip_job;

static void strip_task(void *ctx, int s) {
    strip_job *j = (strip_job *)ctx;
    const size_t r0 = (size_t)s * 8;
    const size_t r1 = r0 + 8 < j->rows ? r0 + 8 : j->rows;
    matmat_rows(j->type, j->base, j->rb, r0, r1, j->rows, j->cols, j->x, j->y, j->tokens);
}

int orc_matmat_mt(int type, const void *w, size_t rows, size_t cols,
                  const float *x, float *y, size_t tokens) {
    if (tokens == 1) return orc_project(type, w, rows, cols, x, y);
    size_t rb;
    if (matmat_check(type, w, rows, cols, x, y, tokens, &rb) != 0) return -1;
    strip_job j = { type, (const unsigned char *)w, rb, rows, cols, tokens, x, y };
    orc_pool_run((int)((rows + 7) / 8), strip_task, &j);
    return 0;
}
