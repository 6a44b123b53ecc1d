/* int8.c — restatement of the reference's int8 activation lane for Q4_K
 * (the x86 rendition that an AVX2 build of ingot compiles).
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker, never the product.
 *
 * The lane exists when ingot is built with -mavx2 -mfma
 * (third_party/ingot/src/kernels.c:30-35, 636-645): the matvec takes it on
 * request (INGOT_SDOT=1, kernels.c:812-838 and ingot_q4_k_matvec_int8
 * 799-810) and the batched matmat by default from two tokens
 * (kernels.c:1700-1751). The as-built x86 reference (ingot with its own -O2,
 * no -march) has neither; this file is the checker for the library's
 * opt-in int8 mode and is pinned against an AVX2 build of the reference.
 *
 * Compiled with -std=c11 -O2 -ffp-contract=off like the rest of the oracle:
 * where the reference uses an FMA intrinsic this file calls fmaf; everywhere
 * else every product and sum is its own rounding, in the reference's order.
 *
 * SPDX-License-Identifier: MIT */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define QK 256

static int32_t sat16(int32_t v) { return v > 32767 ? 32767 : (v < -32768 ? -32768 : v); }
static int8_t sat8(int32_t v) { return (int8_t)(v > 127 ? 127 : (v < -128 ? -128 : v)); }

/* kernels.c:675-708: absmax scale, q = round-half-even(x * (127 / amax)),
 * saturating packs, the eight 32-value sums of the (pre-pack) integers. */
float orc_q8_quantize_block(const float *x, int8_t *q, int32_t sums[8]) {
    float amax = 0.0f;
    for (int i = 0; i < QK; i++) {
        const float a = fabsf(x[i]);
        amax = a > amax ? a : amax;
    }
    if (!(amax > 0.0f)) {
        memset(q, 0, QK);
        memset(sums, 0, 8 * sizeof(*sums));
        return 0.0f;
    }
    const float scale = amax / 127.0f;
    const float inverse = 127.0f / amax;
    for (int g = 0; g < 8; g++) {
        int32_t s = 0;
        for (int i = 0; i < 32; i++) {
            const float v = x[32 * g + i] * inverse;
            const int32_t r = (int32_t)nearbyintf(v);     /* CVTPS2DQ, round to nearest even */
            s += r;
            q[32 * g + i] = sat8(sat16(r));
        }
        sums[g] = s;
    }
    return scale;
}

/* q4_k_nibbles (kernels.c:1129-1153): sub-block j's 32 quants are the low
 * (j even) or high (j odd) nibbles of bytes 32 * (j / 2) .. of the quants. */
static uint32_t nib(const unsigned char *blk, int j, int i) {
    const unsigned char b = blk[16 + 32 * (j / 2) + i];
    return (j & 1) ? (uint32_t)(b >> 4) : (uint32_t)(b & 15u);
}

int32_t orc_q4k_int8_dot(const unsigned char *blk, const int8_t *xq, int j) {
    int32_t d = 0;
    for (int i = 0; i < 32; i++) d += (int32_t)nib(blk, j, i) * (int32_t)xq[32 * j + i];
    return d;
}

/* q5_k_quants (kernels.c:1155-1185): sub-block j's 32 quants are the nibbles
 * of bytes 48 + 32 * (j / 2) .. (low for j even, high for j odd) plus 16
 * when bit j of qh[i] (bytes 16 ..) is set. */
int32_t orc_q5k_int8_dot(const unsigned char *blk, const int8_t *xq, int j) {
    int32_t d = 0;
    for (int i = 0; i < 32; i++) {
        const unsigned char b = blk[48 + 32 * (j / 2) + i];
        const uint32_t q = ((j & 1) ? (uint32_t)(b >> 4) : (uint32_t)(b & 15u)) +
                           ((uint32_t)((blk[16 + i] >> j) & 1u) << 4);
        d += (int32_t)q * (int32_t)xq[32 * j + i];
    }
    return d;
}

static int32_t kq_int8_dot(int type, const unsigned char *blk, const int8_t *xq, int j) {
    return type == ORC_Q5_K ? orc_q5k_int8_dot(blk, xq, j) : orc_q4k_int8_dot(blk, xq, j);
}

/* kernels.c:712-739 (q4_k_dot_block_x86): per group, the low then the high
 * sub-block: total += (d * sc) * dot - (dmin * m) * sum; times the
 * activation scale. */
static float dot_block_int8(const unsigned char *blk, const int8_t *xq, float xscale,
                            const int32_t sums[8]) {
    const float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    const float dmin = orc_f16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
    float total = 0.0f;
    for (int g = 0; g < 4; g++) {
        unsigned char sl, ml, sh, mh;
        orc_scale_min(blk + 4, 2 * g, &sl, &ml);
        orc_scale_min(blk + 4, 2 * g + 1, &sh, &mh);
        const float dl = (float)orc_q4k_int8_dot(blk, xq, 2 * g);
        const float dh = (float)orc_q4k_int8_dot(blk, xq, 2 * g + 1);
        total += d * (float)sl * dl - dmin * (float)ml * (float)sums[2 * g];
        total += d * (float)sh * dh - dmin * (float)mh * (float)sums[2 * g + 1];
    }
    return total * xscale;
}

/* kernels.c:741-772 (ingot_q4_k_matvec_x86int8). */
int orc_q4k_matvec_int8(const void *w, size_t rows, size_t cols, const float *x, float *y) {
    if (w == NULL || x == NULL || y == NULL || rows == 0 || cols == 0 || cols % QK != 0)
        return -1;
    const size_t nb = cols / QK, rb = nb * 144;
    int8_t *q = malloc(cols);
    float *sc = malloc(nb * sizeof *sc);
    int32_t *sums = malloc(nb * 8 * sizeof *sums);
    if (q == NULL || sc == NULL || sums == NULL) {
        free(q); free(sc); free(sums);
        return -1;
    }
    for (size_t b = 0; b < nb; b++) sc[b] = orc_q8_quantize_block(x + b * QK, q + b * QK, sums + 8 * b);
    const unsigned char *base = (const unsigned char *)w;
    for (size_t r = 0; r < rows; r++) {
        float s = 0.0f;
        for (size_t b = 0; b < nb; b++)
            s += dot_block_int8(base + r * rb + b * 144, q + b * QK, sc[b], sums + 8 * b);
        y[r] = s;
    }
    free(q); free(sc); free(sums);
    return 0;
}

/* kernels.c:893-920 (qk_token_tile, no INGOT_QK_TILE override). */
static size_t token_tile(size_t cols) {
    size_t tile = (4u << 20) / (cols * sizeof(float));
    if (tile > 128) tile = 128;
    if (tile < 32) tile = 32;
    tile &= ~(size_t)1;
    return tile < 2 ? 2 : tile;
}

/* kernels.c:1495-1581 (qk_matmat_rows_x86) and 1591-1679 (qk_matmat_sdot):
 * the activations quantised once per (token, super-block); per super-block
 * and row, tokens of a tile in groups of four take the FMA epilogue
 * (total = fma(dot, scale, total); total = fma(-xsum, offset, total)), the
 * rest of the tile the plain one (total += scale * dot - offset * xsum); the
 * super-block's total times the activation scale is added to the output.
 * tokens == 1 is the matvec (kernels.c:1726), which with INGOT_SDOT=1 is the
 * int8 matvec above (kernels.c:819-834). */
static int kq_matmat_int8(int type, const void *w, size_t rows, size_t cols, const float *x,
                          float *y, size_t tokens) {
    if (w == NULL || x == NULL || y == NULL || rows == 0 || cols == 0 || tokens == 0 ||
        cols % QK != 0)
        return -1;
    const size_t ub = type == ORC_Q5_K ? 176 : 144;
    const size_t nb = cols / QK, rb = nb * ub;
    int8_t *q = malloc(tokens * cols);
    float *xs = malloc(nb * tokens * sizeof *xs);
    float *xsum = malloc(nb * 8 * tokens * sizeof *xsum);
    float *acc = malloc(tokens * sizeof *acc);
    if (q == NULL || xs == NULL || xsum == NULL || acc == NULL) {
        free(q); free(xs); free(xsum); free(acc);
        return -1;
    }
    for (size_t t = 0; t < tokens; t++)
        for (size_t b = 0; b < nb; b++) {
            int32_t s8[8];
            xs[b * tokens + t] = orc_q8_quantize_block(x + t * cols + b * QK, q + t * cols + b * QK, s8);
            for (int j = 0; j < 8; j++) xsum[(b * 8 + (size_t)j) * tokens + t] = (float)s8[j];
        }
    const size_t tile = token_tile(cols);
    const unsigned char *base = (const unsigned char *)w;
    for (size_t r = 0; r < rows; r++) {
        for (size_t t0 = 0; t0 < tokens; t0 += tile) {
            const size_t cnt = tokens - t0 < tile ? tokens - t0 : tile;
            for (size_t t = 0; t < cnt; t++) acc[t] = 0.0f;
            for (size_t b = 0; b < nb; b++) {
                const unsigned char *blk = base + r * rb + b * ub;
                const float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
                const float dmin = orc_f16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
                float scale[8], offset[8];
                for (int j = 0; j < 8; j++) {
                    unsigned char s, m;
                    orc_scale_min(blk + 4, j, &s, &m);
                    scale[j] = d * (float)s;
                    offset[j] = dmin * (float)m;
                }
                size_t t = 0;
                for (; t + 4 <= cnt; t += 4)
                    for (size_t k = 0; k < 4; k++) {
                        const size_t tt = t0 + t + k;
                        float total = 0.0f;
                        for (int j = 0; j < 8; j++) {
                            const float dot = (float)kq_int8_dot(type, blk, q + tt * cols + b * QK, j);
                            total = fmaf(dot, scale[j], total);
                            total = fmaf(-xsum[(b * 8 + (size_t)j) * tokens + tt], offset[j], total);
                        }
                        acc[t + k] = acc[t + k] + total * xs[b * tokens + tt];
                    }
                for (; t < cnt; t++) {
                    const size_t tt = t0 + t;
                    float total = 0.0f;
                    for (int j = 0; j < 8; j++) {
                        const float dot = (float)kq_int8_dot(type, blk, q + tt * cols + b * QK, j);
                        total += scale[j] * dot - offset[j] * xsum[(b * 8 + (size_t)j) * tokens + tt];
                    }
                    acc[t] += total * xs[b * tokens + tt];
                }
            }
            for (size_t t = 0; t < cnt; t++) y[(t0 + t) * rows + r] = acc[t];
        }
    }
    free(q); free(xs); free(xsum); free(acc);
    return 0;
}

int orc_q4k_matmat_int8(const void *w, size_t rows, size_t cols, const float *x, float *y,
                        size_t tokens) {
    if (tokens == 1) return orc_q4k_matvec_int8(w, rows, cols, x, y);
    return kq_matmat_int8(ORC_Q4_K, w, rows, cols, x, y, tokens);
}

/* Q5_K through the same batched lane (kernels.c:2573-2595); its matvec has no
 * int8 form (tokens == 1 is the exact matvec, kernels.c:2576-2577). */
int orc_q5k_matmat_int8(const void *w, size_t rows, size_t cols, const float *x, float *y,
                        size_t tokens) {
    if (tokens == 1) return orc_matvec(ORC_Q5_K, w, rows, cols, x, y);
    return kq_matmat_int8(ORC_Q5_K, w, rows, cols, x, y, tokens);
}
