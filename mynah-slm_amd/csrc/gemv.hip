// gemv.hip — decode GEMV y = W·x straight off unchanged GGUF blocks (gfx950).
//
// Replaces the reference's per-type matvec kernels:
//   Q4_K  third_party/ingot/src/kernels.c:94-115, 319-337, 812-844
//   Q6_K  third_party/ingot/src/kernels.c:2096-2124, 2176-2199, 2305-2318
//   Q8_0  third_party/ingot/src/kernels.c:2518-2551
// Same value of every weight (the decoded value is exact in f32, see the
// formats), f32 accumulation in a different order; outputs agree with the
// reference to |gpu - ref| / max(1, |ref|) <= 1e-4.
//
// Work decomposition (all three formats):
//   * workgroup = 4 waves of 64 lanes; each wave owns 8*R consecutive rows;
//   * lane = (row group rg = lane/8, unit u = lane%8); a lane handles the
//     rows rg, rg+8, ..., rg+8(R-1) of its wave and, per 256-weight super-
//     block, the 32 weights of "unit u" in each of them;
//   * all lanes walk the super-blocks of their rows in step, so each loop
//     iteration reads R * 8 row segments of one block each, with 16-byte
//     (Q4_K) or dword (Q6_K/Q8_0, 2-byte-aligned blocks) loads;
//   * x is staged once per workgroup in LDS in a padded layout chosen so the
//     8 units' 16-byte reads fall in distinct banks while the 8 row groups
//     read identical addresses (broadcast); the x values a lane reads are
//     reused for its R rows from registers;
//   * the zero-point terms are folded: sum_t (q_t - z) x_t = sum_t q_t x_t -
//     z * sum_t x_t, with the run sums of x precomputed next to x in LDS, so
//     each weight costs one byte->float conversion and one FMA;
//   * the 8 unit partials of a row are combined with an xor butterfly.
//
// SPDX-License-Identifier: MIT
#include "common.hip.h"

#define WG 256

// Stage x into LDS: x[i] at lx[i + 4 * (i >> PAD)], and the sums of each
// run of RUN consecutive values at ls[i / RUN]. cols is a multiple of RUN
// and of 4; every 4-thread group is wholly inside or outside [0, cols).
template <int PAD, int RUN>
MYNAH_DEV void stage_x(const float *__restrict__ x, uint32_t cols, float *lx, float *ls) {
    static_assert(RUN == 8 || RUN == 16 || RUN == 32, "run");
    for (uint32_t i = 4 * threadIdx.x; i < cols; i += 4 * WG) {
        const float4 v = *(const float4 *)(x + i);
        *(float4 *)(lx + i + 4 * (i >> PAD)) = v;
        float s = (v.x + v.y) + (v.z + v.w);
        s += __shfl_xor(s, 1, 64);
        if (RUN >= 16) s += __shfl_xor(s, 2, 64);
        if (RUN >= 32) s += __shfl_xor(s, 4, 64);
        if ((threadIdx.x & (RUN / 4 - 1)) == 0) ls[i / RUN] = s;
    }
}

// ── Q4_K ────────────────────────────────────────────────────────────────────
// Block (144 B, 16-byte aligned): d f16 @0, dmin f16 @2, scales[12] @4,
// qs[128] @16. Unit u = 2g + hh covers qs[32g + 16hh .. +15]: low nibbles are
// weights 64g + 16hh + t (sub-block 2g), high nibbles 64g + 32 + 16hh + t
// (sub-block 2g + 1). 6-bit (scale, min) of sub-block j:
//   j < 4: sc = s[j] & 63, m = s[j+4] & 63
//   j >= 4: sc = (s[j+4] & 15) | (s[j-4] >> 6) << 4,
//           m = (s[j+4] >> 4) | (s[j] >> 6) << 4.
// x layout: pad 4 floats per 64 (block of 256 -> 272), run sums of 16.

MYNAH_DEV void q4k_scale(uint32_t s0, uint32_t s1, uint32_t s2, bool high, float &sc, float &m) {
    // s0, s1, s2: scale dwords (bytes 0-3, 4-7, 8-11) shifted so that byte
    // j & 3 is in bits 0..7.
    const uint32_t a = high ? ((s2 & 15u) | ((s0 >> 2) & 48u)) : (s0 & 63u);
    const uint32_t b = high ? (((s2 >> 4) & 15u) | ((s1 >> 2) & 48u)) : (s1 & 63u);
    sc = (float)a;
    m = (float)b;
}

template <int R>
MYNAH_DEV void q4k_gemv(const uint8_t *__restrict__ w, const float *__restrict__ x,
                        float *__restrict__ y, uint32_t rows, uint32_t nb) {
    extern __shared__ float lds[];
    const uint32_t cols = nb * 256u;
    float *lx = lds;
    float *ls = lds + cols + cols / 16;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t rg = lane >> 3, u = lane & 7u, g = u >> 1, hh = u & 1u;
    const uint32_t row0 = (blockIdx.x * 4u + wave) * (8u * R) + rg;
    const size_t rb = (size_t)nb * 144u;

    const uint8_t *wr[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t row = row0 + 8u * r;
        wr[r] = w + (size_t)(row < rows ? row : rows - 1u) * rb;
    }
    stage_x<6, 16>(x, cols, lx, ls);
    __syncthreads();

    const bool high = g >= 2;                 // sub-blocks 2g, 2g+1 >= 4
    const uint32_t sh = 16u * (g & 1u);       // byte (2g) & 3 -> bit offset
    const uint32_t offA = 68u * g + 16u * hh, offB = offA + 32u;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;

#pragma unroll 2
    for (uint32_t b = 0; b < nb; b++) {
        const float *xb = lx + 272u * b;
        float xa[16], xc[16];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float4 va = *(const float4 *)(xb + offA + 4 * k);
            const float4 vc = *(const float4 *)(xb + offB + 4 * k);
            xa[4 * k] = va.x; xa[4 * k + 1] = va.y; xa[4 * k + 2] = va.z; xa[4 * k + 3] = va.w;
            xc[4 * k] = vc.x; xc[4 * k + 1] = vc.y; xc[4 * k + 2] = vc.z; xc[4 * k + 3] = vc.w;
        }
        const float sumA = ls[16u * b + 4u * g + hh], sumC = ls[16u * b + 4u * g + 2u + hh];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t *blk = wr[r] + 144u * b;
            const uint4 hdr = *(const uint4 *)blk;
            const uint4 q = *(const uint4 *)(blk + 16u + 16u * u);
            const float d = f16_to_f32(hdr.x), dmin = f16_to_f32(hdr.x >> 16);
            float scA, mA, scC, mC;
            q4k_scale(hdr.y >> sh, hdr.z >> sh, hdr.w >> sh, high, scA, mA);
            q4k_scale(hdr.y >> (sh + 8u), hdr.z >> (sh + 8u), hdr.w >> (sh + 8u), high, scC, mC);
            const uint32_t qv[4] = {q.x, q.y, q.z, q.w};
            float dotA = 0.0f, dotC = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t lo = qv[k] & 0x0f0f0f0fu, hi = (qv[k] >> 4) & 0x0f0f0f0fu;
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    dotA = fmaf(byte_f(lo, t), xa[4 * k + t], dotA);
                    dotC = fmaf(byte_f(hi, t), xc[4 * k + t], dotC);
                }
            }
            const float part = (d * scA) * dotA + (d * scC) * dotC;
            acc[r] += part - dmin * (mA * sumA + mC * sumC);
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float v = group8_sum(acc[r]);
        const uint32_t row = row0 + 8u * r;
        if (u == 0 && row < rows) y[row] = v;
    }
}

// ── Q6_K ────────────────────────────────────────────────────────────────────
// Block (210 B, 2-byte aligned): ql[128] @0, qh[64] @128, int8 sc[16] @192,
// d f16 @208. Unit u = 4h + p covers, for each quarter k = 0..3 of half h,
// the 8 weights 128h + 32k + 8p + t: low 4 bits from ql[64h + 32(k&1) + 8p + t]
// (low nibble for k < 2, high for k >= 2), top 2 bits (qh[32h + 8p + t] >> 2k)
// & 3, scale sc[8h + 2k + p/2], value d * sc * (q - 32).
// Fields sit at even offsets, so each 8-byte field is read as the aligned
// dwords that contain it and realigned with v_alignbyte (no unaligned loads,
// and no dword that holds no byte of the block is touched).
// x layout: pad 4 floats per 128 (block of 256 -> 264), run sums of 8.

MYNAH_DEV void load8_2a(const uint8_t *p, uint32_t &lo, uint32_t &hi) {
    const uint32_t s = (uint32_t)(uintptr_t)p & 3u;
    const uint32_t *a = (const uint32_t *)(p - s);
    const uint32_t d0 = a[0], d1 = a[1], d2 = a[2];
    lo = align_bytes(d1, d0, s);
    hi = align_bytes(d2, d1, s);
}

template <int R>
MYNAH_DEV void q6k_gemv(const uint8_t *__restrict__ w, const float *__restrict__ x,
                        float *__restrict__ y, uint32_t rows, uint32_t nb) {
    extern __shared__ float lds[];
    const uint32_t cols = nb * 256u;
    float *lx = lds;
    float *ls = lds + cols + cols / 32;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t rg = lane >> 3, u = lane & 7u, h = u >> 2, p = u & 3u;
    const uint32_t row0 = (blockIdx.x * 4u + wave) * (8u * R) + rg;
    const size_t rb = (size_t)nb * 210u;

    const uint8_t *wr[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t row = row0 + 8u * r;
        wr[r] = w + (size_t)(row < rows ? row : rows - 1u) * rb;
    }
    stage_x<7, 8>(x, cols, lx, ls);
    __syncthreads();

    const uint32_t sc_shift = 8u * (p >> 1);
    const uint32_t xoff = 132u * h + 8u * p;          // padded 128h + 8p
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;

#pragma unroll 2
    for (uint32_t b = 0; b < nb; b++) {
        const float *xb = lx + 264u * b + xoff;
        float xv[4][8];
        float xs[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float4 v0 = *(const float4 *)(xb + 32 * k);
            const float4 v1 = *(const float4 *)(xb + 32 * k + 4);
            xv[k][0] = v0.x; xv[k][1] = v0.y; xv[k][2] = v0.z; xv[k][3] = v0.w;
            xv[k][4] = v1.x; xv[k][5] = v1.y; xv[k][6] = v1.z; xv[k][7] = v1.w;
            xs[k] = ls[32u * b + 16u * h + 4u * k + p];
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t *blk = wr[r] + 210u * b;
            uint32_t a0, a1, c0, c1, h0, h1, s0, s1;
            load8_2a(blk + 64u * h + 8u * p, a0, a1);
            load8_2a(blk + 64u * h + 32u + 8u * p, c0, c1);
            load8_2a(blk + 128u + 32u * h + 8u * p, h0, h1);
            load8_2a(blk + 192u + 8u * h, s0, s1);
            const uint32_t ds = (uint32_t)(uintptr_t)(blk + 208) & 3u;
            const uint32_t dword = *(const uint32_t *)(blk + 208 - ds);
            const float d = f16_to_f32(dword >> (8u * ds));
            const float sc[4] = {
                (float)(int)(int8_t)(s0 >> sc_shift), (float)(int)(int8_t)(s0 >> (sc_shift + 16u)),
                (float)(int)(int8_t)(s1 >> sc_shift), (float)(int)(int8_t)(s1 >> (sc_shift + 16u))};
            const uint32_t av[2] = {a0, a1}, cv[2] = {c0, c1}, hv[2] = {h0, h1};
            float dot[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const uint32_t qk[4] = {
                    (av[i] & 0x0f0f0f0fu) | ((hv[i] << 4) & 0x30303030u),
                    (cv[i] & 0x0f0f0f0fu) | ((hv[i] << 2) & 0x30303030u),
                    ((av[i] >> 4) & 0x0f0f0f0fu) | (hv[i] & 0x30303030u),
                    ((cv[i] >> 4) & 0x0f0f0f0fu) | ((hv[i] >> 2) & 0x30303030u)};
#pragma unroll
                for (int k = 0; k < 4; k++)
#pragma unroll
                    for (int t = 0; t < 4; t++)
                        dot[k] = fmaf(byte_f(qk[k], t), xv[k][4 * i + t], dot[k]);
            }
            float part = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; k++) part = fmaf(sc[k], fmaf(-32.0f, xs[k], dot[k]), part);
            acc[r] = fmaf(d, part, acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float v = group8_sum(acc[r]);
        const uint32_t row = row0 + 8u * r;
        if (u == 0 && row < rows) y[row] = v;
    }
}

// ── Q8_0 ────────────────────────────────────────────────────────────────────
// Block (34 B, 2-byte aligned): d f16 @0, int8 qs[32] @2; value qs * d.
// Unit u handles block 8i + u of its row at step i (32 weights). The block is
// read as the nine aligned dwords that contain it. (q + 128) is the unsigned
// byte q ^ 0x80, so sum q x = sum (q ^ 0x80) x - 128 sum x.
// x layout: pad 4 floats per 32 (block of 32 -> 36), run sums of 32.

template <int R>
MYNAH_DEV void q80_gemv(const uint8_t *__restrict__ w, const float *__restrict__ x,
                        float *__restrict__ y, uint32_t rows, uint32_t nblk) {
    extern __shared__ float lds[];
    const uint32_t cols = nblk * 32u;
    float *lx = lds;
    float *ls = lds + cols + cols / 8;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t rg = lane >> 3, u = lane & 7u;
    const uint32_t row0 = (blockIdx.x * 4u + wave) * (8u * R) + rg;
    const size_t rb = (size_t)nblk * 34u;

    const uint8_t *wr[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint32_t row = row0 + 8u * r;
        wr[r] = w + (size_t)(row < rows ? row : rows - 1u) * rb;
    }
    stage_x<5, 32>(x, cols, lx, ls);
    __syncthreads();

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;

    for (uint32_t j = u; j < nblk; j += 8u) {
        const float *xb = lx + 36u * j;
        float xv[32];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float4 v = *(const float4 *)(xb + 4 * k);
            xv[4 * k] = v.x; xv[4 * k + 1] = v.y; xv[4 * k + 2] = v.z; xv[4 * k + 3] = v.w;
        }
        const float xsum = ls[j];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint8_t *blk = wr[r] + 34u * j;
            const uint32_t s = (uint32_t)(uintptr_t)blk & 3u;
            const uint32_t *a = (const uint32_t *)(blk - s);
            uint32_t raw[9];
#pragma unroll
            for (int k = 0; k < 9; k++) raw[k] = a[k];
            const float d = f16_to_f32(s ? (raw[0] >> 16) : raw[0]);
            float dot = 0.0f;
#pragma unroll
            for (int m = 0; m < 8; m++) {
                const uint32_t qm = (s ? raw[m + 1] : align_bytes(raw[m + 1], raw[m], 2u)) ^ 0x80808080u;
#pragma unroll
                for (int t = 0; t < 4; t++) dot = fmaf(byte_f(qm, t), xv[4 * m + t], dot);
            }
            acc[r] = fmaf(d, fmaf(-128.0f, xsum, dot), acc[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float v = group8_sum(acc[r]);
        const uint32_t row = row0 + 8u * r;
        if (u == 0 && row < rows) y[row] = v;
    }
}

#define GEMV_ENTRY(fmt, R)                                                                   \
    extern "C" __global__ void __launch_bounds__(WG)                                         \
        mynah_##fmt##_gemv_r##R(const uint8_t *__restrict__ w, const float *__restrict__ x, \
                                float *__restrict__ y, uint32_t rows, uint32_t nb) {       \
        fmt##_gemv<R>(w, x, y, rows, nb);                                                    \
    }

GEMV_ENTRY(q4k, 1)
GEMV_ENTRY(q4k, 2)
GEMV_ENTRY(q4k, 4)
GEMV_ENTRY(q6k, 1)
GEMV_ENTRY(q6k, 2)
GEMV_ENTRY(q6k, 4)
GEMV_ENTRY(q80, 1)
GEMV_ENTRY(q80, 2)
GEMV_ENTRY(q80, 4)

// ── bit-exact dequantisation ────────────────────────────────────────────────
// Same operation order as the reference decoders, so every value is the
// identical f32 (kernels.c:117-136 Q4_K, 2176-2199 Q6_K, 2518-2523 Q8_0).
// One thread per 32 output values; `units` = rows * cols / 32.

extern "C" __global__ void __launch_bounds__(WG)
mynah_dequant(const uint8_t *__restrict__ w, float *__restrict__ y, uint32_t type,
              uint32_t rows, uint32_t cols) {
    const size_t unit = (size_t)blockIdx.x * WG + threadIdx.x;
    const size_t per_row = cols / 32u;
    if (unit >= (size_t)rows * per_row) return;
    const size_t row = unit / per_row, c = unit % per_row;   // 32-value group in row
    float out[32];
    if (type == 12u) {
        const uint8_t *blk = w + row * (cols / 256u) * 144u + (c / 8u) * 144u;
        const uint32_t j = (uint32_t)(c % 8u), g = j >> 1;
        const float d = f16_to_f32(blk[0] | (blk[1] << 8));
        const float dmin = f16_to_f32(blk[2] | (blk[3] << 8));
        const uint8_t *s = blk + 4;
        uint32_t sc, m;
        if (j < 4) { sc = s[j] & 63u; m = s[j + 4] & 63u; }
        else {
            sc = (s[j + 4] & 15u) | ((s[j - 4] >> 6) << 4);
            m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
        }
        const float dd = d * (float)sc, mm = dmin * (float)m;
        const uint8_t *qs = blk + 16 + 32u * g;
        for (int i = 0; i < 32; i++) {
            const uint32_t q = (j & 1u) ? (qs[i] >> 4) : (qs[i] & 15u);
            out[i] = dd * (float)q - mm;
        }
    } else if (type == 14u) {
        const uint8_t *blk = w + row * (cols / 256u) * 210u + (c / 8u) * 210u;
        const uint32_t qq = (uint32_t)(c % 8u), h = qq >> 2, k = qq & 3u;
        const float d = f16_to_f32(blk[208] | (blk[209] << 8));
        const int8_t *sc = (const int8_t *)(blk + 192);
        const uint8_t *ql = blk + 64u * h + 32u * (k & 1u), *qh = blk + 128u + 32u * h;
        for (int i = 0; i < 32; i++) {
            const uint32_t lo = (k < 2) ? (ql[i] & 15u) : (ql[i] >> 4);
            const int q = (int)(lo | (((qh[i] >> (2u * k)) & 3u) << 4)) - 32;
            out[i] = d * (float)sc[8u * h + 2u * k + (uint32_t)i / 16u] * (float)q;
        }
    } else {
        const uint8_t *blk = w + row * (cols / 32u) * 34u + c * 34u;
        const float d = f16_to_f32(blk[0] | (blk[1] << 8));
        for (int i = 0; i < 32; i++) out[i] = (float)(int8_t)blk[2 + i] * d;
    }
    float *dst = y + row * cols + c * 32u;
    for (int i = 0; i < 32; i++) dst[i] = out[i];
}
