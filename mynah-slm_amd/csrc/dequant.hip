// dequant.hip — matrix dequantisation bit-identical to the reference.
//
// SPDX-License-Identifier: MIT
#include "common.hip.h"

// ── bit-exact dequantisation ────────────────────────────────────────────────
// Same operation order as the reference decoders, so every value is the
// identical f32 (kernels.c:117-136 Q4_K, 1812-1833 Q5_K, 2176-2199 Q6_K,
// 2518-2523 Q8_0, 2353-2360 Q4_0). One thread per 32 output values; `units`
// = rows * cols / 32.

extern "C" __global__ void __launch_bounds__(256)
mynah_dequant(const uint8_t *__restrict__ w, float *__restrict__ y, uint32_t type,
              uint32_t rows, uint32_t cols) {
    const size_t unit = (size_t)blockIdx.x * 256u + threadIdx.x;
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
    } else if (type == 13u) {
        const uint8_t *blk = w + row * (cols / 256u) * 176u + (c / 8u) * 176u;
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
        const uint8_t *qh = blk + 16, *qs = blk + 48 + 32u * g;
        for (int i = 0; i < 32; i++) {
            const uint32_t q = ((j & 1u) ? (qs[i] >> 4) : (qs[i] & 15u)) + (((qh[i] >> j) & 1u) << 4);
            out[i] = dd * (float)q - mm;
        }
    } else if (type == 2u) {
        const uint8_t *blk = w + row * (cols / 32u) * 18u + c * 18u;
        const float d = f16_to_f32(blk[0] | (blk[1] << 8));
        for (int i = 0; i < 16; i++) {
            out[i] = d * (float)((int)(blk[2 + i] & 15u) - 8);
            out[16 + i] = d * (float)((int)(blk[2 + i] >> 4) - 8);
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
