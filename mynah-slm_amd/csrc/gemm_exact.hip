// gemm_exact.hip — batched Y[tokens][rows] = X[tokens][cols] · W^T in the
// exact batched order of the reference (the prefill GEMM).
//
// The reference's exact batched core (third_party/ingot/src/kernels.c:
// 1053-1104, scalar branch of qk_gemm_block 1017-1026) decodes a super-block
// of each row into 256 f32 values (dequant_block 1030-1039, q6_dequant_block
// 2176-2199, eight q8_0_dequant_block 2635-2639), then for every (row, token)
// sums w[i] * x[i] for i = 0..255 in order from 0 and adds that sum to the
// (row, token) accumulator, super-block after super-block. This kernel keeps
// that order exactly: every decoded value is exact in f32 before its one
// rounding (one fma gives it), each product and each sum is its own rounding
// (no contraction), so every output is bit-identical to the reference.
//
// The same kernel in the matvec order (ORD = 1) is the prefill GEMM of the
// resident decoder: every (row, token) output is then the one the
// reference's matvec (kernels.c:94-115, 319-337; 2525-2551) gives for that
// token — Q4_K interleaves the low- and high-nibble weights of each byte of
// a group, Q8_0 folds its sum into the row every 32 values, Q6_K is the same
// in both orders — so a prompt filled in batches leaves the bits a
// token-by-token fill would. With `res` set the output is res + W x (the
// reference's residual add, src/arch_qwen3.c:224, 234; res may alias y).
//
// Tiling: a workgroup of 256 threads owns 64 rows x 64 tokens; thread
// (tr, tc) = (tid / 16, tid % 16) owns rows tr + 16 k and tokens tc + 16 j,
// k, j < 4: 16 independent chains. Each super-block is processed in two
// halves of 128 values: the workgroup decodes the 64 rows' half into LDS and
// copies the 64 tokens' half of x beside it (rows padded to 132 floats), then
// every thread walks i = 0..127 in order for its 16 chains (LDS reads of 4
// consecutive values). The next half's weights and x are fetched into
// registers while the current half is summed.
//
// SPDX-License-Identifier: MIT
#include "common.hip.h"

#define GM_ROWS 64
#define GM_TOK 64
#define GM_HALF 128
#define GM_LD (GM_HALF + 4)

typedef float gm_f4 __attribute__((ext_vector_type(4)));

// Raw bytes one thread needs to decode its 32 values (sub-block sb) of one
// row's super-block, and the decode into dst[0..31] in natural order.
struct GmQ4K {
    uint4 hdr;      // d, dmin, 12 scale bytes
    uint4 q[2];     // the 32 quant bytes of group sb / 2
    __device__ __forceinline__ void load(const uint8_t *blk, uint32_t sb) {
        hdr = *(const uint4 *)blk;
        const uint4 *p = (const uint4 *)(blk + 16u + 32u * (sb >> 1));
        q[0] = p[0];
        q[1] = p[1];
    }
    __device__ __forceinline__ void decode(uint32_t sb, float *dst) const {
#pragma clang fp contract(off)
        const float d = f16_to_f32(hdr.x), dmin = f16_to_f32(hdr.x >> 16);
        // Scale byte j of the 12 (kernels.c:83-92 scale_min), by selects so
        // nothing is indexed at run time.
        auto sc = [&](uint32_t j) -> uint32_t {
            const uint32_t wd = j < 4u ? hdr.y : (j < 8u ? hdr.z : hdr.w);
            return (wd >> (8u * (j & 3u))) & 0xffu;
        };
        uint32_t scv, mv;
        if (sb < 4) {
            scv = sc(sb) & 63u;
            mv = sc(sb + 4) & 63u;
        } else {
            scv = (sc(sb + 4) & 15u) | ((sc(sb - 4) >> 6) << 4);
            mv = (sc(sb + 4) >> 4) | ((sc(sb) >> 6) << 4);
        }
        const float d1 = d * (float)scv, m1 = dmin * (float)mv;
        const uint32_t w[8] = {q[0].x, q[0].y, q[0].z, q[0].w, q[1].x, q[1].y, q[1].z, q[1].w};
        const uint32_t shift = (sb & 1u) ? 4u : 0u;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t n = (w[k] >> shift) & 0x0f0f0f0fu;
            dst[4 * k] = __builtin_fmaf(d1, ubyte_f<0>(n), -m1);
            dst[4 * k + 1] = __builtin_fmaf(d1, ubyte_f<1>(n), -m1);
            dst[4 * k + 2] = __builtin_fmaf(d1, ubyte_f<2>(n), -m1);
            dst[4 * k + 3] = __builtin_fmaf(d1, ubyte_f<3>(n), -m1);
        }
    }
};

// 8 dwords starting at a 2-byte aligned address.
MYNAH_DEV void load8_u16al(const uint8_t *p, uint32_t *out) {
    const uint32_t s = (uint32_t)(uintptr_t)p & 3u;
    const uint32_t *a = (const uint32_t *)(p - s);
    uint32_t r[9];
#pragma unroll
    for (int k = 0; k < 9; k++) r[k] = a[k];
#pragma unroll
    for (int k = 0; k < 8; k++) out[k] = align_bytes(r[k + 1], r[k], s);
}

struct GmQ6K {
    uint32_t ql[8], qh[8], sd;   // sd: the two int8 scales (low 16 bits), d (high 16)
    __device__ __forceinline__ void load(const uint8_t *blk, uint32_t sb) {
        const uint32_t h = sb >> 2, k = sb & 3u;
        load8_u16al(blk + 64u * h + 32u * (k & 1u), ql);
        load8_u16al(blk + 128u + 32u * h, qh);
        const uint16_t sc2 = *(const uint16_t *)(blk + 192u + 2u * sb);
        const uint16_t dd = *(const uint16_t *)(blk + 208u);
        sd = (uint32_t)sc2 | ((uint32_t)dd << 16);
    }
    __device__ __forceinline__ void decode(uint32_t sb, float *dst) const {
#pragma clang fp contract(off)
        const uint32_t k = sb & 3u;
        const float d = f16_to_f32(sd >> 16);
        const float ds0 = d * (float)(int)(int8_t)(sd & 0xffu);
        const float ds1 = d * (float)(int)(int8_t)((sd >> 8) & 0xffu);
        const float n0 = -32.0f * ds0, n1 = -32.0f * ds1;
        const uint32_t ns = (k < 2) ? 0u : 4u, hs = 2u * k;
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const uint32_t q6 = ((ql[m] >> ns) & 0x0f0f0f0fu) | (((qh[m] >> hs) & 0x03030303u) << 4);
            const float a = m < 4 ? ds0 : ds1, b = m < 4 ? n0 : n1;
            dst[4 * m] = __builtin_fmaf(a, ubyte_f<0>(q6), b);
            dst[4 * m + 1] = __builtin_fmaf(a, ubyte_f<1>(q6), b);
            dst[4 * m + 2] = __builtin_fmaf(a, ubyte_f<2>(q6), b);
            dst[4 * m + 3] = __builtin_fmaf(a, ubyte_f<3>(q6), b);
        }
    }
};

struct GmQ80 {
    uint32_t q[8], d;
    __device__ __forceinline__ void load(const uint8_t *blk8, uint32_t sb) {
        const uint8_t *blk = blk8 + 34u * sb;
        d = *(const uint16_t *)blk;
        load8_u16al(blk + 2, q);
    }
    __device__ __forceinline__ void decode(uint32_t, float *dst) const {
#pragma clang fp contract(off)
        const float dd = f16_to_f32(d), n128 = -128.0f * dd;
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const uint32_t v = q[m] ^ 0x80808080u;
            dst[4 * m] = __builtin_fmaf(dd, ubyte_f<0>(v), n128);
            dst[4 * m + 1] = __builtin_fmaf(dd, ubyte_f<1>(v), n128);
            dst[4 * m + 2] = __builtin_fmaf(dd, ubyte_f<2>(v), n128);
            dst[4 * m + 3] = __builtin_fmaf(dd, ubyte_f<3>(v), n128);
        }
    }
};

// The x half (64 tokens x 128 values) of unit u, half h: 8 float4 per thread,
// token idx / 32 and float4 idx % 32 for idx = tid + 256 k.
MYNAH_DEV void gm_fetch_x(gm_f4 (&xr)[8], const float *__restrict__ x, uint32_t tid, uint32_t tok0,
                          uint32_t tokens, uint32_t cols, uint32_t u, uint32_t h) {
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t idx = tid + 256u * (uint32_t)k, xt = idx >> 5, xq = idx & 31u;
        const uint32_t t = tok0 + xt < tokens ? tok0 + xt : tokens - 1u;
        xr[k] = *(const gm_f4 *)(x + (size_t)t * cols + 256u * u + GM_HALF * h + 4u * xq);
    }
}

// ORD: 0 the batched order, 1 the matvec order; FMT the block type.
template <class Raw, uint32_t UB, int ORD = 0, int FMT = 0>
MYNAH_DEV void gemm_exact(const uint8_t *__restrict__ w, const float *__restrict__ x,
                          float *__restrict__ y, uint32_t rows, uint32_t cols, uint32_t tokens,
                          uint32_t row_bytes, const float *res = nullptr) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) float wl[GM_ROWS][GM_LD];
    __shared__ __attribute__((aligned(16))) float xl[GM_TOK][GM_LD];
    const uint32_t tid = threadIdx.x, tr = tid >> 4, tc = tid & 15u;
    const uint32_t row0 = blockIdx.x * GM_ROWS, tok0 = blockIdx.y * GM_TOK;
    const uint32_t units = cols / 256u;
    // Decode role: row dr of the tile, 32-value piece dp of the half.
    const uint32_t dr = tid >> 2, dp = tid & 3u;
    const uint32_t drow = row0 + dr < rows ? row0 + dr : rows - 1u;
    const uint8_t *wrow = w + (size_t)drow * row_bytes;
    // x role: 8 float4 per thread per half, token xt = idx / 32, float4 xq.
    gm_f4 xr[8];
    Raw raw;

    float acc[4][4], s[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[a][b] = 0.0f;
    raw.load(wrow, dp);
    gm_fetch_x(xr, x, tid, tok0, tokens, cols, 0u, 0u);
    for (uint32_t u = 0; u < units; u++) {
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) s[a][b] = 0.0f;
#pragma unroll
        for (uint32_t h = 0; h < 2; h++) {
            float vals[32];
            raw.decode(4u * h + dp, vals);
#pragma unroll
            for (int k = 0; k < 8; k++)
                *(float4 *)&wl[dr][32u * dp + 4 * k] =
                    make_float4(vals[4 * k], vals[4 * k + 1], vals[4 * k + 2], vals[4 * k + 3]);
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const uint32_t idx = tid + 256u * (uint32_t)k;
                *(gm_f4 *)&xl[idx >> 5][4u * (idx & 31u)] = xr[k];
            }
            __syncthreads();
            const uint32_t nu = h == 0 ? u : u + 1u, nh = h ^ 1u;
            if (nu < units) {
                raw.load(wrow + UB * nu, 4u * nh + dp);
                gm_fetch_x(xr, x, tid, tok0, tokens, cols, nu, nh);
            }
            if (ORD == 1 && FMT == 12) {
                // Q4_K matvec order: per group of 64, value j then 32 + j.
                for (uint32_t g = 0; g < GM_HALF; g += 64)
                    for (uint32_t j = 0; j < 32; j += 4) {
                        float4 wl4[4], wh4[4], xl4[4], xh4[4];
#pragma unroll
                        for (int a = 0; a < 4; a++) {
                            wl4[a] = *(const float4 *)&wl[tr + 16u * a][g + j];
                            wh4[a] = *(const float4 *)&wl[tr + 16u * a][g + 32u + j];
                        }
#pragma unroll
                        for (int b = 0; b < 4; b++) {
                            xl4[b] = *(const float4 *)&xl[tc + 16u * b][g + j];
                            xh4[b] = *(const float4 *)&xl[tc + 16u * b][g + 32u + j];
                        }
#pragma unroll
                        for (int a = 0; a < 4; a++)
#pragma unroll
                            for (int b = 0; b < 4; b++) {
                                s[a][b] = s[a][b] + wl4[a].x * xl4[b].x;
                                s[a][b] = s[a][b] + wh4[a].x * xh4[b].x;
                                s[a][b] = s[a][b] + wl4[a].y * xl4[b].y;
                                s[a][b] = s[a][b] + wh4[a].y * xh4[b].y;
                                s[a][b] = s[a][b] + wl4[a].z * xl4[b].z;
                                s[a][b] = s[a][b] + wh4[a].z * xh4[b].z;
                                s[a][b] = s[a][b] + wl4[a].w * xl4[b].w;
                                s[a][b] = s[a][b] + wh4[a].w * xh4[b].w;
                            }
                    }
            } else {
                for (uint32_t i = 0; i < GM_HALF; i += 4) {
                    float4 wv[4], xv[4];
#pragma unroll
                    for (int a = 0; a < 4; a++) wv[a] = *(const float4 *)&wl[tr + 16u * a][i];
#pragma unroll
                    for (int b = 0; b < 4; b++) xv[b] = *(const float4 *)&xl[tc + 16u * b][i];
#pragma unroll
                    for (int a = 0; a < 4; a++)
#pragma unroll
                        for (int b = 0; b < 4; b++) {
                            s[a][b] = s[a][b] + wv[a].x * xv[b].x;
                            s[a][b] = s[a][b] + wv[a].y * xv[b].y;
                            s[a][b] = s[a][b] + wv[a].z * xv[b].z;
                            s[a][b] = s[a][b] + wv[a].w * xv[b].w;
                        }
                    if (ORD == 1 && FMT == 8 && (i & 31u) == 28u) {
                        // Q8_0 matvec order: each 32-value block's sum joins
                        // the row total on its own.
#pragma unroll
                        for (int a = 0; a < 4; a++)
#pragma unroll
                            for (int b = 0; b < 4; b++) {
                                acc[a][b] = acc[a][b] + s[a][b];
                                s[a][b] = 0.0f;
                            }
                    }
                }
            }
            __syncthreads();
        }
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int b = 0; b < 4; b++) acc[a][b] = acc[a][b] + s[a][b];
    }
#pragma unroll
    for (int a = 0; a < 4; a++) {
        const uint32_t r = row0 + tr + 16u * a;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const uint32_t t = tok0 + tc + 16u * b;
            if (r < rows && t < tokens) {
                const size_t o = (size_t)t * rows + r;
                y[o] = res ? res[o] + acc[a][b] : acc[a][b];
            }
        }
    }
}

// Grid (ceil(rows / 64), ceil(tokens / 64)), block 256; cols % 256 == 0;
// x 16-byte aligned. Q4_K rows 16-byte aligned, Q6_K / Q8_0 2-byte aligned.
#define GEMM_EXACT_ENTRY(name, RAW, UB)                                                        \
    extern "C" __global__ void __launch_bounds__(256)                                          \
        name(const uint8_t *__restrict__ w, const float *__restrict__ x, float *__restrict__ y, \
             uint32_t rows, uint32_t cols, uint32_t tokens, uint32_t row_bytes) {              \
        gemm_exact<RAW, UB>(w, x, y, rows, cols, tokens, row_bytes);                           \
    }

GEMM_EXACT_ENTRY(mynah_q4k_gemm_exact, GmQ4K, 144u)
GEMM_EXACT_ENTRY(mynah_q6k_gemm_exact, GmQ6K, 210u)
GEMM_EXACT_ENTRY(mynah_q80_gemm_exact, GmQ80, 272u)

// The matvec order, with the residual epilogue (res may be NULL or alias y).
#define GEMM_MV_ENTRY(name, RAW, UB, FMT)                                                      \
    extern "C" __global__ void __launch_bounds__(256)                                          \
        name(const uint8_t *__restrict__ w, const float *__restrict__ x, float *y,             \
             uint32_t rows, uint32_t cols, uint32_t tokens, uint32_t row_bytes,                \
             const float *res) {                                                               \
        gemm_exact<RAW, UB, 1, FMT>(w, x, y, rows, cols, tokens, row_bytes, res);              \
    }

GEMM_MV_ENTRY(mynah_q4k_gemm_mv, GmQ4K, 144u, 12)
GEMM_MV_ENTRY(mynah_q6k_gemm_mv, GmQ6K, 210u, 14)
GEMM_MV_ENTRY(mynah_q80_gemm_mv, GmQ80, 272u, 8)
