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
// token — Q4_K (and Q5_K) interleaves the low- and high-nibble weights of each byte of
// a group (the decoded weights and x are stored in LDS in that order, so
// the inner loop stays a sequential walk), Q8_0 folds its sum into the row
// every 32 values, Q6_K is the same in both orders — so a prompt filled in
// batches leaves the bits a token-by-token fill would. With `res` set the output is res + W x (the
// reference's residual add, src/arch_qwen3.c:224, 234; res may alias y).
//
// Tiling: a workgroup of 256 threads owns 64 rows x 64 tokens; thread
// (tr, tc) = (tid / 16, tid % 16) owns rows tr + 16 k and tokens tc + 16 j,
// k, j < 4: 16 independent chains. Each super-block is processed in four
// stages of 64 values: the workgroup decodes the 64 rows' stage into LDS (16
// values per thread) and copies the 64 tokens' stage of x beside it (rows
// padded to 68 floats), then every thread walks i = 0..63 in order for its
// 16 chains (LDS reads of 4 consecutive values). The next stage's weights
// and x are fetched into registers while the current one is summed. 35 KB
// of LDS per workgroup: four workgroups (16 waves) per CU.
//
// SPDX-License-Identifier: MIT
#include "common.hip.h"

#define GM_ROWS 64
#define GM_TOK 64
#define GM_STAGE 64
#define GM_LD (GM_STAGE + 4)

typedef float gm_f4 __attribute__((ext_vector_type(4)));

// Each holder keeps the raw bytes one thread needs for piece p (0..15) of a
// super-block — its 16 values in LDS order — and decodes them into dst.

// n dwords starting at a 2-byte aligned address.
template <int N>
MYNAH_DEV void loadn_u16al(const uint8_t *p, uint32_t *out) {
    const uint32_t s = (uint32_t)(uintptr_t)p & 3u;
    const uint32_t *a = (const uint32_t *)(p - s);
    uint32_t r[N + 1];
#pragma unroll
    for (int k = 0; k <= N; k++) r[k] = a[k];
#pragma unroll
    for (int k = 0; k < N; k++) out[k] = align_bytes(r[k + 1], r[k], s);
}

// (scale, min) of Q4_K sub-block sb (kernels.c:83-92 scale_min).
MYNAH_DEV void gm_q4k_sm(uint4 hdr, uint32_t sb, float d, float dmin, float &ds, float &dm) {
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
    ds = d * (float)scv;
    dm = dmin * (float)mv;
}

// Q4_K, natural order: piece p = values 16 p .. 16 p + 15, i.e. quant bytes
// 16 (p & 1) .. + 15 of group p / 4, nibble (p / 2) & 1 (sub-block p / 2).
template <bool ASM = true> struct GmQ4KT {
    uint4 hdr, q;
    __device__ __forceinline__ void load(const uint8_t *blk, uint32_t p) {
        hdr = *(const uint4 *)blk;
        q = *(const uint4 *)(blk + 16u + 32u * (p >> 2) + 16u * (p & 1u));
    }
    __device__ __forceinline__ void decode(uint32_t p, float *dst) const {
#pragma clang fp contract(off)
        float d1, m1;
        gm_q4k_sm(hdr, p >> 1, f16_to_f32(hdr.x), f16_to_f32(hdr.x >> 16), d1, m1);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
        const uint32_t shift = ((p >> 1) & 1u) ? 4u : 0u;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t n = (w[k] >> shift) & 0x0f0f0f0fu;
            dst[4 * k] = __builtin_fmaf(d1, ubyte_sel<ASM, 0>(n), -m1);
            dst[4 * k + 1] = __builtin_fmaf(d1, ubyte_sel<ASM, 1>(n), -m1);
            dst[4 * k + 2] = __builtin_fmaf(d1, ubyte_sel<ASM, 2>(n), -m1);
            dst[4 * k + 3] = __builtin_fmaf(d1, ubyte_sel<ASM, 3>(n), -m1);
        }
    }
};
using GmQ4K = GmQ4KT<true>;

// Q4_K in the matvec order: the LDS order of group g is lo_0, hi_0, lo_1,
// hi_1, ... (the low-nibble weight j and the high-nibble weight 32 + j of
// the group, which the matvec sums one after the other). Piece p covers
// quant bytes 8 (p & 3) .. + 7 of group p / 4, both nibbles.
template <bool ASM = true> struct GmQ4KMvT {
    uint4 hdr;
    uint2 q;
    __device__ __forceinline__ void load(const uint8_t *blk, uint32_t p) {
        hdr = *(const uint4 *)blk;
        q = *(const uint2 *)(blk + 16u + 32u * (p >> 2) + 8u * (p & 3u));
    }
    __device__ __forceinline__ void decode(uint32_t p, float *dst) const {
#pragma clang fp contract(off)
        const uint32_t g = p >> 2;
        const float d = f16_to_f32(hdr.x), dmin = f16_to_f32(hdr.x >> 16);
        float dl, ml, dh, mh;
        gm_q4k_sm(hdr, 2u * g, d, dmin, dl, ml);
        gm_q4k_sm(hdr, 2u * g + 1u, d, dmin, dh, mh);
        const uint32_t w[2] = {q.x, q.y};
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const uint32_t lo = w[k] & 0x0f0f0f0fu, hi = (w[k] >> 4) & 0x0f0f0f0fu;
            dst[8 * k + 0] = __builtin_fmaf(dl, ubyte_sel<ASM, 0>(lo), -ml);
            dst[8 * k + 1] = __builtin_fmaf(dh, ubyte_sel<ASM, 0>(hi), -mh);
            dst[8 * k + 2] = __builtin_fmaf(dl, ubyte_sel<ASM, 1>(lo), -ml);
            dst[8 * k + 3] = __builtin_fmaf(dh, ubyte_sel<ASM, 1>(hi), -mh);
            dst[8 * k + 4] = __builtin_fmaf(dl, ubyte_sel<ASM, 2>(lo), -ml);
            dst[8 * k + 5] = __builtin_fmaf(dh, ubyte_sel<ASM, 2>(hi), -mh);
            dst[8 * k + 6] = __builtin_fmaf(dl, ubyte_sel<ASM, 3>(lo), -ml);
            dst[8 * k + 7] = __builtin_fmaf(dh, ubyte_sel<ASM, 3>(hi), -mh);
        }
    }
};
using GmQ4KMv = GmQ4KMvT<true>;

// Q5_K (kernels.c:1812-1833 q5_dequant_block, the decoder of its batched
// core, 2573-2595): Q4_K's pieces, with the fifth bit of each weight from
// qh: bytes 16 (p & 1) .. + 15 of qh, bit p / 2 (the sub-block).
template <bool ASM = true> struct GmQ5KT {
    uint4 hdr, q, h;
    __device__ __forceinline__ void load(const uint8_t *blk, uint32_t p) {
        hdr = *(const uint4 *)blk;
        h = *(const uint4 *)(blk + 16u + 16u * (p & 1u));
        q = *(const uint4 *)(blk + 48u + 32u * (p >> 2) + 16u * (p & 1u));
    }
    __device__ __forceinline__ void decode(uint32_t p, float *dst) const {
#pragma clang fp contract(off)
        float d1, m1;
        gm_q4k_sm(hdr, p >> 1, f16_to_f32(hdr.x), f16_to_f32(hdr.x >> 16), d1, m1);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w}, hb[4] = {h.x, h.y, h.z, h.w};
        const uint32_t shift = ((p >> 1) & 1u) ? 4u : 0u, bit = p >> 1;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t n = ((w[k] >> shift) & 0x0f0f0f0fu) | (((hb[k] >> bit) & 0x01010101u) << 4);
            dst[4 * k] = __builtin_fmaf(d1, ubyte_sel<ASM, 0>(n), -m1);
            dst[4 * k + 1] = __builtin_fmaf(d1, ubyte_sel<ASM, 1>(n), -m1);
            dst[4 * k + 2] = __builtin_fmaf(d1, ubyte_sel<ASM, 2>(n), -m1);
            dst[4 * k + 3] = __builtin_fmaf(d1, ubyte_sel<ASM, 3>(n), -m1);
        }
    }
};
using GmQ5K = GmQ5KT<true>;

// Q5_K in the matvec order (kernels.c:1785-1810): Q4_KMv's pieces and LDS
// order; qh bytes 8 (p & 3) .. + 7, bits 2 g (low) and 2 g + 1 (high).
template <bool ASM = true> struct GmQ5KMvT {
    uint4 hdr;
    uint2 q, h;
    __device__ __forceinline__ void load(const uint8_t *blk, uint32_t p) {
        hdr = *(const uint4 *)blk;
        h = *(const uint2 *)(blk + 16u + 8u * (p & 3u));
        q = *(const uint2 *)(blk + 48u + 32u * (p >> 2) + 8u * (p & 3u));
    }
    __device__ __forceinline__ void decode(uint32_t p, float *dst) const {
#pragma clang fp contract(off)
        const uint32_t g = p >> 2;
        const float d = f16_to_f32(hdr.x), dmin = f16_to_f32(hdr.x >> 16);
        float dl, ml, dh, mh;
        gm_q4k_sm(hdr, 2u * g, d, dmin, dl, ml);
        gm_q4k_sm(hdr, 2u * g + 1u, d, dmin, dh, mh);
        const uint32_t w[2] = {q.x, q.y}, hb[2] = {h.x, h.y};
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const uint32_t lo = (w[k] & 0x0f0f0f0fu) | (((hb[k] >> (2u * g)) & 0x01010101u) << 4);
            const uint32_t hi =
                ((w[k] >> 4) & 0x0f0f0f0fu) | (((hb[k] >> (2u * g + 1u)) & 0x01010101u) << 4);
            dst[8 * k + 0] = __builtin_fmaf(dl, ubyte_sel<ASM, 0>(lo), -ml);
            dst[8 * k + 1] = __builtin_fmaf(dh, ubyte_sel<ASM, 0>(hi), -mh);
            dst[8 * k + 2] = __builtin_fmaf(dl, ubyte_sel<ASM, 1>(lo), -ml);
            dst[8 * k + 3] = __builtin_fmaf(dh, ubyte_sel<ASM, 1>(hi), -mh);
            dst[8 * k + 4] = __builtin_fmaf(dl, ubyte_sel<ASM, 2>(lo), -ml);
            dst[8 * k + 5] = __builtin_fmaf(dh, ubyte_sel<ASM, 2>(hi), -mh);
            dst[8 * k + 6] = __builtin_fmaf(dl, ubyte_sel<ASM, 3>(lo), -ml);
            dst[8 * k + 7] = __builtin_fmaf(dh, ubyte_sel<ASM, 3>(hi), -mh);
        }
    }
};
using GmQ5KMv = GmQ5KMvT<true>;

// Q6_K: piece p = values 16 p .. + 15 = weight 128 h + 32 k + l for
// h = p / 8, k = (p / 2) & 3, l = 16 (p & 1) .. + 15; scale byte p.
template <bool ASM = true> struct GmQ6KT {
    uint32_t ql[4], qh[4], sd;   // sd: the int8 scale (low byte), d (high 16)
    __device__ __forceinline__ void load(const uint8_t *blk, uint32_t p) {
        const uint32_t h = p >> 3, k = (p >> 1) & 3u, l0 = 16u * (p & 1u);
        loadn_u16al<4>(blk + 64u * h + 32u * (k & 1u) + l0, ql);
        loadn_u16al<4>(blk + 128u + 32u * h + l0, qh);
        const uint8_t sc = blk[192u + p];
        const uint16_t dd = *(const uint16_t *)(blk + 208u);
        sd = (uint32_t)sc | ((uint32_t)dd << 16);
    }
    __device__ __forceinline__ void decode(uint32_t p, float *dst) const {
#pragma clang fp contract(off)
        const uint32_t k = (p >> 1) & 3u;
        const float d = f16_to_f32(sd >> 16);
        const float ds = d * (float)(int)(int8_t)(sd & 0xffu);
        const float n32 = -32.0f * ds;
        const uint32_t ns = (k < 2) ? 0u : 4u, hs = 2u * k;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const uint32_t q6 = ((ql[m] >> ns) & 0x0f0f0f0fu) | (((qh[m] >> hs) & 0x03030303u) << 4);
            dst[4 * m] = __builtin_fmaf(ds, ubyte_sel<ASM, 0>(q6), n32);
            dst[4 * m + 1] = __builtin_fmaf(ds, ubyte_sel<ASM, 1>(q6), n32);
            dst[4 * m + 2] = __builtin_fmaf(ds, ubyte_sel<ASM, 2>(q6), n32);
            dst[4 * m + 3] = __builtin_fmaf(ds, ubyte_sel<ASM, 3>(q6), n32);
        }
    }
};
using GmQ6K = GmQ6KT<true>;

// Q8_0 (a 256-value unit = eight 34-byte blocks): piece p = values
// 16 (p & 1) .. + 15 of block p / 2.
template <bool ASM = true> struct GmQ80T {
    uint32_t q[4], d;
    __device__ __forceinline__ void load(const uint8_t *blk8, uint32_t p) {
        const uint8_t *blk = blk8 + 34u * (p >> 1);
        d = *(const uint16_t *)blk;
        loadn_u16al<4>(blk + 2 + 16u * (p & 1u), q);
    }
    __device__ __forceinline__ void decode(uint32_t, float *dst) const {
#pragma clang fp contract(off)
        const float dd = f16_to_f32(d), n128 = -128.0f * dd;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const uint32_t v = q[m] ^ 0x80808080u;
            dst[4 * m] = __builtin_fmaf(dd, ubyte_sel<ASM, 0>(v), n128);
            dst[4 * m + 1] = __builtin_fmaf(dd, ubyte_sel<ASM, 1>(v), n128);
            dst[4 * m + 2] = __builtin_fmaf(dd, ubyte_sel<ASM, 2>(v), n128);
            dst[4 * m + 3] = __builtin_fmaf(dd, ubyte_sel<ASM, 3>(v), n128);
        }
    }
};
using GmQ80 = GmQ80T<true>;

// The x stage (64 tokens x 64 values) of unit u, stage st: 4 float4 per
// thread, token idx / 16 and float4 idx % 16 for idx = tid + 256 k.
MYNAH_DEV void gm_fetch_x(gm_f4 (&xr)[4], const float *__restrict__ x, uint32_t tid, uint32_t tok0,
                          uint32_t tokens, uint32_t cols, uint32_t u, uint32_t st) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t idx = tid + 256u * (uint32_t)k, xt = idx >> 4, xq = idx & 15u;
        const uint32_t t = tok0 + xt < tokens ? tok0 + xt : tokens - 1u;
        xr[k] = *(const gm_f4 *)(x + (size_t)t * cols + 256u * u + GM_STAGE * st + 4u * xq);
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
    // Decode role: row dr of the tile, 16-value piece dp of the stage.
    const uint32_t dr = tid >> 2, dp = tid & 3u;
    const uint32_t drow = row0 + dr < rows ? row0 + dr : rows - 1u;
    const uint8_t *wrow = w + (size_t)drow * row_bytes;
    gm_f4 xr[4];
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
        for (uint32_t st = 0; st < 4; st++) {
            float vals[16];
            raw.decode(4u * st + dp, vals);
#pragma unroll
            for (int k = 0; k < 4; k++)
                *(float4 *)&wl[dr][16u * dp + 4 * k] =
                    make_float4(vals[4 * k], vals[4 * k + 1], vals[4 * k + 2], vals[4 * k + 3]);
            if (ORD == 1 && (FMT == 12 || FMT == 13)) {
                // x in the matvec order of the stage's group: position 2 j + h
                // holds x[32 h + j].
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const uint32_t idx = tid + 256u * (uint32_t)k, xq = idx & 15u;
                    const uint32_t hh = xq >> 3, j = 4u * (xq & 7u);
                    float *dst = &xl[idx >> 4][2u * j + hh];
                    dst[0] = xr[k].x; dst[2] = xr[k].y; dst[4] = xr[k].z; dst[6] = xr[k].w;
                }
            } else {
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const uint32_t idx = tid + 256u * (uint32_t)k;
                    *(gm_f4 *)&xl[idx >> 4][4u * (idx & 15u)] = xr[k];
                }
            }
            __syncthreads();
            const uint32_t nu = st == 3 ? u + 1u : u, nst = (st + 1u) & 3u;
            if (nu < units) {
                raw.load(wrow + UB * nu, 4u * nst + dp);
                gm_fetch_x(xr, x, tid, tok0, tokens, cols, nu, nst);
            }
            for (uint32_t i = 0; i < GM_STAGE; i += 4) {
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
                    // Q8_0 matvec order: each 32-value block's sum joins the
                    // row total on its own.
#pragma unroll
                    for (int a = 0; a < 4; a++)
#pragma unroll
                        for (int b = 0; b < 4; b++) {
                            acc[a][b] = acc[a][b] + s[a][b];
                            s[a][b] = 0.0f;
                        }
                }
            }
            __syncthreads();
        }
        if (!(ORD == 1 && FMT == 8)) {
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 4; b++) acc[a][b] = acc[a][b] + s[a][b];
        }
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
// x 16-byte aligned. Q4_K / Q5_K rows 16-byte aligned, Q6_K / Q8_0 2-byte
// aligned.
#define GEMM_EXACT_ENTRY(name, RAW, UB)                                                        \
    extern "C" __global__ void __launch_bounds__(256)                                          \
        name(const uint8_t *__restrict__ w, const float *__restrict__ x, float *__restrict__ y, \
             uint32_t rows, uint32_t cols, uint32_t tokens, uint32_t row_bytes) {              \
        gemm_exact<RAW, UB>(w, x, y, rows, cols, tokens, row_bytes);                           \
    }

GEMM_EXACT_ENTRY(mynah_q4k_gemm_exact, GmQ4K, 144u)
GEMM_EXACT_ENTRY(mynah_q5k_gemm_exact, GmQ5K, 176u)
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

GEMM_MV_ENTRY(mynah_q4k_gemm_mv, GmQ4KMv, 144u, 12)
GEMM_MV_ENTRY(mynah_q5k_gemm_mv, GmQ5KMv, 176u, 13)
GEMM_MV_ENTRY(mynah_q6k_gemm_mv, GmQ6K, 210u, 14)
GEMM_MV_ENTRY(mynah_q80_gemm_mv, GmQ80, 272u, 8)
