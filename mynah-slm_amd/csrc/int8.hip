// int8.hip — the int8 activation lane of Q4_K products: the activation
// quantiser, the int8 matvec and the batched int8 GEMM on the matrix cores.
//
// The reference computes this lane in an AVX2 + FMA build of ingot
// (third_party/ingot/src/kernels.c:636-788 for the matvec, 1120-1751 for the
// batched form). Its arithmetic, which these kernels keep:
//   * quantiser (kernels.c:675-708): per 256-value super-block of a token,
//     amax = max |x|; scale = amax / 127, q = round-half-even(x * (127 / amax))
//     as int8; the eight sums of q over 32-value sub-blocks (all zero when
//     amax is 0);
//   * integer dots: Q4_K quants (0..15) times q over each 32-value sub-block,
//     exact in int32 whatever the order;
//   * matvec epilogue (kernels.c:712-739): per super-block
//     total = 0; per group g: total += d*sc*dot - dmin*m*sum for the low then
//     the high sub-block (products and sums separately rounded); the block's
//     value total * scale, summed over the row's super-blocks in order from 0;
//   * batched epilogue (kernels.c:1495-1581): per super-block and
//     (row, token), with scale_j = d*sc_j, offset_j = dmin*m_j:
//     total = fma(dot_j, scale_j, total); total = fma(-sum_j, offset_j, total)
//     for j = 0..7, for the tokens of a token tile that fall in whole groups
//     of four; the tile's last (count % 4) tokens take
//     total += scale_j*dot_j - offset_j*sum_j; then acc += total * scale,
//     super-block after super-block. The token tile is
//     clamp(4 MiB / (4 cols), 32, 128) rounded down to even (kernels.c:893-920).
// So every output is bit-identical to that build of the reference.
//
// Quantised activations live in HBM as xq[token][cols] int8,
// xs[token][cols / 256] f32 and xsum[token][cols / 32] int32.
//
// SPDX-License-Identifier: MIT
#include "common.hip.h"
#include "scratch.h"

typedef int i32x4 __attribute__((ext_vector_type(4)));

// The workspace of the allocation-free int8 product: one fixed array per
// device (each GPU that loads the code object holds its own copy until the
// process ends). The host resolves its device address by name when it loads
// the code object and passes that address to the kernels below as their xq /
// xs / xsum operands; nothing reads it before the quantiser has written it.
// No kernel names it (they take its address as an argument), so `used`
// keeps it in the code object's symbol table; the braces make this a
// definition with C linkage (a bare `extern "C"` would only declare it).
extern "C" {
__device__ __attribute__((aligned(256), used, visibility("default")))
unsigned char mynah_scratch[MYNAH_SCRATCH_BYTES];
}

// The (scale, min) pair of sub-block j from the 12 scale bytes s0..s2
// (kernels.c:83-92, scale_min), selects only.
MYNAH_DEV void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t j, uint32_t *sc,
                             uint32_t *m) {
    auto byte = [&](uint32_t k) -> uint32_t {
        const uint32_t wd = k < 4u ? s0 : (k < 8u ? s1 : s2);
        return (wd >> (8u * (k & 3u))) & 0xffu;
    };
    if (j < 4u) {
        *sc = byte(j) & 63u;
        *m = byte(j + 4u) & 63u;
    } else {
        *sc = (byte(j + 4u) & 15u) | ((byte(j - 4u) >> 6) << 4);
        *m = (byte(j + 4u) >> 4) | ((byte(j) >> 6) << 4);
    }
}

// ── quantiser ───────────────────────────────────────────────────────────
// One wave per (token, super-block); lane l holds values 4l..4l+3, so the
// lanes 8s..8s+7 hold sub-block s.
extern "C" __global__ __launch_bounds__(256) void mynah_q8_quantize(
    const float *__restrict__ x, int8_t *__restrict__ xq, float *__restrict__ xs,
    int32_t *__restrict__ xsum, uint32_t n_units, uint32_t nb, uint32_t cols) {
#pragma clang fp contract(off)
    const uint32_t u = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (u >= n_units) return;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t t = u / nb, b = u - t * nb;
    const size_t off = (size_t)t * cols + 256u * b + 4u * lane;
    const float4 v = *(const float4 *)(x + off);
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    for (int m = 32; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
    uint32_t packed = 0u;
    int32_t s = 0;
    float scale = 0.0f;
    if (amax > 0.0f) {
        scale = amax / 127.0f;
        const float inv = 127.0f / amax;
        const int32_t q0 = (int32_t)__builtin_rintf(v.x * inv);
        const int32_t q1 = (int32_t)__builtin_rintf(v.y * inv);
        const int32_t q2 = (int32_t)__builtin_rintf(v.z * inv);
        const int32_t q3 = (int32_t)__builtin_rintf(v.w * inv);
        s = q0 + q1 + q2 + q3;
        // |q| <= 127 here (|x| <= amax), so the saturating packs are identities.
        packed = ((uint32_t)q0 & 0xffu) | (((uint32_t)q1 & 0xffu) << 8) |
                 (((uint32_t)q2 & 0xffu) << 16) | ((uint32_t)q3 << 24);
    }
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    s += __shfl_xor(s, 4, 64);
    *(uint32_t *)(xq + off) = packed;
    if ((lane & 7u) == 0u) xsum[(size_t)u * 8u + (lane >> 3)] = s;
    if (lane == 0u) xs[u] = scale;
}

// ── int8 matvec (tokens == 1) ───────────────────────────────────────────
// One thread per (row, super-block): a workgroup owns `rpw` whole rows
// (rpw * nb <= 256 when nb <= 256), computes every block value into LDS, and
// one thread per row sums its row's values in order.
MYNAH_DEV float q4k_block_int8(const uint8_t *__restrict__ blk, const int8_t *__restrict__ q,
                               float xscale, const int32_t *__restrict__ sums) {
#pragma clang fp contract(off)
    const uint4 hdr = *(const uint4 *)blk;
    uint4 qs[8];
#pragma unroll
    for (int k = 0; k < 8; k++) qs[k] = ((const uint4 *)(blk + 16))[k];
    uint4 xv[16];
#pragma unroll
    for (int k = 0; k < 16; k++) xv[k] = ((const uint4 *)q)[k];
    const int4 s0 = ((const int4 *)sums)[0], s1 = ((const int4 *)sums)[1];
    const int32_t sm[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    const float d = f16_to_f32(hdr.x), dmin = f16_to_f32(hdr.x >> 16);
    float total = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        // Group g: quant bytes 32g..32g+31 = qs[2g], qs[2g+1]; the low nibbles
        // are sub-block 2g, the high ones 2g+1.
        const uint32_t wq[8] = {qs[2 * g].x,     qs[2 * g].y,     qs[2 * g].z,     qs[2 * g].w,
                                qs[2 * g + 1].x, qs[2 * g + 1].y, qs[2 * g + 1].z, qs[2 * g + 1].w};
        const uint4 xl0 = xv[4 * g], xl1 = xv[4 * g + 1], xh0 = xv[4 * g + 2], xh1 = xv[4 * g + 3];
        const uint32_t wl[8] = {xl0.x, xl0.y, xl0.z, xl0.w, xl1.x, xl1.y, xl1.z, xl1.w};
        const uint32_t wh[8] = {xh0.x, xh0.y, xh0.z, xh0.w, xh1.x, xh1.y, xh1.z, xh1.w};
        int32_t dl = 0, dh = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            dl = __builtin_amdgcn_sdot4((int)(wq[k] & 0x0f0f0f0fu), (int)wl[k], dl, false);
            dh = __builtin_amdgcn_sdot4((int)((wq[k] >> 4) & 0x0f0f0f0fu), (int)wh[k], dh, false);
        }
        uint32_t sl, ml, sh, mh;
        q4k_scale_min(hdr.y, hdr.z, hdr.w, 2u * g, &sl, &ml);
        q4k_scale_min(hdr.y, hdr.z, hdr.w, 2u * g + 1u, &sh, &mh);
        total += d * (float)sl * (float)dl - dmin * (float)ml * (float)sm[2 * g];
        total += d * (float)sh * (float)dh - dmin * (float)mh * (float)sm[2 * g + 1];
    }
    return total * xscale;
}

extern "C" __global__ __launch_bounds__(256) void mynah_q4k_gemv_int8(
    const uint8_t *__restrict__ w, const int8_t *__restrict__ xq, const float *__restrict__ xs,
    const int32_t *__restrict__ xsum, float *__restrict__ y, uint32_t rows, uint32_t nb,
    uint32_t rpw) {
#pragma clang fp contract(off)
    extern __shared__ float blockv[];   // rpw * nb values
    const uint32_t r0 = blockIdx.x * rpw;
    const uint32_t nrows = rows - r0 < rpw ? rows - r0 : rpw;
    const uint32_t n = nrows * nb;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const uint32_t rr = i / nb, b = i - rr * nb;
        const uint8_t *blk = w + ((size_t)(r0 + rr) * nb + b) * 144u;
        blockv[i] = q4k_block_int8(blk, xq + 256u * b, xs[b], xsum + 8u * b);
    }
    __syncthreads();
    for (uint32_t rr = threadIdx.x; rr < nrows; rr += blockDim.x) {
        float s = 0.0f;
        for (uint32_t b = 0; b < nb; b++) s += blockv[rr * nb + b];
        y[r0 + rr] = s;
    }
}

// ── batched int8 GEMM (tokens >= 2) ─────────────────────────────────────
// A workgroup is 2 x 2 waves; wave (wr, wt) owns GI_TR 16-row tiles and GI_TT
// 16-token tiles: rows R0 + 16 (GI_TR wr + i), tokens T0 + 16 (GI_TT wt + k).
// Per super-block and sub-block j, one v_mfma_i32_16x16x32_i8 per tile gives
// the tile's integer dots: lane l feeds row (l % 16) of the tile with the 8
// quants 8 (l / 16) .. +7 of the sub-block (A operand) and token (l % 16) with
// the same 8 activation positions (B operand), and receives the dots of rows
// 4 (l / 16) + e, e = 0..3, for token l % 16. Sub-blocks 2g and 2g+1 are the
// low and high nibbles of the same 8 quant bytes: one 8-byte read per group.
// Operands go through LDS: per super-block the workgroup copies its rows'
// quant bytes (Q5_K: qh and qs), its tokens' activations, sub-block sums and
// scales straight from global memory into LDS (global_load_lds_dwordx4 /
// _dword: no registers, nothing for the compiler to move), double buffered,
// the next super-block's copy in flight while the current one is summed;
// scale_j and offset_j of the rows are computed into LDS from the block
// headers. One barrier per super-block. Quants and activations sit in LDS
// chunk-major ([16-byte chunk][row or token][16 bytes]), so the 16 rows or
// tokens one operand read spans are 16 bytes apart and every read of a
// sub-block is the same per-lane address plus a constant. The dots of
// sub-block j + 1 are issued before the epilogue of j.
// Q5_K (FMT 13, kernels.c:1155-1185 q5_k_quants): the same tiles, the quant
// bytes at block offset 48 instead of 16, and each lane also holds the 8 qh
// bytes of its 8 positions: bit j of qh[i] is the fifth bit (+16) of weight
// i of sub-block j.
// Bytes of one row's staged quant data per super-block: Q4_K qs (block bytes
// 16 .. 143), Q5_K qh + qs (block bytes 16 .. 175).
template <int FMT>
constexpr uint32_t gi_qb() { return FMT == 13 ? 160u : 128u; }

typedef __attribute__((address_space(3))) void gi_lds_void;

// Copy super-block b of the workgroup's rows and tokens into LDS buffer
// (lq, lx, lsum, lxs); wave w takes every fourth 64-chunk piece. Rows and
// tokens past the ends read the last one (their results are not stored).
// Copy super-block b of the workgroup's rows and tokens into LDS buffer
// (lq, lx, lsum, lxs): lq[c][r] = 16-byte chunk c of row r's staged bytes,
// lx[c][t] = chunk c of token t's 256 activations, lsum[t] = its 8 sums,
// lxs[t] = its scale. Each copy instruction fills 1 KiB (64 lanes x 16
// bytes); wave w takes every fourth one. Rows and tokens past the ends read
// the last one (their results are not stored).
template <int FMT, int GI_ROWS, int GI_TOK>
MYNAH_DEV void gi_stage_async(uint8_t *lq, int8_t *lx, int32_t *lsum, float *lxs,
                              const uint8_t *__restrict__ w, const int8_t *__restrict__ xq,
                              const float *__restrict__ xs, const int32_t *__restrict__ xsum,
                              uint32_t R0, uint32_t T0, uint32_t rows, uint32_t tokens,
                              uint32_t cols, uint32_t nb, size_t rb, uint32_t b, uint32_t wave,
                              uint32_t lane) {
    constexpr uint32_t QB = gi_qb<FMT>(), CPR = QB / 16u, UB = FMT == 13 ? 176u : 144u;
    constexpr uint32_t NQ = GI_ROWS * CPR / 64u, NX = GI_TOK * 16u / 64u, NS = GI_TOK * 2u / 64u;
    // Workgroup-uniform bases; per-lane offsets stay below 4 GiB (at most 64
    // rows or tokens of the tile).
    const uint8_t *wb = w + (size_t)R0 * rb + (size_t)b * UB + 16u;
    const int8_t *xb = xq + (size_t)T0 * cols + 256u * b;
    const int32_t *sb = xsum + ((size_t)T0 * nb + b) * 8u;
    const uint32_t rmax = rows - 1u - R0, tmax = tokens - 1u - T0;
#pragma unroll
    for (uint32_t k = 0; k < (NQ + 3u) / 4u; k++) {
        const uint32_t n = 4u * k + wave;
        if (n < NQ) {
            const uint32_t p = 64u * n + lane, c = p / GI_ROWS, r = p - c * GI_ROWS;
            const uint32_t rr = r < rmax ? r : rmax;
            __builtin_amdgcn_global_load_lds((const void *)(wb + (uint32_t)(rr * (uint32_t)rb +
                                                                              16u * c)),
                                             (gi_lds_void *)(lq + 1024u * n), 16, 0, 0);
        }
    }
#pragma unroll
    for (uint32_t k = 0; k < (NX + 3u) / 4u; k++) {
        const uint32_t n = 4u * k + wave;
        if (n < NX) {
            const uint32_t p = 64u * n + lane, c = p / GI_TOK, t = p - c * GI_TOK;
            const uint32_t tt = t < tmax ? t : tmax;
            __builtin_amdgcn_global_load_lds((const void *)(xb + (uint32_t)(tt * cols + 16u * c)),
                                             (gi_lds_void *)(lx + 1024u * n), 16, 0, 0);
        }
    }
#pragma unroll
    for (uint32_t k = 0; k < (NS + 3u) / 4u; k++) {
        const uint32_t n = 4u * k + wave;
        if (n < NS) {
            const uint32_t p = 64u * n + lane, t = p >> 1, tt = t < tmax ? t : tmax;
            __builtin_amdgcn_global_load_lds(
                (const void *)(sb + (uint32_t)(tt * nb * 8u + 4u * (p & 1u))),
                (gi_lds_void *)(lsum + 256u * n), 16, 0, 0);
        }
    }
    if (wave == 3u && lane < (uint32_t)GI_TOK) {
        const uint32_t tt = lane < tmax ? lane : tmax;
        __builtin_amdgcn_global_load_lds((const void *)(xs + (size_t)T0 * nb + b + tt * nb),
                                         (gi_lds_void *)lxs, 4, 0, 0);
    }
}

// Scale and offset of sub-blocks hj, hj + 1 of the staged row, into LDS.
template <int GI_ROWS>
MYNAH_DEV void gi_stage(float *buf, const uint4 hdr, uint32_t hj, uint32_t row) {
#pragma clang fp contract(off)
    const float d = f16_to_f32(hdr.x), dmin = f16_to_f32(hdr.x >> 16);
    uint32_t s0, m0, s1, m1;
    q4k_scale_min(hdr.y, hdr.z, hdr.w, hj, &s0, &m0);
    q4k_scale_min(hdr.y, hdr.z, hdr.w, hj + 1u, &s1, &m1);
    buf[hj * GI_ROWS + row] = d * (float)s0;
    buf[(hj + 1u) * GI_ROWS + row] = d * (float)s1;
    buf[(8u + hj) * GI_ROWS + row] = dmin * (float)m0;
    buf[(9u + hj) * GI_ROWS + row] = dmin * (float)m1;
}

// One super-block's dots and epilogue from the LDS buffers: lane l's rows
// 16 (GI_TR wr + i) + l % 16 and tokens 16 (GI_TT wt + k) + l % 16, quant and
// activation positions 32 g + 8 (l / 16) .. +7 of group g / sub-block j;
// tot[i][k][e] over j = 0..7 in order, then acc += tot * xs. MIXED: some
// lane has a token outside the groups of four, which takes the plain form.
template <int FMT, bool MIXED, int GI_TR, int GI_TT>
MYNAH_DEV void gi_block(float (&acc)[GI_TR][GI_TT][4], const uint8_t *lq, const int8_t *lx,
                        const int32_t *lsum, const float *lxs, const float4 *sbuf, uint32_t wr,
                        uint32_t wt, uint32_t lane, const bool (&fma_path)[GI_TT]) {
#pragma clang fp contract(off)
    constexpr int GI_ROWS = 32 * GI_TR, GI_TOK = 32 * GI_TT;
    const uint32_t lm = lane & 15u, lk = lane >> 4;
    // Lane l reads the 8 bytes at position 8 (l / 16) of a 32-byte group:
    // chunk 2 g + (l / 16) / 2 of its row / token, half (l / 16) % 2.
    const uint32_t lo = 16u * (lk >> 1), hb = 8u * (lk & 1u);
    const uint8_t *qrow[GI_TR];
    const int8_t *xrow[GI_TT];
    uint32_t tl[GI_TT];
#pragma unroll
    for (int i = 0; i < GI_TR; i++)
        qrow[i] = lq + 16u * (16u * (GI_TR * wr + (uint32_t)i) + lm) + hb + lo * GI_ROWS;
#pragma unroll
    for (int k = 0; k < GI_TT; k++) {
        tl[k] = 16u * (GI_TT * wt + (uint32_t)k) + lm;
        xrow[k] = lx + 16u * tl[k] + hb + lo * GI_TOK;
    }
    unsigned long long qh[GI_TR];
    if (FMT == 13) {
#pragma unroll
        for (int i = 0; i < GI_TR; i++) qh[i] = *(const unsigned long long *)qrow[i];
    }
    // Dots of sub-block j: the quant bytes of group j / 2 of each row tile
    // (Q5_K: its qs start at chunk 2), nibble j % 2, times the activations
    // of sub-block j of each token tile. The loop below stays rolled (runtime
    // j), so no more than two sub-blocks' dots are ever live.
    auto dots = [&](i32x4 (&dt)[GI_TR][GI_TT], uint32_t j) {
        unsigned long long xb[GI_TT];
#pragma unroll
        for (int k = 0; k < GI_TT; k++)
            xb[k] = *(const unsigned long long *)(xrow[k] + 16u * GI_TOK * 2u * j);
#pragma unroll
        for (int i = 0; i < GI_TR; i++) {
            const uint32_t c = (FMT == 13 ? 2u : 0u) + 2u * (j >> 1);
            const unsigned long long qa =
                *(const unsigned long long *)(qrow[i] + 16u * GI_ROWS * c);
            unsigned long long q = (qa >> (4u * (j & 1u))) & 0x0f0f0f0f0f0f0f0full;
            if (FMT == 13) q |= ((qh[i] >> j) & 0x0101010101010101ull) << 4;
#pragma unroll
            for (int k = 0; k < GI_TT; k++) {
                const i32x4 zero = {0, 0, 0, 0};
                dt[i][k] = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)q, (long)xb[k], zero, 0, 0,
                                                                 0);
            }
        }
    };
    float tot[GI_TR][GI_TT][4];
#pragma unroll
    for (int i = 0; i < GI_TR; i++)
#pragma unroll
        for (int k = 0; k < GI_TT; k++)
#pragma unroll
            for (int e = 0; e < 4; e++) tot[i][k][e] = 0.0f;
    // tot = fma(-xsum_j, offset_j, fma(dot_j, scale_j, tot)) for sub-block j.
    auto epi = [&](const i32x4 (&dt)[GI_TR][GI_TT], uint32_t j) {
        float xsj[GI_TT];
#pragma unroll
        for (int k = 0; k < GI_TT; k++) xsj[k] = (float)lsum[8u * tl[k] + j];
#pragma unroll
        for (int i = 0; i < GI_TR; i++) {
            const uint32_t slot = (16u * (GI_TR * wr + i)) / 4u + lk;
            const float4 sc = sbuf[j * (GI_ROWS / 4) + slot];
            const float4 of = sbuf[(8u + j) * (GI_ROWS / 4) + slot];
            const float scv[4] = {sc.x, sc.y, sc.z, sc.w};
            const float ofv[4] = {of.x, of.y, of.z, of.w};
#pragma unroll
            for (int k = 0; k < GI_TT; k++) {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float dv = (float)dt[i][k][e];
                    float f = __builtin_fmaf(dv, scv[e], tot[i][k][e]);
                    f = __builtin_fmaf(-xsj[k], ofv[e], f);
                    if (MIXED) {
                        const float p = tot[i][k][e] + (scv[e] * dv - ofv[e] * xsj[k]);
                        f = fma_path[k] ? f : p;
                    }
                    tot[i][k][e] = f;
                }
            }
        }
    };
    // Two register sets of dots, alternating: the dots of sub-block j + 1
    // are issued before the epilogue of j, with no copies between them.
    i32x4 da[GI_TR][GI_TT], db[GI_TR][GI_TT];
    dots(da, 0u);
#pragma unroll 1
    for (uint32_t j = 0; j < 6u; j += 2u) {
        dots(db, j + 1u);
        epi(da, j);
        dots(da, j + 2u);
        epi(db, j + 1u);
    }
    dots(db, 7u);
    epi(da, 6u);
    epi(db, 7u);
#pragma unroll
    for (int i = 0; i < GI_TR; i++)
#pragma unroll
        for (int k = 0; k < GI_TT; k++) {
            const float xsv = lxs[tl[k]];
#pragma unroll
            for (int e = 0; e < 4; e++) acc[i][k][e] = acc[i][k][e] + tot[i][k][e] * xsv;
        }
}

template <int FMT, int GI_TR, int GI_TT>
MYNAH_DEV void gemm_int8(const uint8_t *__restrict__ w, const int8_t *__restrict__ xq,
                         const float *__restrict__ xs, const int32_t *__restrict__ xsum,
                         float *__restrict__ y, uint32_t rows, uint32_t cols, uint32_t tokens,
                         uint32_t nb, uint32_t tile) {
    constexpr int GI_ROWS = 32 * GI_TR, GI_TOK = 32 * GI_TT;
    constexpr uint32_t QB = gi_qb<FMT>();
    __shared__ __attribute__((aligned(16))) uint8_t lq[2][GI_ROWS * QB];
    __shared__ __attribute__((aligned(16))) int8_t lx[2][GI_TOK * 256];
    __shared__ __attribute__((aligned(16))) int32_t lsum[2][GI_TOK * 8];
    __shared__ __attribute__((aligned(16))) float lxs[2][GI_TOK];
    __shared__ float4 so[2][16 * GI_ROWS / 4];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t wr = wave & 1u, wt = wave >> 1;
    const uint32_t R0 = blockIdx.x * GI_ROWS, T0 = blockIdx.y * GI_TOK;
    const size_t rb = (size_t)nb * (FMT == 13 ? 176u : 144u);
    const uint32_t lm = lane & 15u, lk = lane >> 4;

    uint32_t tok[GI_TT];
    bool fma_path[GI_TT];
    bool all_fma = true;
#pragma unroll
    for (int k = 0; k < GI_TT; k++) {
        const uint32_t t = T0 + 16u * (GI_TT * wt + k) + lm;
        tok[k] = t;
        const uint32_t tc = t < tokens ? t : tokens - 1u;
        const uint32_t t0 = tc - tc % tile;
        const uint32_t cnt = tokens - t0 < tile ? tokens - t0 : tile;
        fma_path[k] = tc - t0 < (cnt & ~3u);
        all_fma = all_fma && fma_path[k];
    }
    const bool mixed = !__all(all_fma);
    // Scale staging: thread tid owns row tid / 4 of the workgroup, sub-blocks
    // 2 (tid % 4) and 2 (tid % 4) + 1 (threads beyond 4 GI_ROWS stage nothing).
    const uint32_t srow = tid >> 2, hj = 2u * (tid & 3u);
    const bool stager = srow < GI_ROWS;
    uint32_t hr = R0 + (stager ? srow : 0u);
    hr = hr < rows ? hr : rows - 1u;
    const uint8_t *hrow = w + (size_t)hr * rb;
    constexpr uint32_t UB = FMT == 13 ? 176u : 144u;

    float acc[GI_TR][GI_TT][4];
#pragma unroll
    for (int i = 0; i < GI_TR; i++)
#pragma unroll
        for (int k = 0; k < GI_TT; k++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[i][k][e] = 0.0f;

    gi_stage_async<FMT, GI_ROWS, GI_TOK>(lq[0], lx[0], lsum[0], lxs[0], w, xq, xs, xsum, R0, T0,
                                         rows, tokens, cols, nb, rb, 0u, wave, lane);
    uint4 hdr = *(const uint4 *)hrow;
    __builtin_amdgcn_s_waitcnt(0);
    if (stager) gi_stage<GI_ROWS>((float *)so[0], hdr, hj, srow);
    __syncthreads();
    for (uint32_t b = 0; b < nb; b++) {
        const uint32_t c = b & 1u;
        const bool more = b + 1u < nb;
        if (more) {
            gi_stage_async<FMT, GI_ROWS, GI_TOK>(lq[c ^ 1u], lx[c ^ 1u], lsum[c ^ 1u],
                                                 lxs[c ^ 1u], w, xq, xs, xsum, R0, T0, rows,
                                                 tokens, cols, nb, rb, b + 1u, wave, lane);
            hdr = *(const uint4 *)(hrow + (size_t)(b + 1u) * UB);
        }
        if (mixed)
            gi_block<FMT, true>(acc, lq[c], lx[c], lsum[c], lxs[c], so[c], wr, wt, lane,
                                fma_path);
        else
            gi_block<FMT, false>(acc, lq[c], lx[c], lsum[c], lxs[c], so[c], wr, wt, lane,
                                 fma_path);
        if (more) {
            __builtin_amdgcn_s_waitcnt(0);
            if (stager) gi_stage<GI_ROWS>((float *)so[c ^ 1u], hdr, hj, srow);
        }
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < GI_TR; i++)
#pragma unroll
        for (int k = 0; k < GI_TT; k++) {
            if (tok[k] >= tokens) continue;
            float *yo = y + (size_t)tok[k] * rows;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t r = R0 + 16u * (GI_TR * wr + i) + 4u * lk + e;
                if (r < rows) yo[r] = acc[i][k][e];
            }
        }
}

#define GEMM_INT8(NAME, FMT, TR, TT)                                                         \
    extern "C" __global__ __launch_bounds__(256, 2) void NAME##_##TR##TT(                    \
        const uint8_t *__restrict__ w, const int8_t *__restrict__ xq,                        \
        const float *__restrict__ xs, const int32_t *__restrict__ xsum,                      \
        float *__restrict__ y, uint32_t rows, uint32_t cols, uint32_t tokens, uint32_t nb,   \
        uint32_t tile) {                                                                     \
        gemm_int8<FMT, TR, TT>(w, xq, xs, xsum, y, rows, cols, tokens, nb, tile);            \
    }
GEMM_INT8(mynah_q4k_gemm_int8, 12, 1, 1)
GEMM_INT8(mynah_q4k_gemm_int8, 12, 1, 2)
GEMM_INT8(mynah_q4k_gemm_int8, 12, 2, 1)
GEMM_INT8(mynah_q4k_gemm_int8, 12, 2, 2)
GEMM_INT8(mynah_q5k_gemm_int8, 13, 2, 2)
