// gemm_mfma.hip — the exact batched GEMM with its products on the matrix
// cores and only the ordered sums on the VALU.
//
// Same outputs, bit for bit, as gemm_exact.hip in both of its orders (the
// reference's batched order, third_party/ingot/src/kernels.c:1017-1039,
// 1053-1104, 2635-2648, and the matvec order of kernels.c:94-115, 319-337,
// 2525-2551): each super-block sum starts from 0 and takes the products
// w[i] * x[i] one at a time in that order, and the row total takes the
// super-block sums in order.
//
// Products: v_mfma_f32_16x16x1_4b_f32 with a zero accumulator forms the
// 4 x 16 x 16 outer products a_i * b_j of one column step; each is
// round(a_i * b_j) + 0, the bits of v_mul_f32 except that a -0 product
// comes out +0 (checked on gfx950 over 4.2 million operand pairs of this
// instruction and 8.4 million of its 32 x 32 sibling: normal, subnormal,
// zero, infinite and NaN operands, every one equal or a zero of the other
// sign). A zero's sign cannot reach a sum here: a running sum
// starts at +0 and x + (+0) == x + (-0) for every x except -0, which a sum
// that starts at +0 never holds (only -0 + -0 gives -0). Each product is then
// added to its running sum with its own v_add_f32 (no contraction), in
// column order — the same roundings as the VALU kernel, at one VALU
// instruction per product instead of two. The instruction's accumulate form
// (D = A B + C) cannot carry the sums: on gfx950 it rounds once, like fma
// (equal to fmaf on 16.8 million single and chained cases, and unlike a
// multiply then an add on a third of them), where the reference rounds the
// product and the sum separately.
//
// Tiling: a workgroup of 256 threads owns 64 rows x 64 tokens; wave w the
// tokens 16 w .. 16 w + 15. Per column step k lane l feeds A = w[row l][k]
// (the MFMA's four blocks are rows 0..15, .., 48..63) and B = x[token
// 16 w + l % 16][k] (every block sees the same 16 tokens); lane l then holds,
// in register r, the product of row 16 (r / 4) + 4 (l / 16) + r % 4 and
// token l % 16. The weights are decoded into LDS a 64-value
// stage at a time with the decoders of gemm_exact.hip (16 values per
// thread), x is copied beside them (for the Q4_K / Q5_K matvec order in the
// interleaved order), and the next stage is fetched into registers while the
// current one is summed. Within a stage each column's products land in their
// own registers and the next column's MFMA is issued before this column's
// adds (scheduling barriers pin that order), so the matrix core and the VALU
// work at the same time.
//
// Split K (gridDim.z > 1): workgroup z takes the units [z U / Z, (z + 1) U /
// Z); z = 0 stores the running row total of its units (from 0, in order) to
// part[0][token][row], every other z stores each unit's sum to
// part[u][token][row]; mynah_gemm_fold then continues the total from slot 0
// over the later units in order (and adds res), the row total the single
// launch would give. Not for the Q8_0 matvec order, whose row total takes
// every 32-value block sum.
//
// SPDX-License-Identifier: MIT
#include "common.hip.h"

#define GF_ROWS 64
#define GF_TOK 64
#define GF_STAGE 64
#define GF_LD (GF_STAGE + 4)

typedef float gf_f32x16 __attribute__((ext_vector_type(16)));

// Row of the tile that register r of lane l holds.
MYNAH_DEV uint32_t gf_row(int r, uint32_t lane) {
    return 16u * (uint32_t)(r >> 2) + 4u * (lane >> 4) + (uint32_t)(r & 3);
}

template <class Raw, uint32_t UB, int ORD = 0, int FMT = 0>
MYNAH_DEV void gemm_mfma(const uint8_t *__restrict__ w, const float *__restrict__ x, float *y,
                         uint32_t rows, uint32_t cols, uint32_t tokens, uint32_t row_bytes,
                         const float *res, float *__restrict__ part) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) float wl[GF_ROWS][GF_LD];
    __shared__ __attribute__((aligned(16))) float xl[GF_TOK][GF_LD];
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
    const uint32_t row0 = blockIdx.x * GF_ROWS, tok0 = blockIdx.y * GF_TOK;
    const uint32_t units = cols / 256u;
    const uint32_t nz = gridDim.z, z = blockIdx.z;
    const uint32_t u0 = (uint32_t)(((uint64_t)units * z) / nz);
    const uint32_t u1 = (uint32_t)(((uint64_t)units * (z + 1u)) / nz);
    const bool split = nz > 1u;
    // Decode role: row dr of the tile, 16-value piece dp of the stage.
    const uint32_t dr = tid >> 2, dp = tid & 3u;
    const uint32_t drow = row0 + dr < rows ? row0 + dr : rows - 1u;
    const uint8_t *wrow = w + (size_t)drow * row_bytes;
    // MFMA operands: A = row `lane` of the tile, B = token tb of the tile.
    const uint32_t tb = 16u * wave + (lane & 15u);
    gm_f4 xr[4];
    Raw raw;
    const gf_f32x16 zero = {};
    gf_f32x16 acc = zero, s = zero;

    if (u0 < u1) {
        raw.load(wrow + UB * u0, dp);
        gm_fetch_x(xr, x, tid, tok0, tokens, cols, u0, 0u);
    }
    for (uint32_t u = u0; u < u1; u++) {
        s = zero;
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
            if (nu < u1) {
                raw.load(wrow + UB * nu, 4u * nst + dp);
                gm_fetch_x(xr, x, tid, tok0, tokens, cols, nu, nst);
            }
            // Software-pipelined by one column: the products of column k + 1
            // are issued (into their own registers) before the 16 adds of
            // column k, so the matrix core works while the VALU adds.
            float4 a4 = *(const float4 *)&wl[lane][0];
            float4 b4 = *(const float4 *)&xl[tb][0];
            gf_f32x16 pc = __builtin_amdgcn_mfma_f32_16x16x1f32(a4.x, b4.x, zero, 0, 0, 0);
#pragma unroll
            for (uint32_t i = 0; i < GF_STAGE; i += 4) {
                float4 an = a4, bn = b4;
                if (i + 4u < GF_STAGE) {
                    an = *(const float4 *)&wl[lane][i + 4u];
                    bn = *(const float4 *)&xl[tb][i + 4u];
                }
                const float av[5] = {a4.x, a4.y, a4.z, a4.w, an.x};
                const float bv[5] = {b4.x, b4.y, b4.z, b4.w, bn.x};
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    gf_f32x16 pn = zero;
                    if (c < 3 || i + 4u < GF_STAGE)
                        pn = __builtin_amdgcn_mfma_f32_16x16x1f32(av[c + 1], bv[c + 1],
                                                                  zero, 0, 0, 0);
                    // Nothing crosses these: the next column's MFMA stays
                    // ahead of this column's adds.
                    __builtin_amdgcn_sched_barrier(0);
                    s = s + pc;
                    __builtin_amdgcn_sched_barrier(0);
                    pc = pn;
                }
                if (ORD == 1 && FMT == 8 && (i & 31u) == 28u) {
                    // Q8_0 matvec order: each 32-value block's sum joins the
                    // row total on its own.
                    acc = acc + s;
                    s = zero;
                }
                a4 = an;
                b4 = bn;
            }
            __syncthreads();
        }
        if (!(ORD == 1 && FMT == 8)) {
            if (split && z > 0u) {
                // Unit u's sums, for the in-order fold.
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const uint32_t row = row0 + gf_row(r, lane);
                    const uint32_t t = tok0 + tb;
                    if (row < rows && t < tokens)
                        part[((size_t)u * tokens + t) * rows + row] = s[r];
                }
            } else {
                acc = acc + s;
            }
        }
    }
    if (split) {
        // The first split's units start the row total: its running sum from
        // 0 is what the fold would reach after them, stored in slot 0.
        if (z == 0u) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const uint32_t row = row0 + gf_row(r, lane);
                const uint32_t t = tok0 + tb;
                if (row < rows && t < tokens) part[(size_t)t * rows + row] = acc[r];
            }
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const uint32_t row = row0 + gf_row(r, lane);
        const uint32_t t = tok0 + tb;
        if (row < rows && t < tokens) {
            const size_t o = (size_t)t * rows + row;
            y[o] = res ? res[o] + acc[r] : acc[r];
        }
    }
}

// Grid (ceil(rows / 64), ceil(tokens / 64), Z), block 256; cols % 256 == 0;
// x 16-byte aligned; Q4_K / Q5_K rows 16-byte aligned, Q6_K / Q8_0 2-byte
// aligned. ORD 0 = the batched order, 1 = the matvec order; res (may be
// NULL or alias y) is added when Z == 1; part: Z > 1 only.
#define GEMM_MFMA_ENTRY(name, RAW, UB, ORD, FMT)                                               \
    extern "C" __global__ void __launch_bounds__(256, 2)                                       \
        name(const uint8_t *__restrict__ w, const float *__restrict__ x, float *y,             \
             uint32_t rows, uint32_t cols, uint32_t tokens, uint32_t row_bytes,                \
             const float *res, float *part) {                                                  \
        gemm_mfma<RAW, UB, ORD, FMT>(w, x, y, rows, cols, tokens, row_bytes, res, part);       \
    }

GEMM_MFMA_ENTRY(mynah_q4k_gemm_exact_mfma, GmQ4KT<false>, 144u, 0, 12)
GEMM_MFMA_ENTRY(mynah_q5k_gemm_exact_mfma, GmQ5KT<false>, 176u, 0, 13)
GEMM_MFMA_ENTRY(mynah_q6k_gemm_exact_mfma, GmQ6KT<false>, 210u, 0, 14)
GEMM_MFMA_ENTRY(mynah_q80_gemm_exact_mfma, GmQ80T<false>, 272u, 0, 8)
GEMM_MFMA_ENTRY(mynah_q4k_gemm_mv_mfma, GmQ4KMvT<false>, 144u, 1, 12)
GEMM_MFMA_ENTRY(mynah_q5k_gemm_mv_mfma, GmQ5KMvT<false>, 176u, 1, 13)
GEMM_MFMA_ENTRY(mynah_q6k_gemm_mv_mfma, GmQ6KT<false>, 210u, 1, 14)
GEMM_MFMA_ENTRY(mynah_q80_gemm_mv_mfma, GmQ80T<false>, 272u, 1, 8)

// The in-order fold of split-K unit sums: y[t][r] = (res[t][r] +) the row
// total continued from part[0][t][r] (the first split's running total over
// its units 0 .. first - 1) over part[u][t][r], u = first .. units - 1, in
// order — the row total of the reference's order. One thread per output,
// consecutive rows consecutive threads; the loads go out four at a time.
extern "C" __global__ void __launch_bounds__(256)
mynah_gemm_fold(const float *__restrict__ part, const float *res, float *y, uint32_t rows,
                uint32_t tokens, uint32_t first, uint32_t units) {
#pragma clang fp contract(off)
    const uint64_t n = (uint64_t)rows * tokens;
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float acc = part[i];
    uint32_t u = first;
    for (; u + 4u <= units; u += 4u) {
        float v[4];
#pragma unroll
        for (uint32_t k = 0; k < 4; k++) v[k] = part[(size_t)(u + k) * n + i];
#pragma unroll
        for (uint32_t k = 0; k < 4; k++) acc = acc + v[k];
    }
    for (; u < units; u++) acc = acc + part[(size_t)u * n + i];
    y[i] = res ? res[i] + acc : acc;
}

// Test hook for the product claim at the top of this file (no reference
// counterpart). Per workgroup (one wave): 64 values of a and of b, lane l
// feeding A and B of block l / 16 at row / column l % 16, and 1024 of c.
// prod = the instruction with a zero accumulator, acc = the same with c as
// the accumulator; mul and fused = the VALU's a * b and fmaf(a, b, c) of the
// same operand pairs. Every output is in the instruction's layout: lane l,
// register r holds block r / 4, row 4 (l / 16) + r % 4, column l % 16, at
// index 1024 blockIdx + 16 l + r.
extern "C" __global__ void __launch_bounds__(64)
mynah_mfma_probe(const float *__restrict__ a, const float *__restrict__ b,
                 const float *__restrict__ c, float *__restrict__ prod,
                 float *__restrict__ acc, float *__restrict__ mul, float *__restrict__ fused) {
#pragma clang fp contract(off)
    const uint32_t l = threadIdx.x;
    const size_t base = 64u * (size_t)blockIdx.x, out = 16u * (base + l);
    const gf_f32x16 zero = {};
    gf_f32x16 cv;
#pragma unroll
    for (int r = 0; r < 16; r++) cv[r] = c[out + r];
    const gf_f32x16 p = __builtin_amdgcn_mfma_f32_16x16x1f32(a[base + l], b[base + l], zero, 0, 0, 0);
    const gf_f32x16 q = __builtin_amdgcn_mfma_f32_16x16x1f32(a[base + l], b[base + l], cv, 0, 0, 0);
#pragma unroll
    for (uint32_t r = 0; r < 16; r++) {
        const uint32_t blk = r / 4u, row = 4u * (l / 16u) + r % 4u, col = l % 16u;
        const float x = a[base + 16u * blk + row], y = b[base + 16u * blk + col];
        prod[out + r] = p[r];
        acc[out + r] = q[r];
        mul[out + r] = x * y;
        fused[out + r] = __builtin_fmaf(x, y, cv[r]);
    }
}
