// gemv_exact.hip — decode GEMV bit-identical to the reference's CPU kernels.
//
// The reference's matvec sums in one fixed f32 order, and on these inputs its
// own rounding error reaches ~1e-4 of max(1, |y|): a reordered sum cannot
// stay within that of it everywhere. These kernels therefore reproduce the
// as-built x86 order exactly (same products, same roundings, no contraction):
//   Q4_K  third_party/ingot/src/kernels.c:94-115 (dot_block) and 319-337: per
//         super-block one running sum, the low-nibble weight 64g+i then the
//         high-nibble weight 64g+32+i for i = 0..31, g = 0..3; weight value
//         (d*sc)*q - dmin*m (one rounding); row sum of block sums in order.
//   Q6_K  kernels.c:2096-2124 + 2176-2199 + 2037-2041: decode the 256 values
//         (d*sc)*(q-32), sequential dot from weight 0, row sum in order.
//   Q8_0  kernels.c:2518-2546: values q*d, sequential dot per 32-block, row
//         sum in order.
// Every weight value is exact in f32 before its final rounding, so a single
// fused multiply-add produces the identical value: (d*sc)*q - dmin*m as
// fma(d*sc, q, -dmin*m); (d*sc)*(q-32) as fma(d*sc, q6, -32*d*sc) with q6 the
// raw 6-bit code; q*d as fma(d, q + 128, -128*d) with q + 128 = q ^ 0x80. The
// product with x and the sum stay separate roundings, as in the reference.
//
// No product is ever fused with a sum here: the library is compiled with
// -ffp-contract=off and every summing function repeats it as a pragma.
//
// Decomposition: lane = output row (64 rows per workgroup); a "unit" is one
// super-block (Q4_K, Q6_K) or one 32-value block (Q8_0); wave w of the W waves
// of a workgroup computes the unit sums of units w, w+W, ... of its 64 rows.
// The unit index is wave-uniform, so x is read with scalar loads and fed to
// the VALU as SGPR operands. Each phase of W units lands in LDS and wave 0
// folds it into the running row sums in unit order.
//
// SPDX-License-Identifier: MIT
#include "common.hip.h"

#define EX_ROWS 64
#define EX_MAX_WAVES 16

// ── Q4_K: 144-byte block, 16-byte aligned ──────────────────────────────────

template <int J>
MYNAH_DEV void q4k_sm(uint32_t s0, uint32_t s1, uint32_t s2, float &sc, float &m) {
    if (J < 4) {
        sc = (float)((s0 >> (8 * J)) & 63u);
        m = (float)((s1 >> (8 * J)) & 63u);
    } else {
        const uint32_t k = 8 * (J - 4);
        sc = (float)(((s2 >> k) & 15u) | (((s0 >> (k + 6)) & 3u) << 4));
        m = (float)(((s2 >> (k + 4)) & 15u) | (((s1 >> (k + 6)) & 3u) << 4));
    }
}

template <int G>
MYNAH_DEV float q4k_group(const uint32_t *q, float d, float dmin, uint32_t s0, uint32_t s1,
                          uint32_t s2, const float *__restrict__ x, float acc) {
#pragma clang fp contract(off)
    float sa, ma, sb, mb;
    q4k_sm<2 * G>(s0, s1, s2, sa, ma);
    q4k_sm<2 * G + 1>(s0, s1, s2, sb, mb);
    const float da = d * sa, db = d * sb, oa = dmin * ma, ob = dmin * mb;
#pragma unroll
    for (int m = 0; m < 8; m++) {
        const uint32_t v = q[8 * G + m];
        const uint32_t lo = v & 0x0f0f0f0fu, hi = (v >> 4) & 0x0f0f0f0fu;
        const float ql[4] = {ubyte_f<0>(lo), ubyte_f<1>(lo), ubyte_f<2>(lo), ubyte_f<3>(lo)};
        const float qh[4] = {ubyte_f<0>(hi), ubyte_f<1>(hi), ubyte_f<2>(hi), ubyte_f<3>(hi)};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float wa = __builtin_fmaf(da, ql[t], -oa);
            acc = acc + wa * x[64 * G + 4 * m + t];
            const float wb = __builtin_fmaf(db, qh[t], -ob);
            acc = acc + wb * x[64 * G + 32 + 4 * m + t];
        }
    }
    return acc;
}

// The batched reference (kernels.c:1017-1039: dequant_block, then a plain
// sequential dot) walks the same weights in natural order: the 32 low-nibble
// weights of sub-block 2g, then the 32 high-nibble weights of 2g+1.
template <int G>
MYNAH_DEV float q4k_group_seq(const uint32_t *q, float d, float dmin, uint32_t s0, uint32_t s1,
                              uint32_t s2, const float *__restrict__ x, float acc) {
#pragma clang fp contract(off)
    float sa, ma, sb, mb;
    q4k_sm<2 * G>(s0, s1, s2, sa, ma);
    q4k_sm<2 * G + 1>(s0, s1, s2, sb, mb);
    const float da = d * sa, db = d * sb, oa = dmin * ma, ob = dmin * mb;
#pragma unroll
    for (int half = 0; half < 2; half++) {
        const float dd = half ? db : da, oo = half ? ob : oa;
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const uint32_t v = q[8 * G + m];
            const uint32_t n = half ? ((v >> 4) & 0x0f0f0f0fu) : (v & 0x0f0f0f0fu);
            const float qf[4] = {ubyte_f<0>(n), ubyte_f<1>(n), ubyte_f<2>(n), ubyte_f<3>(n)};
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const float w = __builtin_fmaf(dd, qf[t], -oo);
                acc = acc + w * x[64 * G + 32 * half + 4 * m + t];
            }
        }
    }
    return acc;
}

template <bool SEQ>
MYNAH_DEV float q4k_unit(const uint8_t *__restrict__ blk, const float *__restrict__ x) {
    const uint4 *p = (const uint4 *)blk;
    uint32_t v[36];
#pragma unroll
    for (int k = 0; k < 9; k++) {
        const uint4 c = p[k];
        v[4 * k] = c.x; v[4 * k + 1] = c.y; v[4 * k + 2] = c.z; v[4 * k + 3] = c.w;
    }
    const float d = f16_to_f32(v[0]), dmin = f16_to_f32(v[0] >> 16);
    const uint32_t s0 = v[1], s1 = v[2], s2 = v[3];
    const uint32_t *q = v + 4;
    float acc = 0.0f;
    if (SEQ) {
        acc = q4k_group_seq<0>(q, d, dmin, s0, s1, s2, x, acc);
        acc = q4k_group_seq<1>(q, d, dmin, s0, s1, s2, x, acc);
        acc = q4k_group_seq<2>(q, d, dmin, s0, s1, s2, x, acc);
        acc = q4k_group_seq<3>(q, d, dmin, s0, s1, s2, x, acc);
    } else {
        acc = q4k_group<0>(q, d, dmin, s0, s1, s2, x, acc);
        acc = q4k_group<1>(q, d, dmin, s0, s1, s2, x, acc);
        acc = q4k_group<2>(q, d, dmin, s0, s1, s2, x, acc);
        acc = q4k_group<3>(q, d, dmin, s0, s1, s2, x, acc);
    }
    return acc;
}

// ── Q6_K: 210-byte block, 2-byte aligned ───────────────────────────────────
// Read as the 53 aligned dwords that hold it; realigned dword k (block bytes
// 4k..4k+3) = alignbyte(raw[k+1], raw[k], s) with s = block address & 3.
// d (bytes 208..209) sits in raw[52] at byte s.

MYNAH_DEV float q6k_unit(const uint8_t *__restrict__ blk, const float *__restrict__ x) {
#pragma clang fp contract(off)
    const uint32_t s = (uint32_t)(uintptr_t)blk & 3u;
    const uint32_t *a = (const uint32_t *)(blk - s);
    uint32_t raw[53];
#pragma unroll
    for (int k = 0; k < 53; k++) raw[k] = a[k];
    uint32_t v[52];
#pragma unroll
    for (int k = 0; k < 52; k++) v[k] = align_bytes(raw[k + 1], raw[k], s);
    const float d = f16_to_f32(raw[52] >> (8u * s));
    float dsc[16], n32[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        dsc[j] = d * (float)(int)(int8_t)(v[48 + j / 4] >> (8 * (j % 4)));
        n32[j] = -32.0f * dsc[j];
    }
    float acc = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int k = 0; k < 4; k++)
#pragma unroll
            for (int m = 0; m < 8; m++) {
                const uint32_t ql = v[16 * h + 8 * (k & 1) + m];
                const uint32_t qh = v[32 + 8 * h + m];
                const uint32_t nib = (k < 2) ? (ql & 0x0f0f0f0fu) : ((ql >> 4) & 0x0f0f0f0fu);
                const uint32_t q6 = nib | (((qh >> (2 * k)) & 0x03030303u) << 4);
                const int j = 8 * h + 2 * k + (m >= 4 ? 1 : 0);
                const float qf[4] = {ubyte_f<0>(q6), ubyte_f<1>(q6), ubyte_f<2>(q6), ubyte_f<3>(q6)};
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const float w = __builtin_fmaf(dsc[j], qf[t], n32[j]);
                    acc = acc + w * x[128 * h + 32 * k + 4 * m + t];
                }
            }
    return acc;
}

// ── Q8_0: 34-byte block, 2-byte aligned ────────────────────────────────────

MYNAH_DEV float q80_block(const uint8_t *__restrict__ blk, const float *__restrict__ x,
                          float acc) {
#pragma clang fp contract(off)
    const uint32_t s = (uint32_t)(uintptr_t)blk & 3u;
    const uint32_t *a = (const uint32_t *)(blk - s);
    uint32_t raw[9];
#pragma unroll
    for (int k = 0; k < 9; k++) raw[k] = a[k];
    const float d = f16_to_f32(s ? (raw[0] >> 16) : raw[0]);
    const float n128 = -128.0f * d;
#pragma unroll
    for (int m = 0; m < 8; m++) {
        const uint32_t q = (s ? raw[m + 1] : align_bytes(raw[m + 1], raw[m], 2u)) ^ 0x80808080u;
        const float qf[4] = {ubyte_f<0>(q), ubyte_f<1>(q), ubyte_f<2>(q), ubyte_f<3>(q)};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float w = __builtin_fmaf(d, qf[t], n128);
            acc = acc + w * x[4 * m + t];
        }
    }
    return acc;
}

// ── driver ─────────────────────────────────────────────────────────────────
// SEQ selects the batched reference's order (kernels.c:1053-1104): natural
// weight order within a Q4_K block, and Q8_0 summed in 256-value units of
// eight blocks (kernels.c:2635-2648). Q6_K is the same in both.

template <int FMT, bool SEQ>
MYNAH_DEV float unit_sum(const uint8_t *__restrict__ row, uint32_t u, const float *__restrict__ x) {
    if (FMT == 12) return q4k_unit<SEQ>(row + 144u * u, x + 256u * u);
    if (FMT == 14) return q6k_unit(row + 210u * u, x + 256u * u);
    if (!SEQ) return q80_block(row + 34u * u, x + 32u * u, 0.0f);
    float acc = 0.0f;
#pragma unroll
    for (int b = 0; b < 8; b++) acc = q80_block(row + 272u * u + 34u * b, x + 256u * u + 32u * b, acc);
    return acc;
}

template <int FMT, bool SEQ>
MYNAH_DEV void gemv_exact(const uint8_t *__restrict__ w, const float *__restrict__ x,
                          float *__restrict__ y, uint32_t rows, uint32_t units, uint32_t row_bytes) {
#pragma clang fp contract(off)
    __shared__ float part[EX_MAX_WAVES][EX_ROWS];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nw = __builtin_amdgcn_readfirstlane(blockDim.x >> 6);
    const uint32_t row = blockIdx.x * EX_ROWS + lane;
    const uint8_t *wr = w + (size_t)(row < rows ? row : rows - 1u) * row_bytes;
    float total = 0.0f;
    for (uint32_t p = 0; p < units; p += nw) {
        const uint32_t u = p + wave;
        float s = 0.0f;
        if (u < units) s = unit_sum<FMT, SEQ>(wr, u, x);
        part[wave][lane] = s;
        __syncthreads();
        if (wave == 0) {
            const uint32_t n = units - p < nw ? units - p : nw;
            for (uint32_t k = 0; k < n; k++) total = total + part[k][lane];
        }
        __syncthreads();
    }
    if (wave == 0 && row < rows) y[row] = total;
}

#define GEMV_EXACT_ENTRY(name, FMT, SEQ)                                                   \
    extern "C" __global__ void __launch_bounds__(EX_ROWS * EX_MAX_WAVES)                  \
        name(const uint8_t *__restrict__ w, const float *__restrict__ x,                  \
             float *__restrict__ y, uint32_t rows, uint32_t units, uint32_t row_bytes) {  \
        gemv_exact<FMT, SEQ>(w, x, y, rows, units, row_bytes);                             \
    }

GEMV_EXACT_ENTRY(mynah_q4k_gemv_exact, 12, false)
GEMV_EXACT_ENTRY(mynah_q6k_gemv_exact, 14, false)
GEMV_EXACT_ENTRY(mynah_q80_gemv_exact, 8, false)
GEMV_EXACT_ENTRY(mynah_q4k_gemv_exact_seq, 12, true)
GEMV_EXACT_ENTRY(mynah_q80_gemv_exact_seq, 8, true)


// ── grouped launches with fused epilogues (the resident decode step) ───────
// One launch covers up to EX_GROUP_MAX matrices; workgroup t serves the
// 64-row tile t - tile0 of the descriptor whose [tile0, next tile0) range
// holds t. Epilogues, each the reference's own f32 operation on the exact
// row sum: y = res + Wx (src/arch_qwen3.c:224, 234 — mynah_slm_add), and for
// a paired matrix w2 (ffn_up next to ffn_gate) y = (g * sigmoid(g)) * u with
// the reference's overflow-safe sigmoid (src/kernels.c:193-205). `ypos`
// moves y by ypos[0] * ystride: the K / V projections write straight into
// the cache slot of the current position (src/arch_qwen3.c:194-199).

#define EX_GROUP_MAX 8

struct GemvDesc {
    const uint8_t *w;
    const uint8_t *w2;
    const float *x;
    float *y;
    const float *res;
    const uint32_t *ypos;
    const float *norm_w;
    unsigned long long *keys;    // per-workgroup argmax keys of the rows (head)
    uint32_t ystride, rows, units, row_bytes, type, tile0, cols;
    float eps;
    uint32_t pad;
};

struct GemvGroup {
    uint32_t n, pad;
    GemvDesc d[EX_GROUP_MAX];
};

MYNAH_DEV float sigmoid_ref(float v) {
#pragma clang fp contract(off)
    if (v >= 0.0f) return 1.0f / (1.0f + expf(-v));
    const float e = expf(v);
    return e / (1.0f + e);
}

template <int FMT>
MYNAH_DEV float unit_any(const GemvDesc &g, const uint8_t *r1, const uint8_t *r2, uint32_t u,
                         const float *__restrict__ x) {
    if (u < g.units) return unit_sum<FMT, false>(r1, u, x);
    return unit_sum<FMT, false>(r2, u - g.units, x);
}

template <bool NORM>
MYNAH_DEV void group_body(const GemvDesc &g, uint32_t t, const float *__restrict__ x) {
#pragma clang fp contract(off)
    __shared__ float part[EX_MAX_WAVES][EX_ROWS];
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nw = __builtin_amdgcn_readfirstlane(blockDim.x >> 6);
    const uint32_t row = (t - g.tile0) * EX_ROWS + lane;
    const size_t roff = (size_t)(row < g.rows ? row : g.rows - 1u) * g.row_bytes;
    const uint8_t *r1 = g.w + roff;
    const uint8_t *r2 = g.w2 ? g.w2 + roff : r1;
    const uint32_t total_units = g.w2 ? 2u * g.units : g.units;
    float t1 = 0.0f, t2 = 0.0f;
    for (uint32_t p = 0; p < total_units; p += nw) {
        const uint32_t u = p + wave;
        float s = 0.0f;
        if (u < total_units) {
            if (g.type == 12u) s = unit_any<12>(g, r1, r2, u, x);
            else if (g.type == 14u) s = unit_any<14>(g, r1, r2, u, x);
            else s = unit_any<8>(g, r1, r2, u, x);
        }
        part[wave][lane] = s;
        __syncthreads();
        if (wave == 0) {
            const uint32_t n = total_units - p < nw ? total_units - p : nw;
            for (uint32_t k = 0; k < n; k++) {
                if (p + k < g.units) t1 = t1 + part[k][lane];
                else t2 = t2 + part[k][lane];
            }
        }
        __syncthreads();
    }
    if (wave == 0) {
        float v = t1;
        if (g.w2) v = t1 * sigmoid_ref(t1) * t2;
        else if (g.res && row < g.rows) v = g.res[row] + t1;
        if (row < g.rows) {
            float *y = g.y + (g.ypos ? (size_t)g.ypos[0] * g.ystride : 0);
            y[row] = v;
        }
        if (g.keys) {
            const unsigned long long k = wave_max_u64(row < g.rows ? argmax_key(v, row) : 0ull);
            if (lane == 0) g.keys[t - g.tile0] = k;
        }
    }
}

// With norm_w set, the input is RMSNorm(x) * norm_w (src/kernels.c:118-128:
// double sum of squares, s = (float)(1 / sqrt(sum / n + eps)), (x * s) * w),
// computed by every workgroup into LDS before its GEMV; this replaces the
// reference's separate rms_norm call feeding the projections
// (src/arch_qwen3.c:201, 226, 239). Dynamic LDS: cols floats.
extern "C" __global__ void __launch_bounds__(EX_ROWS * EX_MAX_WAVES)
mynah_gemv_group(const GemvGroup grp) {
#pragma clang fp contract(off)
    extern __shared__ float hx[];
    __shared__ double shd[EX_MAX_WAVES];
    const uint32_t t = blockIdx.x;
    uint32_t i = 0;
    while (i + 1 < grp.n && t >= grp.d[i + 1].tile0) i++;
    const GemvDesc &g = grp.d[i];
    if (g.norm_w == nullptr) {
        group_body<false>(g, t, g.x);
        return;
    }
    double acc = 0.0;
    for (uint32_t k = threadIdx.x; k < g.cols; k += blockDim.x) acc += (double)g.x[k] * (double)g.x[k];
    const double sum = block_sum_d(acc, shd);
    const float s = (float)(1.0 / sqrt(sum / (double)g.cols + (double)g.eps));
    for (uint32_t k = threadIdx.x; k < g.cols; k += blockDim.x) hx[k] = g.x[k] * s * g.norm_w[k];
    __syncthreads();
    group_body<true>(g, t, hx);
}
