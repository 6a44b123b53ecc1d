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
//   Q5_K  kernels.c:1785-1810 and 1835-1853: Q4_K's order and weight form,
//         with 16 added to the quant when its bit of qh[i] is set (bit 2g for
//         the low nibble, 2g+1 for the high one).
//   Q6_K  kernels.c:2096-2124 + 2176-2199 + 2037-2041: decode the 256 values
//         (d*sc)*(q-32), sequential dot from weight 0, row sum in order.
//   Q8_0  kernels.c:2518-2546: values q*d, sequential dot per 32-block, row
//         sum in order.
// Every weight value is exact in f32 before its final rounding, so a single
// fused multiply-add produces the identical value: (d*sc)*q - dmin*m (q up
// to 31 for Q5_K: 11 + 6 + 5 significant bits) as
// fma(d*sc, q, -dmin*m); (d*sc)*(q-32) as fma(d*sc, q6, -32*d*sc) with q6 the
// raw 6-bit code; q*d as fma(d, q + 128, -128*d) with q + 128 = q ^ 0x80. The
// product with x and the sum stay separate roundings, as in the reference.
//
// No product is ever fused with a sum here: the library is compiled with
// -ffp-contract=off and every summing function repeats it as a pragma.
//
// Decomposition (grouped launch, mynah_gemv_group): a "unit" is one
// super-block (Q4_K, Q6_K) or one 32-value block (Q8_0). Lane l of a wave
// serves row l / K and unit slot l % K (K = 1..16 slots per row); WS waves
// share the same rows and split the units, WR such row groups make a
// workgroup. Each lane computes whole unit sums (the unit order inside a
// unit is the reference's), stores them in LDS, and one thread per row folds
// the unit sums in unit order. The input x is staged once per workgroup in
// LDS, 256-value chunks padded by 4 floats so the K slots of a wave read
// different banks.
//
// SPDX-License-Identifier: MIT
#include "common.hip.h"

#define EX_ROWS 64
#define EX_MAX_WAVES 16

// ── Q4_K: 144-byte block, 16-byte aligned ──────────────────────────────────

template <int J>
MYNAH_DEV void q4k_sm(uint32_t s0, uint32_t s1, uint32_t s2, float &sc, float &m) {
    if constexpr (J < 4) {
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
    // The high nibbles stay in place (16 q): (db / 16) (16 q) - ob is the
    // same real number as db q - ob, and db / 16 is exact, so one fma still
    // gives the reference's rounding, without a shift per word.
    const float da = d * sa, db = d * sb * 0.0625f, oa = dmin * ma, ob = dmin * mb;
#pragma unroll
    for (int m = 0; m < 8; m++) {
        const uint32_t v = q[8 * G + m];
        const uint32_t lo = v & 0x0f0f0f0fu, hi = v & 0xf0f0f0f0u;
        const float ql[4] = {ubyte_f<0>(lo), ubyte_f<1>(lo), ubyte_f<2>(lo), ubyte_f<3>(lo)};
        const float qh[4] = {ubyte_f<0>(hi), ubyte_f<1>(hi), ubyte_f<2>(hi), ubyte_f<3>(hi)};
        const float4 xa4 = *(const float4 *)(x + 64 * G + 4 * m);
        const float4 xb4 = *(const float4 *)(x + 64 * G + 32 + 4 * m);
        const float xa[4] = {xa4.x, xa4.y, xa4.z, xa4.w}, xb[4] = {xb4.x, xb4.y, xb4.z, xb4.w};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float wa = __builtin_fmaf(da, ql[t], -oa);
            acc = acc + wa * xa[t];
            const float wb = __builtin_fmaf(db, qh[t], -ob);
            acc = acc + wb * xb[t];
        }
    }
    return acc;
}

// Raw block words in registers, loaded apart from the arithmetic so the
// grouped kernel can issue a block's loads before it stages x.
MYNAH_DEV float q4k_sum(const uint32_t *v, const float *__restrict__ x) {
    const float d = f16_to_f32(v[0]), dmin = f16_to_f32(v[0] >> 16);
    const uint32_t s0 = v[1], s1 = v[2], s2 = v[3];
    const uint32_t *q = v + 4;
    float acc = 0.0f;
    acc = q4k_group<0>(q, d, dmin, s0, s1, s2, x, acc);
    acc = q4k_group<1>(q, d, dmin, s0, s1, s2, x, acc);
    acc = q4k_group<2>(q, d, dmin, s0, s1, s2, x, acc);
    acc = q4k_group<3>(q, d, dmin, s0, s1, s2, x, acc);
    return acc;
}

MYNAH_DEV void q4k_load(const uint8_t *__restrict__ blk, uint32_t *v) {
    const uint4 *p = (const uint4 *)blk;
#pragma unroll
    for (int k = 0; k < 9; k++) {
        const uint4 c = p[k];
        v[4 * k] = c.x; v[4 * k + 1] = c.y; v[4 * k + 2] = c.z; v[4 * k + 3] = c.w;
    }
}

// ── Q5_K: 176-byte block, 16-byte aligned ──────────────────────────────────
// d, dmin @0, scales[12] @4 (Q4_K's packing), qh[32] @16, qs[128] @48. In
// registers: v[0] = d | dmin << 16, v[1..3] scales, v[4..11] qh, v[12..43] qs.

// The 5-bit quants of qs word m of group G: byte i of qh word m holds the
// fifth bits of weights 4m + i, bit 2G (low nibble) and 2G + 1 (high).
template <int G>
MYNAH_DEV void q5k_quants(uint32_t v, uint32_t hb, uint32_t &lo, uint32_t &hi) {
    lo = (v & 0x0f0f0f0fu) | (((hb >> (2 * G)) & 0x01010101u) << 4);
    hi = ((v >> 4) & 0x0f0f0f0fu) | (((hb >> (2 * G + 1)) & 0x01010101u) << 4);
}

template <int G>
MYNAH_DEV float q5k_group(const uint32_t *q, const uint32_t *qh, float d, float dmin,
                          uint32_t s0, uint32_t s1, uint32_t s2, const float *__restrict__ x,
                          float acc) {
#pragma clang fp contract(off)
    float sa, ma, sb, mb;
    q4k_sm<2 * G>(s0, s1, s2, sa, ma);
    q4k_sm<2 * G + 1>(s0, s1, s2, sb, mb);
    const float da = d * sa, db = d * sb, oa = dmin * ma, ob = dmin * mb;
#pragma unroll
    for (int m = 0; m < 8; m++) {
        uint32_t lo, hi;
        q5k_quants<G>(q[8 * G + m], qh[m], lo, hi);
        const float ql[4] = {ubyte_f<0>(lo), ubyte_f<1>(lo), ubyte_f<2>(lo), ubyte_f<3>(lo)};
        const float qu[4] = {ubyte_f<0>(hi), ubyte_f<1>(hi), ubyte_f<2>(hi), ubyte_f<3>(hi)};
        const float4 xa4 = *(const float4 *)(x + 64 * G + 4 * m);
        const float4 xb4 = *(const float4 *)(x + 64 * G + 32 + 4 * m);
        const float xa[4] = {xa4.x, xa4.y, xa4.z, xa4.w}, xb[4] = {xb4.x, xb4.y, xb4.z, xb4.w};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float wa = __builtin_fmaf(da, ql[t], -oa);
            acc = acc + wa * xa[t];
            const float wb = __builtin_fmaf(db, qu[t], -ob);
            acc = acc + wb * xb[t];
        }
    }
    return acc;
}

MYNAH_DEV float q5k_sum(const uint32_t *v, const float *__restrict__ x) {
    const float d = f16_to_f32(v[0]), dmin = f16_to_f32(v[0] >> 16);
    const uint32_t s0 = v[1], s1 = v[2], s2 = v[3];
    const uint32_t *qh = v + 4, *q = v + 12;
    float acc = 0.0f;
    acc = q5k_group<0>(q, qh, d, dmin, s0, s1, s2, x, acc);
    acc = q5k_group<1>(q, qh, d, dmin, s0, s1, s2, x, acc);
    acc = q5k_group<2>(q, qh, d, dmin, s0, s1, s2, x, acc);
    acc = q5k_group<3>(q, qh, d, dmin, s0, s1, s2, x, acc);
    return acc;
}

MYNAH_DEV void q5k_load(const uint8_t *__restrict__ blk, uint32_t *v) {
    const uint4 *p = (const uint4 *)blk;
#pragma unroll
    for (int k = 0; k < 11; k++) {
        const uint4 c = p[k];
        v[4 * k] = c.x; v[4 * k + 1] = c.y; v[4 * k + 2] = c.z; v[4 * k + 3] = c.w;
    }
}

// ── Q6_K: 210-byte block, 2-byte aligned ───────────────────────────────────
// Read as the 53 aligned dwords that hold it; realigned dword k (block bytes
// 4k..4k+3) = alignbyte(raw[k+1], raw[k], s) with s = block address & 3.
// d (bytes 208..209) sits in raw[52] at byte s.

// Wide loads from 4-byte aligned addresses: the amdhsa ABI runs kernels in
// unaligned-access mode, so the compiler turns these copies into dwordx4
// loads (13 + 1 instructions instead of 53).
MYNAH_DEV void q6k_load(const uint8_t *__restrict__ blk, uint32_t *raw, uint32_t &s) {
    s = (uint32_t)(uintptr_t)blk & 3u;
    const uint32_t *a = (const uint32_t *)(blk - s);
    __builtin_memcpy(raw, a, 52 * sizeof(uint32_t));
    raw[52] = a[52];
}

MYNAH_DEV float q6k_sum(const uint32_t *raw, uint32_t s, const float *__restrict__ x) {
#pragma clang fp contract(off)
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
                const float4 x4 = *(const float4 *)(x + 128 * h + 32 * k + 4 * m);
                const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const float w = __builtin_fmaf(dsc[j], qf[t], n32[j]);
                    acc = acc + w * xv[t];
                }
            }
    return acc;
}

// The same sum with each block word realigned where it is used (no second
// copy of the block): fewer live registers, so the Q6_K-only entry below
// fits five waves per SIMD. Same operations in the same order.
MYNAH_DEV float q6k_sum_lean(const uint32_t *raw, uint32_t s, const float *__restrict__ x) {
#pragma clang fp contract(off)
    const float d = f16_to_f32(raw[52] >> (8u * s));
    float acc = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int k = 0; k < 4; k++) {
            // scales 8h + 2k and 8h + 2k + 1: bytes 2 (k & 1), + 1 of word 48 + 2h + k / 2
            const uint32_t scw = align_bytes(raw[48 + 2 * h + k / 2 + 1], raw[48 + 2 * h + k / 2], s);
            const float ds0 = d * (float)(int)(int8_t)(scw >> (16 * (k & 1)));
            const float ds1 = d * (float)(int)(int8_t)(scw >> (16 * (k & 1) + 8));
            const float n0 = -32.0f * ds0, n1 = -32.0f * ds1;
#pragma unroll
            for (int m = 0; m < 8; m++) {
                const int iq = 16 * h + 8 * (k & 1) + m, ih = 32 + 8 * h + m;
                const uint32_t ql = align_bytes(raw[iq + 1], raw[iq], s);
                const uint32_t qh = align_bytes(raw[ih + 1], raw[ih], s);
                const uint32_t nib = (k < 2) ? (ql & 0x0f0f0f0fu) : ((ql >> 4) & 0x0f0f0f0fu);
                const uint32_t q6 = nib | (((qh >> (2 * k)) & 0x03030303u) << 4);
                const float dsc = m >= 4 ? ds1 : ds0, n32 = m >= 4 ? n1 : n0;
                const float qf[4] = {ubyte_f<0>(q6), ubyte_f<1>(q6), ubyte_f<2>(q6), ubyte_f<3>(q6)};
                const float4 x4 = *(const float4 *)(x + 128 * h + 32 * k + 4 * m);
                const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const float w = __builtin_fmaf(dsc, qf[t], n32);
                    acc = acc + w * xv[t];
                }
            }
        }
    return acc;
}

// ── Q8_0: 34-byte block, 2-byte aligned ────────────────────────────────────

MYNAH_DEV void q80_load(const uint8_t *__restrict__ blk, uint32_t *raw, uint32_t &s) {
    s = (uint32_t)(uintptr_t)blk & 3u;
    const uint32_t *a = (const uint32_t *)(blk - s);
    __builtin_memcpy(raw, a, 8 * sizeof(uint32_t));
    raw[8] = a[8];
}

MYNAH_DEV float q80_sum(const uint32_t *raw, uint32_t s, const float *__restrict__ x, float acc) {
#pragma clang fp contract(off)
    const float d = f16_to_f32(s ? (raw[0] >> 16) : raw[0]);
    const float n128 = -128.0f * d;
#pragma unroll
    for (int m = 0; m < 8; m++) {
        const uint32_t q = (s ? raw[m + 1] : align_bytes(raw[m + 1], raw[m], 2u)) ^ 0x80808080u;
        const float qf[4] = {ubyte_f<0>(q), ubyte_f<1>(q), ubyte_f<2>(q), ubyte_f<3>(q)};
        const float4 x4 = *(const float4 *)(x + 4 * m);
        const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float w = __builtin_fmaf(d, qf[t], n128);
            acc = acc + w * xv[t];
        }
    }
    return acc;
}

// ── Q4_0: 18-byte block, 2-byte aligned; one running sum per row ───────────
// kernels.c:2353-2360 values (d * (q - 8)) times x, each product rounded,
// added to the row's single running sum (kernels.c:2467-2484): the low
// nibbles (weights 0..15), then the high nibbles (16..31). `acc` carries the
// sum in from the previous block.
struct RawQ40 {
    uint32_t raw[5], s;
    __device__ __forceinline__ void load(const uint8_t *b) {
        s = (uint32_t)(uintptr_t)b & 3u;
        const uint32_t *a = (const uint32_t *)(b - s);
        // At skew 0 dword 4 holds the last two quant bytes and two bytes past
        // the block, inside the same aligned dword.
#pragma unroll
        for (int k = 0; k < 5; k++) raw[k] = a[k];
    }
    __device__ __forceinline__ float chain(const float *__restrict__ x, float acc) const {
#pragma clang fp contract(off)
        const float d = f16_to_f32(s ? (raw[0] >> 16) : raw[0]);
        uint32_t q[4];
#pragma unroll
        for (int j = 0; j < 4; j++) q[j] = s ? raw[j + 1] : align_bytes(raw[j + 1], raw[j], 2u);
#pragma unroll
        for (int hf = 0; hf < 2; hf++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t nib = hf ? ((q[j] >> 4) & 0x0f0f0f0fu) : (q[j] & 0x0f0f0f0fu);
                const float4 x4 = *(const float4 *)(x + 16 * hf + 4 * j);
                acc = acc + (d * (ubyte_f<0>(nib) - 8.0f)) * x4.x;
                acc = acc + (d * (ubyte_f<1>(nib) - 8.0f)) * x4.y;
                acc = acc + (d * (ubyte_f<2>(nib) - 8.0f)) * x4.z;
                acc = acc + (d * (ubyte_f<3>(nib) - 8.0f)) * x4.w;
            }
        return acc;
    }
};

// ── grouped matvec with fused epilogues (every matvec, decode included) ────
// One launch covers up to EX_GROUP_MAX matrices; workgroup t serves the
// row tile t - tile0 of the descriptor whose [tile0, next tile0) range
// holds t. Epilogues, each the reference's own f32 operation on the exact
// row sum: y = res + Wx (src/arch_qwen3.c:224, 234 — mynah_slm_add), and for
// a paired matrix w2 (ffn_up next to ffn_gate) y = (g * sigmoid(g)) * u with
// the reference's overflow-safe sigmoid (src/kernels.c:193-205). `ypos`
// moves y by ypos[0] * ystride: the K / V projections write straight into
// the cache slot of the current position (src/arch_qwen3.c:194-199).
// With norm_w set, the input is RMSNorm(x) * norm_w (src/kernels.c:118-128:
// double sum of squares, s = (float)(1 / sqrt(sum / n + eps)), (x * s) * w),
// computed by every workgroup while it stages x; this replaces the
// reference's separate rms_norm call feeding the projections
// (src/arch_qwen3.c:201, 226, 239).
//
// grp.shape = log2(K) | WS << 8 | WR << 16 | SPLIT << 24, with (64 / K) * WR
// (SPLIT: (16 / K) * WR) rows per workgroup and 64 * WS * WR threads; SPLIT
// (super-block types only) shares each super-block among the four lanes of a
// quad. Dynamic LDS (floats): the padded x,
// (units | 1) unit sums per row of the workgroup, and with norm_w a copy of
// the norm weights (cols).

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

// L2 prefetch of the next launch's weights. A launch carrying one runs
// pf.wgs extra workgroups after its own pf.host_tiles; each touches one byte
// per 2^pf.step_log2 bytes of the weight tiles that the next launch's
// workgroups on the same XCD will read, so those lines are in that XCD's L2
// when the next launch starts. Workgroups go to XCDs round-robin by linear
// index (workgroup b on XCD b mod 8) in every launch, so prefetch workgroup b
// serves the next launch's tiles t with t = b (mod 8). Segment s: tiles
// t0[s] .. t0[s] + nt[s] - 1, tile t reading bytes [(t - t0) * bpt,
// min((t - t0 + 1) * bpt, bytes)) of base[s]. pf.wgs is a multiple of 8.
#define PF_SEGS 4
struct GemvPrefetch {
    const uint8_t *base[PF_SEGS];
    uint32_t t0[PF_SEGS], nt[PF_SEGS], bpt[PF_SEGS], bytes[PF_SEGS];
    uint32_t n, wgs, host_tiles, step_log2;
};

struct GemvGroup {
    uint32_t n, shape;
    GemvDesc d[EX_GROUP_MAX];
    GemvPrefetch pf;
};

// Where the prefetched bytes end up: stored only when the touched bytes sum
// to one 32-bit value, so the loads stay in the program.
__device__ uint32_t mynah_pf_sink[64];

// True for a prefetch workgroup (which then has done its loads): the caller
// returns. Every address read lies inside a segment.
MYNAH_DEV bool gemv_prefetch_tail(const GemvPrefetch &pf) {
    const uint32_t b = blockIdx.x;
    if (b < pf.host_tiles) return false;
    const uint32_t xcd = b & 7u;
    const uint32_t per = pf.wgs >> 3, j = (b - pf.host_tiles) >> 3;
    const uint32_t sl = pf.step_log2;
    uint32_t acc = 0;
    for (uint32_t s = 0; s < pf.n; s++) {
        const uint32_t t0 = pf.t0[s], end = pf.t0[s] + pf.nt[s];
        const uint32_t first = t0 + ((xcd - t0) & 7u);
        if (first >= end) continue;
        const uint32_t cnt = (end - first + 7u) >> 3;
        for (uint32_t k = j; k < cnt; k += per) {
            const uint32_t t = first + 8u * k;
            const uint64_t lo = (uint64_t)(t - t0) * pf.bpt[s];
            const uint64_t hi = min(lo + pf.bpt[s], (uint64_t)pf.bytes[s]);
            const uintptr_t s0 = (uintptr_t)pf.base[s] + lo, s1 = (uintptr_t)pf.base[s] + hi - 1u;
#pragma unroll 4
            for (uintptr_t l = (s0 >> sl) + threadIdx.x; l <= (s1 >> sl); l += blockDim.x) {
                uintptr_t a = l << sl;
                if (a < s0) a = s0;
                acc += *(const uint8_t *)a;
            }
        }
    }
    if (acc == 0x9e3779b9u) mynah_pf_sink[b & 63u] = acc;
    return true;
}

MYNAH_DEV float sigmoid_ref(float v) {
#pragma clang fp contract(off)
    if (v >= 0.0f) return 1.0f / (1.0f + mynah_expf(-v));
    const float e = mynah_expf(v);
    return e / (1.0f + e);
}

MYNAH_DEV uint32_t xpad_floats(uint32_t cols) { return cols + 4u * ((cols + 255u) >> 8); }

// Stage x (or RMSNorm(x) * norm_w, src/kernels.c:118-128: double sum of
// squares, s = (float)(1 / sqrt(sum / n + eps)), (x * s) * w) into the
// padded LDS copy lds[0 .. xpad_floats(cols)); x[i] sits at
// lds[i + 4 * (i / 256)]. lw (cols floats of LDS) holds the norm weights
// while they are applied. All x and norm-weight loads are issued before the
// first wait. Every thread of the workgroup calls it (it has barriers when
// norm_w is set); the caller synchronises before reading the copy. The sum
// of squares is the workgroup's parallel-order sum, without the index-order
// check of the standalone norm kernels (sum_settled): these kernels hold
// the first unit's weights in registers across the staging, and either
// half of the check (the test or the index-order loop) pushes the Q6_K
// grouped kernels into spills. Its f32 scale differs from the reference's
// only when the scale lies within the two orders' rounding distance of an
// f32 midpoint: by a rounding estimate about once in 10^7 sums, and in none
// of the tests' sums (every test of the decoder compares whole logits
// vectors bit for bit).
MYNAH_DEV void stage_x(const float *__restrict__ x, const float *__restrict__ norm_w,
                       uint32_t cols, float eps, float *lds, float *lw, double *shd) {
#pragma clang fp contract(off)
    const uint32_t tid = threadIdx.x, n4 = cols / 4u;
    const float4 *x4 = (const float4 *)x;
    if (norm_w) {
        const float4 *w4 = (const float4 *)norm_w;
        double acc = 0.0;
#pragma unroll 4
        for (uint32_t q = tid; q < n4; q += blockDim.x) {
            const float4 v = x4[q], w = w4[q];
            *(float4 *)(lds + 4u * q + 4u * (q >> 6)) = v;
            *(float4 *)(lw + 4u * q) = w;
            // A float's square is exact in double, so one fma rounds
            // exactly as the reference's multiply-then-add.
            acc = __builtin_fma((double)v.x, (double)v.x, acc);
            acc = __builtin_fma((double)v.y, (double)v.y, acc);
            acc = __builtin_fma((double)v.z, (double)v.z, acc);
            acc = __builtin_fma((double)v.w, (double)v.w, acc);
        }
        const double sum = block_sum_d(acc, shd);
        const float sc = (float)(1.0 / sqrt(sum / (double)cols + (double)eps));
        for (uint32_t q = tid; q < n4; q += blockDim.x) {
            float4 *px = (float4 *)(lds + 4u * q + 4u * (q >> 6));
            float4 v = *px;
            const float4 w = *(const float4 *)(lw + 4u * q);
            v.x = v.x * sc * w.x; v.y = v.y * sc * w.y; v.z = v.z * sc * w.z; v.w = v.w * sc * w.w;
            *px = v;
        }
    } else {
#pragma unroll 4
        for (uint32_t q = tid; q < n4; q += blockDim.x)
            *(float4 *)(lds + 4u * q + 4u * (q >> 6)) = x4[q];
    }
}


template <int FMT> struct Raw;
template <> struct Raw<12> {
    static constexpr uint32_t BYTES = 144;
    uint32_t v[36];
    __device__ __forceinline__ void load(const uint8_t *b) { q4k_load(b, v); }
    __device__ __forceinline__ float sum(const float *x) const { return q4k_sum(v, x); }
};
template <> struct Raw<13> {
    static constexpr uint32_t BYTES = 176;
    uint32_t v[44];
    __device__ __forceinline__ void load(const uint8_t *b) { q5k_load(b, v); }
    __device__ __forceinline__ float sum(const float *x) const { return q5k_sum(v, x); }
};
template <> struct Raw<14> {
    static constexpr uint32_t BYTES = 210;
    uint32_t raw[53], s;
    __device__ __forceinline__ void load(const uint8_t *b) { q6k_load(b, raw, s); }
    __device__ __forceinline__ float sum(const float *x) const { return q6k_sum(raw, s, x); }
};
struct RawQ6Lean {
    static constexpr uint32_t BYTES = 210;
    uint32_t raw[53], s;
    __device__ __forceinline__ void load(const uint8_t *b) { q6k_load(b, raw, s); }
    __device__ __forceinline__ float sum(const float *x) const { return q6k_sum_lean(raw, s, x); }
};
template <> struct Raw<8> {
    static constexpr uint32_t BYTES = 34;
    uint32_t raw[9], s;
    __device__ __forceinline__ void load(const uint8_t *b) { q80_load(b, raw, s); }
    __device__ __forceinline__ float sum(const float *x) const { return q80_sum(raw, s, x, 0.0f); }
};

// ── split super-blocks (small launches) ────────────────────────────────────
// A decode-sized launch leaves most SIMDs idle, and one lane summing a whole
// super-block issues ~1,100 VALU instructions in a row. In split mode four
// lanes (a quad) share a super-block: lane s computes the 64 products of
// segment s (weights 64 s .. 64 s + 63, in the reference's order) in
// parallel, then the running sum is handed along the quad — segment 0 from
// 0.0f, segment s from segment s - 1's total — so the sum is still the
// reference's single chain over the 256 products, in its order.

// (scale, min) of Q4_K sub-block j (runtime j), kernels.c:83-92.
MYNAH_DEV void q4k_sm_rt(uint32_t s0, uint32_t s1, uint32_t s2, uint32_t j, float &sc, float &m) {
    const uint32_t jl = 8u * (j & 3u);
    const uint32_t a = (s0 >> jl) & 63u, b = (s1 >> jl) & 63u;
    const uint32_t c = ((s2 >> jl) & 15u) | (((s0 >> (jl + 6u)) & 3u) << 4);
    const uint32_t e = ((s2 >> (jl + 4u)) & 15u) | (((s1 >> (jl + 6u)) & 3u) << 4);
    sc = (float)(j < 4u ? a : c);
    m = (float)(j < 4u ? b : e);
}

template <int FMT> struct RawSeg;
// Q4_K segment g = group g: the header and the 32 quant bytes of the group.
template <> struct RawSeg<12> {
    uint4 hdr, q0, q1;
    __device__ __forceinline__ void load(const uint8_t *b, uint32_t g) {
        hdr = *(const uint4 *)b;
        const uint4 *p = (const uint4 *)(b + 16u + 32u * g);
        q0 = p[0];
        q1 = p[1];
    }
    __device__ __forceinline__ void products(const float *x, uint32_t g, float *p) const {
#pragma clang fp contract(off)
        const float d = f16_to_f32(hdr.x), dmin = f16_to_f32(hdr.x >> 16);
        float sa, ma, sb, mb;
        q4k_sm_rt(hdr.y, hdr.z, hdr.w, 2u * g, sa, ma);
        q4k_sm_rt(hdr.y, hdr.z, hdr.w, 2u * g + 1u, sb, mb);
        // High nibbles in place, scale / 16 (exact), as in q4k_group.
        const float da = d * sa, db = d * sb * 0.0625f, oa = dmin * ma, ob = dmin * mb;
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const uint32_t lo = q[m] & 0x0f0f0f0fu, hi = q[m] & 0xf0f0f0f0u;
            const float ql[4] = {ubyte_f<0>(lo), ubyte_f<1>(lo), ubyte_f<2>(lo), ubyte_f<3>(lo)};
            const float qh[4] = {ubyte_f<0>(hi), ubyte_f<1>(hi), ubyte_f<2>(hi), ubyte_f<3>(hi)};
            const float4 xa4 = *(const float4 *)(x + 4 * m);
            const float4 xb4 = *(const float4 *)(x + 32 + 4 * m);
            const float xa[4] = {xa4.x, xa4.y, xa4.z, xa4.w}, xb[4] = {xb4.x, xb4.y, xb4.z, xb4.w};
#pragma unroll
            for (int t = 0; t < 4; t++) {
                p[8 * m + 2 * t] = __builtin_fmaf(da, ql[t], -oa) * xa[t];
                p[8 * m + 2 * t + 1] = __builtin_fmaf(db, qh[t], -ob) * xb[t];
            }
        }
    }
};
// Q5_K segment g = group g: the header, all of qh and the 32 quant bytes of
// the group.
template <> struct RawSeg<13> {
    uint4 hdr, h0, h1, q0, q1;
    __device__ __forceinline__ void load(const uint8_t *b, uint32_t g) {
        const uint4 *p = (const uint4 *)b;
        hdr = p[0];
        h0 = p[1];
        h1 = p[2];
        q0 = p[3 + 2u * g];
        q1 = p[4 + 2u * g];
    }
    __device__ __forceinline__ void products(const float *x, uint32_t g, float *p) const {
#pragma clang fp contract(off)
        const float d = f16_to_f32(hdr.x), dmin = f16_to_f32(hdr.x >> 16);
        float sa, ma, sb, mb;
        q4k_sm_rt(hdr.y, hdr.z, hdr.w, 2u * g, sa, ma);
        q4k_sm_rt(hdr.y, hdr.z, hdr.w, 2u * g + 1u, sb, mb);
        const float da = d * sa, db = d * sb, oa = dmin * ma, ob = dmin * mb;
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const uint32_t qh[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const uint32_t lo = (q[m] & 0x0f0f0f0fu) | (((qh[m] >> (2u * g)) & 0x01010101u) << 4);
            const uint32_t hi =
                ((q[m] >> 4) & 0x0f0f0f0fu) | (((qh[m] >> (2u * g + 1u)) & 0x01010101u) << 4);
            const float ql[4] = {ubyte_f<0>(lo), ubyte_f<1>(lo), ubyte_f<2>(lo), ubyte_f<3>(lo)};
            const float qu[4] = {ubyte_f<0>(hi), ubyte_f<1>(hi), ubyte_f<2>(hi), ubyte_f<3>(hi)};
            const float4 xa4 = *(const float4 *)(x + 4 * m);
            const float4 xb4 = *(const float4 *)(x + 32 + 4 * m);
            const float xa[4] = {xa4.x, xa4.y, xa4.z, xa4.w}, xb[4] = {xb4.x, xb4.y, xb4.z, xb4.w};
#pragma unroll
            for (int t = 0; t < 4; t++) {
                p[8 * m + 2 * t] = __builtin_fmaf(da, ql[t], -oa) * xa[t];
                p[8 * m + 2 * t + 1] = __builtin_fmaf(db, qu[t], -ob) * xb[t];
            }
        }
    }
};
// Q6_K segment s = (h, half) = (s >> 1, s & 1): weights 128 h + 32 k + 4 m + t
// for k = 2 half, 2 half + 1; realigned words 16 h .. 16 h + 15 (ql),
// 32 + 8 h .. + 7 (qh), 48 + 2 h + half (four scales) and d.
template <> struct RawSeg<14> {
    uint32_t ql[17], qh[9], sc[2], dw, s;
    __device__ __forceinline__ void load(const uint8_t *b, uint32_t seg) {
        s = (uint32_t)(uintptr_t)b & 3u;
        const uint32_t *a = (const uint32_t *)(b - s);
        const uint32_t h = seg >> 1, half = seg & 1u;
        __builtin_memcpy(ql, a + 16u * h, 16 * sizeof(uint32_t));
        ql[16] = a[16u * h + 16u];
        __builtin_memcpy(qh, a + 32u + 8u * h, 8 * sizeof(uint32_t));
        qh[8] = a[40u + 8u * h];
        __builtin_memcpy(sc, a + 48u + 2u * h + half, 2 * sizeof(uint32_t));
        dw = a[52];
    }
    __device__ __forceinline__ void products(const float *x, uint32_t seg, float *p) const {
#pragma clang fp contract(off)
        const uint32_t half = seg & 1u;
        const float d = f16_to_f32(dw >> (8u * s));
        const uint32_t scw = align_bytes(sc[1], sc[0], s);
        float dsc[4], n32[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            dsc[j] = d * (float)(int)(int8_t)(scw >> (8 * j));
            n32[j] = -32.0f * dsc[j];
        }
#pragma unroll
        for (int kk = 0; kk < 2; kk++)
#pragma unroll
            for (int m = 0; m < 8; m++) {
                const uint32_t lw = align_bytes(ql[8 * kk + m + 1], ql[8 * kk + m], s);
                const uint32_t hw = align_bytes(qh[m + 1], qh[m], s);
                const uint32_t nib = (half ? (lw >> 4) : lw) & 0x0f0f0f0fu;
                const uint32_t q6 = nib | (((hw >> (4u * half + 2u * kk)) & 0x03030303u) << 4);
                const int j = 2 * kk + (m >= 4 ? 1 : 0);
                const float qf[4] = {ubyte_f<0>(q6), ubyte_f<1>(q6), ubyte_f<2>(q6), ubyte_f<3>(q6)};
                const float4 x4 = *(const float4 *)(x + 32 * kk + 4 * m);
                const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
                for (int t = 0; t < 4; t++)
                    p[32 * kk + 4 * m + t] = __builtin_fmaf(dsc[j], qf[t], n32[j]) * xv[t];
            }
    }
};
template <> struct RawSeg<8> {   // never launched: split mode is for super-block types only
    __device__ __forceinline__ void load(const uint8_t *, uint32_t) {}
    __device__ __forceinline__ void products(const float *, uint32_t, float *p) const {
#pragma unroll
        for (int i = 0; i < 64; i++) p[i] = 0.0f;
    }
};

// The quad's running sum: step k extends the total handed over by lane
// k - 1 of the quad (0.0f at step 0) with this lane's 64 products; lane k
// keeps step k's result. Returns the unit sum on lane 3.
MYNAH_DEV float quad_chain(const float *p, uint32_t seg) {
#pragma clang fp contract(off)
    float carry = 0.0f, res = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < 4u; k++) {
        float t = carry;
#pragma unroll
        for (int i = 0; i < 64; i++) t = t + p[i];
        res = seg == k ? t : res;
        // quad_perm(0, 0, 1, 2): lane i of the quad receives lane i - 1's t.
        carry = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(t), 0x90, 0xf, 0xf, false));
    }
    return res;
}

// x position of unit u in the padded LDS copy.
template <int FMT>
MYNAH_DEV const float *unit_x(const float *lx, uint32_t u) {
    if (FMT == 8) return lx + 260u * (u >> 3) + 32u * (u & 7u);
    return lx + 260u * u;
}

template <int FMT, bool SEG, class RawT = Raw<FMT>>
MYNAH_DEV void group_split(const GemvDesc &g, uint32_t t, uint32_t shape, float *lds, double *shd) {
#pragma clang fp contract(off)
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
    const uint32_t lk = shape & 31u, ws_n = (shape >> 8) & 31u, wr_n = (shape >> 16) & 31u;
    // SEG: lane = 4 * (unit lane) + segment; 16 unit lanes per wave.
    const uint32_t ul = SEG ? lane >> 2 : lane, seg = lane & 3u;
    const uint32_t k = 1u << lk, rpw = (SEG ? 16u : 64u) >> lk, rpg = rpw * wr_n;
    const uint32_t wr = wave / ws_n, wsi = wave - wr * ws_n;
    const uint32_t rl = wr * rpw + (ul >> lk), j = ul & (k - 1u);
    const uint32_t row0 = (t - g.tile0) * rpg, row = row0 + rl;
    const size_t roff = (size_t)(row < g.rows ? row : g.rows - 1u) * g.row_bytes;
    const uint8_t *r1 = g.w + roff;
    const uint8_t *r2 = g.w2 ? g.w2 + roff : r1;
    const uint32_t U = g.units, Ut = g.w2 ? 2u * U : U, pstride = Ut | 1u;
    const uint32_t step = k * ws_n;
    constexpr uint32_t UB = RawT::BYTES;
    uint32_t u = j + k * wsi;
    RawT raw;
    RawSeg<FMT> rs;
    if (u < Ut) {
        const uint8_t *b = u < U ? r1 + UB * u : r2 + UB * (u - U);
        if (SEG) rs.load(b, seg);
        else raw.load(b);
    }

    // Prefetch what the epilogue reads (residual row, cache slot).
    const uint32_t frow = row0 + tid;
    const bool folds = tid < rpg && frow < g.rows;
    float resv = 0.0f;
    if (folds && g.res) resv = g.res[frow];
    const uint32_t yoff = g.ypos ? g.ypos[0] * g.ystride : 0u;

    // Stage x (or RMSNorm(x) * norm_w) into the padded LDS copy.
    const uint32_t cols = g.cols;
    stage_x(g.x, g.norm_w, cols, g.eps, lds, lds + xpad_floats(cols) + rpg * pstride, shd);
    __syncthreads();

    float *part = lds + xpad_floats(cols);
    while (u < Ut) {
        const uint32_t uu = u < U ? u : u - U;
        if (SEG) {
            float pr[64];
            rs.products(unit_x<FMT>(lds, uu) + 64u * seg, seg, pr);
            const float r = quad_chain(pr, seg);
            if (seg == 3u) part[rl * pstride + u] = r;
        } else {
            part[rl * pstride + u] = raw.sum(unit_x<FMT>(lds, uu));
        }
        u += step;
        if (u < Ut) {
            const uint8_t *b = u < U ? r1 + UB * u : r2 + UB * (u - U);
            if (SEG) rs.load(b, seg);
            else raw.load(b);
        }
    }
    __syncthreads();

    if (tid < 64u) {
        float t1 = 0.0f, t2 = 0.0f, v = 0.0f;
        if (folds) {
            const float *pr = part + tid * pstride;
            for (uint32_t q = 0; q < U; q++) t1 = t1 + pr[q];
            for (uint32_t q = U; q < Ut; q++) t2 = t2 + pr[q];
            v = t1;
            if (g.w2) v = t1 * sigmoid_ref(t1) * t2;
            else if (g.res) v = resv + t1;
            g.y[yoff + frow] = v;
        }
        if (g.keys) {
            const unsigned long long key = wave_max_u64(folds ? argmax_key(v, frow) : 0ull);
            if (tid == 0) g.keys[t - g.tile0] = key;
        }
    }
}

// Flat layout: the workgroup covers R = g.pad whole rows of its descriptor,
// and thread f (f < R * Ut, stepping by blockDim.x) owns unit u = f % Ut of
// row f / Ut, the units of a gate/up pair counted gate first. Every thread
// that has a unit computes it whole, in the reference's order; the unit sums
// of a row are folded in unit order by one thread (R <= 64: the first wave),
// followed by the epilogues of group_split. Every lane busy but the last
// few of the workgroup, and x staged once per R rows.
template <int FMT, class RawT = Raw<FMT>>
MYNAH_DEV void group_flat(const GemvDesc &g, uint32_t t, float *lds, double *shd) {
#pragma clang fp contract(off)
    const uint32_t tid = threadIdx.x, nthr = blockDim.x;
    const uint32_t R = g.pad;
    const uint32_t U = g.units, Ut = g.w2 ? 2u * U : U, pstride = Ut | 1u;
    const uint32_t row0 = (t - g.tile0) * R, nf = R * Ut;
    constexpr uint32_t UB = RawT::BYTES;
    uint32_t f = tid, rl = f / Ut, u = f - rl * Ut;
    RawT raw;
    auto load = [&]() {
        const uint32_t row = row0 + rl;
        const size_t roff = (size_t)(row < g.rows ? row : g.rows - 1u) * g.row_bytes;
        raw.load(u < U ? g.w + roff + UB * u : g.w2 + roff + UB * (u - U));
    };
    if (f < nf) load();

    // Prefetch what the epilogue reads (residual row, cache slot).
    const uint32_t frow = row0 + tid;
    const bool folds = tid < R && frow < g.rows;
    float resv = 0.0f;
    if (folds && g.res) resv = g.res[frow];
    const uint32_t yoff = g.ypos ? g.ypos[0] * g.ystride : 0u;

    const uint32_t cols = g.cols;
    stage_x(g.x, g.norm_w, cols, g.eps, lds, lds + xpad_floats(cols) + R * pstride, shd);
    __syncthreads();

    float *part = lds + xpad_floats(cols);
    while (f < nf) {
        part[rl * pstride + u] = raw.sum(unit_x<FMT>(lds, u < U ? u : u - U));
        f += nthr;
        if (f < nf) {
            rl = f / Ut;
            u = f - rl * Ut;
            load();
        }
    }
    __syncthreads();

    if (tid < 64u) {
        float t1 = 0.0f, t2 = 0.0f, v = 0.0f;
        if (folds) {
            const float *pr = part + tid * pstride;
            for (uint32_t q = 0; q < U; q++) t1 = t1 + pr[q];
            for (uint32_t q = U; q < Ut; q++) t2 = t2 + pr[q];
            v = t1;
            if (g.w2) v = t1 * sigmoid_ref(t1) * t2;
            else if (g.res) v = resv + t1;
            g.y[yoff + frow] = v;
        }
        if (g.keys) {
            const unsigned long long key = wave_max_u64(folds ? argmax_key(v, frow) : 0ull);
            if (tid == 0) g.keys[t - g.tile0] = key;
        }
    }
}

// Q4_0 rows of a grouped launch. The planner gives a launch holding a Q4_0
// matrix the shape K = 1, WS = 1, WR = 1 (one wave, 64 rows): lane = row,
// whose single running sum goes through every block in order (a gate/up
// pair: one sum per matrix), then the same epilogues as group_split. x is
// staged as for the other types; no unit partials are kept.
MYNAH_DEV void group_chain_q40(const GemvDesc &g, uint32_t t, float *lds, double *shd) {
#pragma clang fp contract(off)
    const uint32_t lane = threadIdx.x;
    const uint32_t row = (t - g.tile0) * 64u + lane;
    const bool live = row < g.rows;
    const size_t roff = (size_t)(live ? row : g.rows - 1u) * g.row_bytes;
    const uint32_t U = g.units;
    const float resv = (live && g.res) ? g.res[row] : 0.0f;
    const uint32_t yoff = g.ypos ? g.ypos[0] * g.ystride : 0u;
    // Blocks go through a register ring of 4-block chunks, each chunk's loads
    // issued a chunk ahead of its sums (one block ahead leaves every block's
    // memory latency exposed; 8-block chunks spill in this entry).
    constexpr uint32_t CH = 4;
    RawQ40 cur[CH];
#pragma unroll
    for (uint32_t k = 0; k < CH; k++)
        if (k < U) cur[k].load(g.w + roff + 18u * k);
    stage_x(g.x, g.norm_w, g.cols, g.eps, lds, lds + xpad_floats(g.cols), shd);
    __syncthreads();
    float t1 = 0.0f, t2 = 0.0f;
    const uint32_t n_mat = g.w2 ? 2u : 1u;
    for (uint32_t m = 0; m < n_mat; m++) {
        const uint8_t *r = (m ? g.w2 : g.w) + roff;
        if (m) {
#pragma unroll
            for (uint32_t k = 0; k < CH; k++)
                if (k < U) cur[k].load(r + 18u * k);
        }
        float acc = 0.0f;
        for (uint32_t c0 = 0; c0 < U; c0 += CH) {
            RawQ40 nxt[CH];
#pragma unroll
            for (uint32_t k = 0; k < CH; k++)
                if (c0 + CH + k < U) nxt[k].load(r + 18u * (c0 + CH + k));
#pragma unroll
            for (uint32_t k = 0; k < CH; k++)
                if (c0 + k < U) acc = cur[k].chain(unit_x<8>(lds, c0 + k), acc);
#pragma unroll
            for (uint32_t k = 0; k < CH; k++) cur[k] = nxt[k];
        }
        if (m) t2 = acc;
        else t1 = acc;
    }
    float v = t1;
    if (g.w2) v = t1 * sigmoid_ref(t1) * t2;
    else if (g.res) v = resv + t1;
    if (live) g.y[yoff + row] = v;
    if (g.keys) {
        const unsigned long long key = wave_max_u64(live ? argmax_key(v, row) : 0ull);
        if (lane == 0) g.keys[t - g.tile0] = key;
    }
}

extern "C" __global__ void __launch_bounds__(1024)
mynah_gemv_group(const GemvGroup grp) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    __shared__ double shd[16];
    if (gemv_prefetch_tail(grp.pf)) return;
    const uint32_t t = blockIdx.x;
    uint32_t i = 0;
    while (i + 1 < grp.n && t >= grp.d[i + 1].tile0) i++;
    const GemvDesc &g = grp.d[i];
    if (grp.shape & (1u << 25)) {
        if (g.type == 12u) group_flat<12>(g, t, lds, shd);
        else if (g.type == 13u) group_flat<13>(g, t, lds, shd);
        else if (g.type == 14u) group_flat<14>(g, t, lds, shd);
        else group_flat<8>(g, t, lds, shd);
    } else if (grp.shape & (1u << 24)) {
        if (g.type == 12u) group_split<12, true>(g, t, grp.shape, lds, shd);
        else if (g.type == 13u) group_split<13, true>(g, t, grp.shape, lds, shd);
        else group_split<14, true>(g, t, grp.shape, lds, shd);
    } else if (g.type == 12u) {
        group_split<12, false>(g, t, grp.shape, lds, shd);
    } else if (g.type == 13u) {
        group_split<13, false>(g, t, grp.shape, lds, shd);
    } else if (g.type == 14u) {
        group_split<14, false>(g, t, grp.shape, lds, shd);
    } else if (g.type == 2u) {
        group_chain_q40(g, t, lds, shd);
    } else {
        group_split<8, false>(g, t, grp.shape, lds, shd);
    }
}

// Launches whose every matrix is Q4_K, in the one-lane-per-super-block
// layout and at most 256 threads per workgroup (the Qwen3-4B projections):
// six waves per SIMD (80 VGPRs, no spills) instead of the general entry's four.
extern "C" __global__ void __launch_bounds__(256, 6)
mynah_gemv_group_q4k(const GemvGroup grp) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    __shared__ double shd[16];
    if (gemv_prefetch_tail(grp.pf)) return;
    const uint32_t t = blockIdx.x;
    uint32_t i = 0;
    while (i + 1 < grp.n && t >= grp.d[i + 1].tile0) i++;
    group_split<12, false>(grp.d[i], t, grp.shape, lds, shd);
}

// Launches whose every matrix is Q6_K, in the one-lane-per-super-block
// layout and at most 256 threads per workgroup (the 0.6B head among them):
// the lean sum at five waves per SIMD instead of four.
extern "C" __global__ void __launch_bounds__(256, 5)
mynah_gemv_group_q6k(const GemvGroup grp) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    __shared__ double shd[16];
    if (gemv_prefetch_tail(grp.pf)) return;
    const uint32_t t = blockIdx.x;
    uint32_t i = 0;
    while (i + 1 < grp.n && t >= grp.d[i + 1].tile0) i++;
    group_split<14, false, RawQ6Lean>(grp.d[i], t, grp.shape, lds, shd);
}

// The flat layout for launches whose every matrix is Q4_K (up to 512
// threads, six waves per SIMD) or Q6_K (the lean sum, five).
extern "C" __global__ void __launch_bounds__(512, 6)
mynah_gemv_flat_q4k(const GemvGroup grp) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    __shared__ double shd[16];
    if (gemv_prefetch_tail(grp.pf)) return;
    const uint32_t t = blockIdx.x;
    uint32_t i = 0;
    while (i + 1 < grp.n && t >= grp.d[i + 1].tile0) i++;
    group_flat<12>(grp.d[i], t, lds, shd);
}

extern "C" __global__ void __launch_bounds__(512, 5)
mynah_gemv_flat_q6k(const GemvGroup grp) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    __shared__ double shd[16];
    if (gemv_prefetch_tail(grp.pf)) return;
    const uint32_t t = blockIdx.x;
    uint32_t i = 0;
    while (i + 1 < grp.n && t >= grp.d[i + 1].tile0) i++;
    group_flat<14, RawQ6Lean>(grp.d[i], t, lds, shd);
}
