// gemv_fast.hip — the reordered (lane-parallel) decode GEMV, grouped, with
// the same fused prologue / epilogues as the exact grouped kernel.
//
// Same weight values as the reference (each decoded exactly), f32 sums in a
// different order: every output differs from the reference only by f32
// rounding (bounded by the recursive-summation bound against an f64 dot).
//
// Workgroup = 4 waves; KS of them (1, 2 or 4, chosen per launch) share a
// tile of 8 rows and split its super-blocks (wave k takes s = k, k + KS,
// ...), so a tile is 32 / KS rows. Lane = (row rg = lane / 8, unit
// u = lane % 8): per 256-weight super-block a lane handles the 32 weights of
// unit u (Q8_0: super-block s holds 32-value blocks 8s .. 8s + 7 and unit u
// takes block 8s + u). The first PRE super-blocks of a lane are loaded before
// x is staged, so the weight fetch overlaps the prologue; the unit partials
// meet in an xor butterfly, the KS wave partials in LDS in a fixed order. x is staged once per
// workgroup in LDS (x[i] at lx[i + 4 * (i / 64)], so the 8 units of a row
// group read distinct banks and the 8 row groups read the same addresses),
// with the sums of each run of 8 values beside it; zero points fold into
// those sums: sum (q - z) x = sum q x - z sum x. A paired matrix (ffn_up
// next to ffn_gate) is computed by the same lane for the SwiGLU epilogue.
//
// SPDX-License-Identifier: MIT
#include "common.hip.h"

#define FG_WG 256
#define FG_ROWS 32

#define FG_PRE 4

// ── raw weight data of one lane for one super-block ───────────────────────

struct RawQ4K { uint4 hdr, q; };
struct RawQ6K { uint32_t a[3], c[3], h[3], s[3], dw, sh; };
struct RawQ80 { uint32_t r[9], sh; bool ok; };

MYNAH_DEV void load(RawQ4K &o, const uint8_t *__restrict__ row, uint32_t s, uint32_t u, uint32_t) {
    const uint8_t *blk = row + 144u * s;
    o.hdr = *(const uint4 *)blk;
    o.q = *(const uint4 *)(blk + 16u + 16u * u);
}

// One dwordx3 load from the 4-byte aligned address at or below p (kernels
// run in unaligned-access mode).
MYNAH_DEV void load3(uint32_t *d, const uint8_t *p) {
    const uint32_t *a = (const uint32_t *)(p - ((uintptr_t)p & 3u));
    __builtin_memcpy(d, a, 3 * sizeof(uint32_t));
}

MYNAH_DEV void load(RawQ6K &o, const uint8_t *__restrict__ row, uint32_t s, uint32_t u, uint32_t) {
    const uint8_t *blk = row + 210u * s;
    const uint32_t h = u >> 2, p = u & 3u;
    o.sh = (uint32_t)(uintptr_t)blk & 3u;   // every field sits at an even offset
    load3(o.a, blk + 64u * h + 8u * p);
    load3(o.c, blk + 64u * h + 32u + 8u * p);
    load3(o.h, blk + 128u + 32u * h + 8u * p);
    load3(o.s, blk + 192u + 8u * h);
    o.dw = *(const uint32_t *)(blk + 208 - o.sh);
}

MYNAH_DEV void load(RawQ80 &o, const uint8_t *__restrict__ row, uint32_t s, uint32_t u,
                    uint32_t nblk) {
    const uint32_t j = 8u * s + u;
    o.ok = j < nblk;
    const uint8_t *blk = row + 34u * (o.ok ? j : 0u);
    o.sh = (uint32_t)(uintptr_t)blk & 3u;
    const uint32_t *a = (const uint32_t *)(blk - o.sh);
    __builtin_memcpy(o.r, a, 8 * sizeof(uint32_t));
    o.r[8] = a[8];
}

// ── one lane's partial over one super-block ───────────────────────────────
// xb / sb: the staged x and run sums of the super-block (x of super-block s at
// lx + 272 s, sums at ls + 32 s).

// Q4_K: unit u = 2g + hh covers qs[32g + 16hh .. +15]; low nibbles are
// weights 64g + 16hh + t (sub-block 2g), high nibbles 64g + 32 + 16hh + t.
MYNAH_DEV float part(const RawQ4K &o, uint32_t u, const float *xb, const float *sb) {
    const uint32_t g = u >> 1, hh = u & 1u;
    const float d = f16_to_f32(o.hdr.x), dmin = f16_to_f32(o.hdr.x >> 16);
    const bool high = g >= 2;
    const uint32_t sh = 16u * (g & 1u);
    float sc[2], mn[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint32_t s0 = o.hdr.y >> (sh + 8 * j), s1 = o.hdr.z >> (sh + 8 * j);
        const uint32_t s2 = o.hdr.w >> (sh + 8 * j);
        sc[j] = (float)(high ? ((s2 & 15u) | ((s0 >> 2) & 48u)) : (s0 & 63u));
        mn[j] = (float)(high ? (((s2 >> 4) & 15u) | ((s1 >> 2) & 48u)) : (s1 & 63u));
    }
    const float *xa = xb + 68u * g + 16u * hh, *xc = xa + 32;
    const uint32_t qv[4] = {o.q.x, o.q.y, o.q.z, o.q.w};
    float da = 0.0f, dc = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float4 va = *(const float4 *)(xa + 4 * k), vc = *(const float4 *)(xc + 4 * k);
        const uint32_t lo = qv[k] & 0x0f0f0f0fu, hi = (qv[k] >> 4) & 0x0f0f0f0fu;
        da = fmaf(ubyte_f<0>(lo), va.x, da); da = fmaf(ubyte_f<1>(lo), va.y, da);
        da = fmaf(ubyte_f<2>(lo), va.z, da); da = fmaf(ubyte_f<3>(lo), va.w, da);
        dc = fmaf(ubyte_f<0>(hi), vc.x, dc); dc = fmaf(ubyte_f<1>(hi), vc.y, dc);
        dc = fmaf(ubyte_f<2>(hi), vc.z, dc); dc = fmaf(ubyte_f<3>(hi), vc.w, dc);
    }
    const uint32_t r = 8u * g + 2u * hh;
    const float sa = sb[r] + sb[r + 1], sc2 = sb[r + 4] + sb[r + 5];
    return fmaf(d * sc[0], da, fmaf(d * sc[1], dc, -dmin * fmaf(mn[0], sa, mn[1] * sc2)));
}

// Q6_K: unit u = 4h + p: for quarter k = 0..3 of half h, weights
// 128h + 32k + 8p + t; low 4 bits from ql[64h + 32(k&1) + 8p + t] (low nibble
// for k < 2), top 2 bits (qh[32h + 8p + t] >> 2k) & 3, scale sc[8h + 2k + p/2],
// value d * sc * (q - 32). Fields are realigned with v_alignbyte.
MYNAH_DEV float part(const RawQ6K &o, uint32_t u, const float *xb, const float *sb) {
    const uint32_t h = u >> 2, p = u & 3u, sh = o.sh;
    const uint32_t av[2] = {align_bytes(o.a[1], o.a[0], sh), align_bytes(o.a[2], o.a[1], sh)};
    const uint32_t cv[2] = {align_bytes(o.c[1], o.c[0], sh), align_bytes(o.c[2], o.c[1], sh)};
    const uint32_t hv[2] = {align_bytes(o.h[1], o.h[0], sh), align_bytes(o.h[2], o.h[1], sh)};
    const uint32_t s0 = align_bytes(o.s[1], o.s[0], sh), s1 = align_bytes(o.s[2], o.s[1], sh);
    const float d = f16_to_f32(o.dw >> (8u * sh));
    const uint32_t shs = 8u * (p >> 1);
    const float sc[4] = {(float)(int)(int8_t)(s0 >> shs), (float)(int)(int8_t)(s0 >> (shs + 16u)),
                         (float)(int)(int8_t)(s1 >> shs), (float)(int)(int8_t)(s1 >> (shs + 16u))};
    float dot[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const uint32_t qk[4] = {
            (av[i] & 0x0f0f0f0fu) | ((hv[i] << 4) & 0x30303030u),
            (cv[i] & 0x0f0f0f0fu) | ((hv[i] << 2) & 0x30303030u),
            ((av[i] >> 4) & 0x0f0f0f0fu) | (hv[i] & 0x30303030u),
            ((cv[i] >> 4) & 0x0f0f0f0fu) | ((hv[i] >> 2) & 0x30303030u)};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float4 v = *(const float4 *)(xb + 136u * h + 32u * k + 4u * (k >> 1) + 8u * p + 4u * i);
            dot[k] = fmaf(ubyte_f<0>(qk[k]), v.x, dot[k]);
            dot[k] = fmaf(ubyte_f<1>(qk[k]), v.y, dot[k]);
            dot[k] = fmaf(ubyte_f<2>(qk[k]), v.z, dot[k]);
            dot[k] = fmaf(ubyte_f<3>(qk[k]), v.w, dot[k]);
        }
    }
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++) acc = fmaf(sc[k], fmaf(-32.0f, sb[16u * h + 4u * k + p], dot[k]), acc);
    return d * acc;
}

// Q8_0: block 8s + u; (q + 128) = q ^ 0x80 as an unsigned byte.
MYNAH_DEV float part(const RawQ80 &o, uint32_t u, const float *xb, const float *sb) {
    if (!o.ok) return 0.0f;
    const float *x = xb + 32u * u + 4u * (u >> 1);
    const float *sm = sb + 4u * u;
    const float d = f16_to_f32(o.sh ? (o.r[0] >> 16) : o.r[0]);
    float dot = 0.0f;
#pragma unroll
    for (int m = 0; m < 8; m++) {
        const uint32_t q = (o.sh ? o.r[m + 1] : align_bytes(o.r[m + 1], o.r[m], 2u)) ^ 0x80808080u;
        const float4 v = *(const float4 *)(x + 4 * m);
        dot = fmaf(ubyte_f<0>(q), v.x, dot);
        dot = fmaf(ubyte_f<1>(q), v.y, dot);
        dot = fmaf(ubyte_f<2>(q), v.z, dot);
        dot = fmaf(ubyte_f<3>(q), v.w, dot);
    }
    const float xs = (sm[0] + sm[1]) + (sm[2] + sm[3]);
    return d * fmaf(-128.0f, xs, dot);
}

// Stage the (optionally RMS-normalised) input into LDS: lx padded, ls[i / 8]
// = sum of x[i .. i + 7]. With norm_w the staged value is the reference's
// (x * s) * w with s = (float)(1 / sqrt(sum x^2 / n + eps)), sum in double.
// x (or RMSNorm(x) * norm_w) into the padded LDS copy plus the 8-value run
// sums; every x and norm-weight load is issued before the first wait (the
// norm weights wait in lw while the sum of squares is reduced).
MYNAH_DEV void fast_stage(const GemvDesc &g, float *lx, float *ls, float *lw, double *shd) {
#pragma clang fp contract(off)
    const uint32_t n4 = g.cols / 4u;
    const float4 *x4 = (const float4 *)g.x;
    if (g.norm_w != nullptr) {
        const float4 *w4 = (const float4 *)g.norm_w;
        double acc = 0.0;
        for (uint32_t q = threadIdx.x; q < n4; q += blockDim.x) {
            const float4 v = x4[q], w = w4[q];
            const uint32_t i = 4u * q;
            *(float4 *)(lx + i + 4u * (i >> 6)) = v;
            *(float4 *)(lw + i) = w;
            // A float's square is exact in double, so one fma rounds
            // exactly as the reference's multiply-then-add.
            acc = __builtin_fma((double)v.x, (double)v.x, acc);
            acc = __builtin_fma((double)v.y, (double)v.y, acc);
            acc = __builtin_fma((double)v.z, (double)v.z, acc);
            acc = __builtin_fma((double)v.w, (double)v.w, acc);
        }
        const double sum = block_sum_d(acc, shd);
        const float s = (float)(1.0 / sqrt(sum / (double)g.cols + (double)g.eps));
        for (uint32_t q = threadIdx.x; q < n4; q += blockDim.x) {
            const uint32_t i = 4u * q;
            float4 *px = (float4 *)(lx + i + 4u * (i >> 6));
            float4 v = *px;
            const float4 w = *(const float4 *)(lw + i);
            v.x = v.x * s * w.x; v.y = v.y * s * w.y; v.z = v.z * s * w.z; v.w = v.w * s * w.w;
            *px = v;
            float r = (v.x + v.y) + (v.z + v.w);
            r += __shfl_xor(r, 1, 64);
            if ((threadIdx.x & 1u) == 0) ls[i / 8u] = r;
        }
    } else {
        for (uint32_t q = threadIdx.x; q < n4; q += blockDim.x) {
            const float4 v = x4[q];
            const uint32_t i = 4u * q;
            *(float4 *)(lx + i + 4u * (i >> 6)) = v;
            float r = (v.x + v.y) + (v.z + v.w);
            r += __shfl_xor(r, 1, 64);
            if ((threadIdx.x & 1u) == 0) ls[i / 8u] = r;
        }
    }
}

// The lane's sum over its super-blocks s = k0, k0 + ks, ... < S of one row;
// the first FG_PRE were loaded into pre[] before the prologue.
template <class Raw>
MYNAH_DEV float lane_sum(const Raw *pre, const uint8_t *__restrict__ row, uint32_t k0, uint32_t ks,
                         uint32_t S, uint32_t u, uint32_t nblk, const float *lx, const float *ls) {
    float acc = 0.0f;
    uint32_t s = k0;
#pragma unroll
    for (int i = 0; i < FG_PRE; i++, s += ks)
        if (s < S) acc += part(pre[i], u, lx + 272u * s, ls + 32u * s);
    for (; s < S; s += ks) {
        Raw r;
        load(r, row, s, u, nblk);
        acc += part(r, u, lx + 272u * s, ls + 32u * s);
    }
    return acc;
}

template <class Raw>
MYNAH_DEV void fast_tile(const GemvDesc &g, uint32_t t, uint32_t ks, float *lx, float *ls,
                         float *lw, double *shd, float (*wp)[2][8]) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t u = lane & 7u, k0 = wave % ks, tile_wave = wave / ks;
    const uint32_t row = (t - g.tile0) * (32u / ks) + 8u * tile_wave + (lane >> 3);
    const size_t roff = (size_t)(row < g.rows ? row : g.rows - 1u) * g.row_bytes;
    const uint32_t S = g.type == 8u ? (g.units + 7u) / 8u : g.units;
    const uint8_t *r1 = g.w + roff, *r2 = g.w2 ? g.w2 + roff : r1;
    Raw p1[FG_PRE], p2[FG_PRE];
    uint32_t s = k0;
#pragma unroll
    for (int i = 0; i < FG_PRE; i++, s += ks) {
        if (s < S) {
            load(p1[i], r1, s, u, g.units);
            if (g.w2) load(p2[i], r2, s, u, g.units);
        }
    }
    const bool folds = k0 == 0 && u == 0 && row < g.rows;
    const float resv = (folds && g.res && !g.w2) ? g.res[row] : 0.0f;
    const size_t yoff = g.ypos ? (size_t)g.ypos[0] * g.ystride : 0u;
    fast_stage(g, lx, ls, lw, shd);
    __syncthreads();
    const float v1 = group8_sum(lane_sum(p1, r1, k0, ks, S, u, g.units, lx, ls));
    const float v2 = g.w2 ? group8_sum(lane_sum(p2, r2, k0, ks, S, u, g.units, lx, ls)) : 0.0f;
    if (u == 0) { wp[wave][0][lane >> 3] = v1; wp[wave][1][lane >> 3] = v2; }
    __syncthreads();
    unsigned long long key = 0ull;
    if (k0 == 0 && u == 0) {
        float a = wp[wave][0][lane >> 3], b = wp[wave][1][lane >> 3];
        for (uint32_t k = 1; k < ks; k++) {
            a += wp[wave + k][0][lane >> 3];
            b += wp[wave + k][1][lane >> 3];
        }
        float v = a;
        if (g.w2) v = a * sigmoid_ref(a) * b;
        else if (g.res) v = resv + a;
        if (row < g.rows) {
            g.y[yoff + row] = v;
            key = argmax_key(v, row);
        }
    }
    if (g.keys) {
        __shared__ unsigned long long wk[4];
        key = wave_max_u64(key);
        if (lane == 0) wk[wave] = key;
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned long long m = wk[0];
            for (int k = 1; k < 4; k++) m = wk[k] > m ? wk[k] : m;
            g.keys[t - g.tile0] = m;
        }
    }
}

// grp.shape carries KS. Dynamic LDS: cols * 17/16 + cols / 8 floats, plus
// cols for the norm weights when norm_w is set.
extern "C" __global__ void __launch_bounds__(FG_WG)
mynah_gemv_fast_group(const GemvGroup grp) {
    extern __shared__ __attribute__((aligned(16))) float lds_f[];
    __shared__ double shd[4];
    __shared__ float wp[4][2][8];
    if (gemv_prefetch_tail(grp.pf)) return;
    const uint32_t t = blockIdx.x;
    uint32_t i = 0;
    while (i + 1 < grp.n && t >= grp.d[i + 1].tile0) i++;
    const GemvDesc &g = grp.d[i];
    float *lx = lds_f;
    float *ls = lds_f + g.cols + g.cols / 16u;
    float *lw = ls + g.cols / 8u;
    const uint32_t ks = grp.shape;
    if (g.type == 12u) fast_tile<RawQ4K>(g, t, ks, lx, ls, lw, shd, wp);
    else if (g.type == 14u) fast_tile<RawQ6K>(g, t, ks, lx, ls, lw, shd, wp);
    else fast_tile<RawQ80>(g, t, ks, lx, ls, lw, shd, wp);
}
