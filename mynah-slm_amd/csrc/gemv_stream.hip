// gemv_stream.hip — the exact GEMV for large matrices with long rows (the
// 151936 x 2560 head of Qwen3-4B, the big Q4_K projections): a persistent
// stream over the super-blocks, bit-identical to the reference like the
// grouped kernel of gemv_exact.hip.
//
// Layout. The launch is sized to the resident capacity (four 4-wave
// workgroups per CU, 107 VGPRs). Each workgroup owns a contiguous, balanced
// range of rows, stages x once, and its waves walk that range's
// super-blocks in rounds of 64 (lane = one super-block, consecutive lanes =
// consecutive blocks in memory); wave w takes every fourth round from round
// (w + workgroup) % 4, so the extra rounds of ragged ranges fall on
// different SIMDs. With long rows a workgroup's range is many rounds deep,
// which the one-unit-per-lane grouped kernel cannot exploit: measured on
// MI355X, 151936 x 2560 Q6_K 81.5 -> 67.5 us, 32768 x 2560 Q4_K 20.3 ->
// 17.4 us; on the 151936 x 1024 head (four super-blocks per row) the
// grouped kernel stays ahead (31.3 against 33-34 us), so the runtime sends
// only rows of eight or more super-blocks here.
//
// Order of operations (the reference's, as in gemv_exact.hip): a lane sums
// its super-block in the as-built order (Q4_K kernels.c:94-115, 319-337;
// Q6_K kernels.c:2096-2124, 2176-2199), the unit sums land in LDS, and one
// thread per row folds them in unit order: total = ((s0 + s1) + s2) + ...
//
// Two forms of the weight value, both bit-identical. The reference's
// weight is exact in f32 before its one rounding (Q4_K (d*sc)*q - dmin*m,
// Q6_K (d*sc)*(q-32)), so any single-rounding form of it gives the same
// bits. MIX = false (the default): v_cvt_f32_ubyte of the code, then an fma.
// MIX = true (MYNAH_GEMV_MIX=1): v_fma_mix_f32 reads one operand as an f16
// half of a register; with a code q alone in the low bits of a half, that
// half is the f16 subnormal q * 2^-24 (exact), so fma_mix(D * 2^24, half,
// C) = round(D * q + C) and the convert folds into the fma (a code at bits
// 4..7 of a half is 16q * 2^-24, paired with D * 2^20; f16 subnormals are
// preserved in the kernels' FP16 denorm mode). It issues fewer
// instructions, but v_fma_mix_f32 runs at the rate of v_cvt_f32_ubyte on
// gfx950 (~1.85 ns per wave64 instruction against ~1.05 ns for an f32 add,
// mul or fma), and measured it is no faster.
//
// SPDX-License-Identifier: MIT
#include "common.hip.h"

#define ST_WAVES 4
// Resident waves per SIMD the kernel is compiled for (register budget
// 512 / ST_OCC VGPRs).
#ifndef ST_OCC
#define ST_OCC 4
#endif

// Scheduling windows: a compiler barrier every ST_WIN inner iterations keeps
// the x reads (LDS) and weight decodes of a whole block from being hoisted
// ahead of the running sum (hundreds of live registers); inside a window
// the compiler interleaves loads, decodes, products and the sum freely.
#ifndef ST_WIN
#define ST_WIN 1
#endif
#define ST_WINDOW(i)                                                              \
    do {                                                                          \
        if (ST_WIN > 0 && ((i) + 1) % (ST_WIN > 0 ? ST_WIN : 1) == 0)               \
            asm volatile("" ::: "memory");                                        \
    } while (0)

#define TWO24 16777216.0f
#define TWO20 1048576.0f

// fma(a, f16 low / high half of b, c): with packed FP32 off the compiler
// selects v_fma_mix_f32 (the f16 operand read from the register half).
MYNAH_DEV float f16_lo(uint32_t b) { return f16_to_f32(b); }
MYNAH_DEV float f16_hi(uint32_t b) { return f16_to_f32(b >> 16); }

// Q4_K group G (sub-blocks 2G, 2G + 1) in the matvec order: for byte i of
// the group's 32, the low-nibble weight 64G + i, then the high-nibble
// weight 64G + 32 + i.
template <int G, bool MIX>
MYNAH_DEV float q4k_group_st(const uint32_t *q, float d, float dmin, uint32_t s0, uint32_t s1,
                             uint32_t s2, const float *x, float acc) {
#pragma clang fp contract(off)
    float sa, ma, sb, mb;
    q4k_sm<2 * G>(s0, s1, s2, sa, ma);
    q4k_sm<2 * G + 1>(s0, s1, s2, sb, mb);
    const float na = -(dmin * ma), nb = -(dmin * mb);
    if (MIX) {
        const float da = (d * sa) * TWO24, db = (d * sb) * TWO20;
#pragma unroll
        for (int m = 0; m < 8; m++) {
            const uint32_t v = q[8 * G + m];
            // halves: a = low nibbles of bytes 0 | 2, b = high nibbles (x16)
            // of bytes 0 | 2; c, e the same for bytes 1 | 3.
            const uint32_t a = v & 0x000f000fu, b = v & 0x00f000f0u;
            const uint32_t v8 = v >> 8;
            const uint32_t c = v8 & 0x000f000fu, e = v8 & 0x00f000f0u;
            const float4 xa = *(const float4 *)(x + 64 * G + 4 * m);
            const float4 xb = *(const float4 *)(x + 64 * G + 32 + 4 * m);
            acc = acc + __builtin_fmaf(da, f16_lo(a), na) * xa.x;
            acc = acc + __builtin_fmaf(db, f16_lo(b), nb) * xb.x;
            acc = acc + __builtin_fmaf(da, f16_lo(c), na) * xa.y;
            acc = acc + __builtin_fmaf(db, f16_lo(e), nb) * xb.y;
            acc = acc + __builtin_fmaf(da, f16_hi(a), na) * xa.z;
            acc = acc + __builtin_fmaf(db, f16_hi(b), nb) * xb.z;
            acc = acc + __builtin_fmaf(da, f16_hi(c), na) * xa.w;
            acc = acc + __builtin_fmaf(db, f16_hi(e), nb) * xb.w;
            ST_WINDOW(m);
        }
        return acc;
    }
    return q4k_group<G>(q, d, dmin, s0, s1, s2, x, acc);
}

template <bool MIX>
MYNAH_DEV float q4k_sum_st(const uint32_t *v, const float *x) {
    const float d = f16_to_f32(v[0]), dmin = f16_to_f32(v[0] >> 16);
    const uint32_t s0 = v[1], s1 = v[2], s2 = v[3];
    const uint32_t *q = v + 4;
    float acc = 0.0f;
    acc = q4k_group_st<0, MIX>(q, d, dmin, s0, s1, s2, x, acc);
    acc = q4k_group_st<1, MIX>(q, d, dmin, s0, s1, s2, x, acc);
    acc = q4k_group_st<2, MIX>(q, d, dmin, s0, s1, s2, x, acc);
    acc = q4k_group_st<3, MIX>(q, d, dmin, s0, s1, s2, x, acc);
    return acc;
}

// Q6_K in the reference's order (weights 0..255). Per qh dword H and its
// ql dword L, the 6-bit codes of four weights are assembled per byte; MIX
// splits them into the halves of two registers (bytes 0 | 2 and 1 | 3),
// one v_perm each.
template <bool MIX>
MYNAH_DEV float q6k_sum_st(const uint32_t *raw, uint32_t s, const float *x) {
#pragma clang fp contract(off)
    if (!MIX) return q6k_sum(raw, s, x);
    const float d = f16_to_f32(raw[52] >> (8u * s));
    float acc = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int k = 0; k < 4; k++)
#pragma unroll
            for (int hm = 0; hm < 2; hm++) {
                // sub-block j = 8h + 2k + hm: weights 128h + 32k + 16hm .. + 15
                const int j = 8 * h + 2 * k + hm;
                const uint32_t scw = align_bytes(raw[48 + j / 4 + 1], raw[48 + j / 4], s);
                const float dsc = d * (float)(int)(int8_t)(scw >> (8 * (j % 4)));
                const float n32 = -32.0f * dsc;
                const float dm = dsc * TWO24;
#pragma unroll
                for (int mm = 0; mm < 4; mm++) {
                    const int m = 4 * hm + mm;
                    const int li = 16 * h + 8 * (k & 1) + m, hi = 32 + 8 * h + m;
                    const uint32_t ql = align_bytes(raw[li + 1], raw[li], s);
                    const uint32_t qh = align_bytes(raw[hi + 1], raw[hi], s);
                    const uint32_t nib = (k < 2) ? (ql & 0x0f0f0f0fu) : ((ql >> 4) & 0x0f0f0f0fu);
                    const uint32_t hb = (2 * k <= 4) ? ((qh << (4 - 2 * k)) & 0x30303030u)
                                                     : ((qh >> (2 * k - 4)) & 0x30303030u);
                    const uint32_t q6 = nib | hb;
                    const uint32_t e = __builtin_amdgcn_perm(q6, q6, 0x0c020c00u);
                    const uint32_t o = __builtin_amdgcn_perm(q6, q6, 0x0c030c01u);
                    const float4 x4 = *(const float4 *)(x + 128 * h + 32 * k + 4 * m);
                    acc = acc + __builtin_fmaf(dm, f16_lo(e), n32) * x4.x;
                    acc = acc + __builtin_fmaf(dm, f16_lo(o), n32) * x4.y;
                    acc = acc + __builtin_fmaf(dm, f16_hi(e), n32) * x4.z;
                    acc = acc + __builtin_fmaf(dm, f16_hi(o), n32) * x4.w;
                    ST_WINDOW(mm);
                }
            }
    return acc;
}

template <int FMT, bool MIX> struct StreamBlock;
template <bool MIX> struct StreamBlock<12, MIX> {
    static constexpr uint32_t BYTES = 144;
    uint32_t v[36];
    __device__ __forceinline__ void load(const uint8_t *b) { q4k_load(b, v); }
    __device__ __forceinline__ float sum(const float *x) const {
        return q4k_sum_st<MIX>(v, x);
    }
};
template <bool MIX> struct StreamBlock<14, MIX> {
    static constexpr uint32_t BYTES = 210;
    uint32_t raw[53], s;
    __device__ __forceinline__ void load(const uint8_t *b) { q6k_load(b, raw, s); }
    __device__ __forceinline__ float sum(const float *x) const {
        return q6k_sum_st<MIX>(raw, s, x);
    }
};

// Host mirror: mynah_stream_desc (runtime_internal.h).
struct StreamDesc {
    const uint8_t *w;
    const float *x;
    float *y;
    const float *norm_w;
    unsigned long long *keys;   // one argmax key per workgroup when set
    uint32_t rows, units, row_bytes, type, cols;
    float eps;
};

template <int FMT, bool MIX>
MYNAH_DEV void stream_body(const StreamDesc &g, float *lds, double *shd) {
#pragma clang fp contract(off)
    typedef StreamBlock<FMT, MIX> Blk;
    constexpr uint32_t UB = Blk::BYTES;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nw = blockDim.x >> 6;
    const uint32_t r0 = (uint32_t)((uint64_t)blockIdx.x * g.rows / gridDim.x);
    const uint32_t r1 = (uint32_t)((uint64_t)(blockIdx.x + 1u) * g.rows / gridDim.x);
    if (r1 == r0) return;                                    // whole workgroup
    const uint32_t U = g.units, nf = (r1 - r0) * U, last = nf - 1u;
    const uint8_t *wb = g.w + (size_t)r0 * g.row_bytes;     // rows are U whole blocks
    const uint32_t cols = g.cols, xp = xpad_floats(cols);
    // nf unit sums, then a spare slot: lanes past the end store there, so
    // the sum is not computed under a branch (the compiler would sink it
    // out of its scheduling windows).
    float *part = lds + xp;
    const uint32_t stride = 64u * nw;

    // Round rb (a wave-uniform block index, a multiple of 64) covers blocks
    // rb + lane of the workgroup's range; lanes past the end reload the
    // last block and store nothing. Wave w takes every nw-th round from
    // round (w + workgroup) % nw, so the extra rounds of ragged ranges fall
    // on different SIMDs in different workgroups.
    uint32_t rb = 64u * ((wave + blockIdx.x) % nw);
    Blk a;
    {
        const uint32_t f = rb + lane;
        a.load(wb + (size_t)(f < nf ? f : last) * UB);
    }

    stage_x(g.x, g.norm_w, cols, g.eps, lds, part + ((nf + 4u) & ~3u), shd);
    __syncthreads();

    while (true) {
        const uint32_t f = rb + lane;
        const float sv = a.sum(lds + 260u * (f % U));
        part[f < nf ? f : nf] = sv;     // slot nf: a spare
        rb += stride;
        if (rb >= nf) break;
        const uint32_t fn = rb + lane;
        a.load(wb + (size_t)(fn < nf ? fn : last) * UB);
    }
    __syncthreads();

    // Fold each row's unit sums in unit order; argmax key per workgroup.
    unsigned long long key = 0ull;
    for (uint32_t r = tid; r < r1 - r0; r += blockDim.x) {
        const float *pr = part + r * U;
        float t = 0.0f;
        for (uint32_t q = 0; q < U; q++) t = t + pr[q];
        g.y[r0 + r] = t;
        if (g.keys) {
            const unsigned long long k = argmax_key(t, r0 + r);
            key = k > key ? k : key;
        }
    }
    if (g.keys) {
        __shared__ unsigned long long wk[16];
        key = wave_max_u64(key);
        if (lane == 0) wk[wave] = key;
        __syncthreads();
        if (tid == 0) {
            for (uint32_t k = 1; k < nw; k++) key = wk[k] > key ? wk[k] : key;
            g.keys[blockIdx.x] = key;
        }
    }
}

// Grid: one workgroup per row range (gridDim.x ranges, balanced to a row);
// blockDim.x = 64 * ST_WAVES. Dynamic LDS (floats): xpad_floats(cols) for
// x, then the range's unit sums (max rows per range * units, plus a spare
// slot, rounded up to 4), then cols for the norm weights when norm_w is set.
#define STREAM_ENTRY(name, MIX)                                                     \
    extern "C" __global__ void __launch_bounds__(64 * ST_WAVES, ST_OCC) name(const StreamDesc g) { \
        extern __shared__ __attribute__((aligned(16))) float lds[];                \
        __shared__ double shd[16];                                                   \
        if (g.type == 12u) stream_body<12, MIX>(g, lds, shd);                        \
        else stream_body<14, MIX>(g, lds, shd);                                      \
    }

STREAM_ENTRY(mynah_gemv_stream, true)
STREAM_ENTRY(mynah_gemv_stream_cvt, false)
