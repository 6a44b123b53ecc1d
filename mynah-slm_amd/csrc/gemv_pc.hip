// gemv_pc.hip — the exact GEMV with the products computed beside the chain,
// for launches too small to fill the chip one super-block per lane.
//
// The reference's order (third_party/ingot/src/kernels.c:94-115, 319-337 for
// Q4_K): each super-block sum starts from 0 and takes its 256 products one at
// a time in a fixed order; the row total takes the super-block sums in order.
// Only the adds are serial. Here a workgroup holds one "adding" wave and four
// "producing" waves. Adding lane f owns super-block f of the workgroup (R
// whole rows x Ut units, f = row * Ut + unit); the four producing lanes
// 4 f .. 4 f + 3 compute its products. A super-block's 256 products are
// made in four stages of 64 (stage s = the reference's group s); producing
// lane q of the quad makes the 16 consecutive products 16 q .. 16 q + 15 of
// the stage, each rounded once as w * x with w = fma(d sc, q, -dmin m) (the
// reference's d sc q - dmin m: d sc q is exact, so the fma rounds once where
// the reference rounds its subtraction), and stores them to an LDS slot.
// The adding lane then adds the stage's 64 products to its running sum in
// order. Stage s is produced while stage s - 1 is added (two slots, one
// barrier per stage), so a launch's critical path is about 256 dependent
// adds per super-block instead of the ~1,100 instructions of one lane doing
// everything. The unit sums are folded in unit order afterwards and the
// epilogues are those of the one-lane kernels (residual, SwiGLU of a
// gate/up pair, KV-cache slot), so every output has the same bits.
//
// SPDX-License-Identifier: MIT
#include "common.hip.h"

#define PC_STRIDE 68u   // floats per super-block in a product slot (64 + 4: no bank conflicts)

// Q4_K: header (d, dmin, 12 scale bytes) and the lane's 8 quant bytes of
// each stage: bytes 16 + 32 s + 8 q .. + 7 hold values 8 q .. 8 q + 7 of
// group s's low nibbles (values 64 s + i) and high nibbles (64 s + 32 + i).
struct PcQ4K {
    static constexpr uint32_t BYTES = 144;
    uint4 hdr;
    uint2 qv[4];
    __device__ __forceinline__ void load(const uint8_t *b, uint32_t q) {
        hdr = *(const uint4 *)b;
#pragma unroll
        for (int s = 0; s < 4; s++) qv[s] = *(const uint2 *)(b + 16u + 32u * (uint32_t)s + 8u * q);
    }
    // Products 16 q .. 16 q + 15 of stage S, in the reference's order
    // (value 64 S + i then 64 S + 32 + i for i = 8 q .. 8 q + 7); xu = the
    // unit's x.
    template <int S>
    __device__ __forceinline__ void products(const float *xu, uint32_t q, float *p) const {
#pragma clang fp contract(off)
        const float d = f16_to_f32(hdr.x), dmin = f16_to_f32(hdr.x >> 16);
        float sa, ma, sb, mb;
        q4k_sm_rt(hdr.y, hdr.z, hdr.w, 2u * S, sa, ma);
        q4k_sm_rt(hdr.y, hdr.z, hdr.w, 2u * S + 1u, sb, mb);
        // High nibbles in place, scale / 16 (exact).
        const float da = d * sa, db = d * sb * 0.0625f, oa = dmin * ma, ob = dmin * mb;
        const float *xa = xu + 64u * S + 8u * q, *xb = xa + 32;
        const float4 a0 = *(const float4 *)xa, a1 = *(const float4 *)(xa + 4);
        const float4 b0 = *(const float4 *)xb, b1 = *(const float4 *)(xb + 4);
        const float xav[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        const float xbv[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
        const uint32_t w2[2] = {qv[S].x, qv[S].y};
#pragma unroll
        for (int m = 0; m < 2; m++) {
            const uint32_t lo = w2[m] & 0x0f0f0f0fu, hi = w2[m] & 0xf0f0f0f0u;
            const float ql[4] = {ubyte_f<0>(lo), ubyte_f<1>(lo), ubyte_f<2>(lo), ubyte_f<3>(lo)};
            const float qh[4] = {ubyte_f<0>(hi), ubyte_f<1>(hi), ubyte_f<2>(hi), ubyte_f<3>(hi)};
#pragma unroll
            for (int t = 0; t < 4; t++) {
                p[8 * m + 2 * t] = __builtin_fmaf(da, ql[t], -oa) * xav[4 * m + t];
                p[8 * m + 2 * t + 1] = __builtin_fmaf(db, qh[t], -ob) * xbv[4 * m + t];
            }
        }
    }
};

template <class Blk>
MYNAH_DEV void group_pc(const GemvDesc &g, uint32_t t, float *lds, double *shd) {
#pragma clang fp contract(off)
    const uint32_t tid = threadIdx.x;
    const bool adder = tid < 64u;
    const uint32_t R = g.pad;
    const uint32_t U = g.units, Ut = g.w2 ? 2u * U : U, pstride = Ut | 1u;
    const uint32_t row0 = (t - g.tile0) * R, nf = R * Ut;
    const uint32_t f = adder ? tid : (tid - 64u) >> 2, q = tid & 3u;
    const bool live = f < nf;
    const uint32_t rl = f / Ut, u = f - rl * Ut;
    const uint32_t uu = u < U ? u : u - U;
    Blk blk;
    if (!adder && live) {
        const uint32_t row = row0 + rl;
        const size_t roff = (size_t)(row < g.rows ? row : g.rows - 1u) * g.row_bytes;
        blk.load((u < U ? g.w : g.w2) + roff + Blk::BYTES * uu, q);
    }

    // Prefetch what the epilogue reads (residual row, cache slot).
    const uint32_t frow = row0 + tid;
    const bool folds = tid < R && frow < g.rows;
    float resv = 0.0f;
    if (folds && g.res) resv = g.res[frow];
    const uint32_t yoff = g.ypos ? g.ypos[0] * g.ystride : 0u;

    const uint32_t cols = g.cols, xf = xpad_floats(cols);
    float *part = lds + xf;
    float *slots = part + ((R * pstride + 3u) & ~3u);
    // The norm weights are staged over the product slots (used only after).
    stage_x(g.x, g.norm_w, cols, g.eps, lds, slots, shd);
    __syncthreads();

    const uint32_t slot_floats = nf * PC_STRIDE;
    const float *xu = lds + 260u * uu;
    float acc = 0.0f;
    float p[16];
#define PC_PRODUCE(S)                                                                     \
    if (!adder && live) {                                                                 \
        blk.template products<S>(xu, q, p);                                               \
        float4 *dst = (float4 *)(slots + ((S) & 1) * slot_floats + f * PC_STRIDE + 16u * q); \
        dst[0] = make_float4(p[0], p[1], p[2], p[3]);                                     \
        dst[1] = make_float4(p[4], p[5], p[6], p[7]);                                     \
        dst[2] = make_float4(p[8], p[9], p[10], p[11]);                                   \
        dst[3] = make_float4(p[12], p[13], p[14], p[15]);                                 \
    }
#define PC_ADD(S)                                                                         \
    if (adder && live) {                                                                  \
        const float4 *src = (const float4 *)(slots + ((S) & 1) * slot_floats + f * PC_STRIDE); \
        _Pragma("unroll") for (int k = 0; k < 16; k++) {                                  \
            const float4 v = src[k];                                                      \
            acc = acc + v.x;                                                              \
            acc = acc + v.y;                                                              \
            acc = acc + v.z;                                                              \
            acc = acc + v.w;                                                              \
        }                                                                                 \
    }
    PC_PRODUCE(0)
    __syncthreads();
    PC_PRODUCE(1)
    PC_ADD(0)
    __syncthreads();
    PC_PRODUCE(2)
    PC_ADD(1)
    __syncthreads();
    PC_PRODUCE(3)
    PC_ADD(2)
    __syncthreads();
    PC_ADD(3)
#undef PC_PRODUCE
#undef PC_ADD
    if (adder && live) part[rl * pstride + u] = acc;
    __syncthreads();

    if (tid < 64u) {
        float t1 = 0.0f, t2 = 0.0f, v = 0.0f;
        if (folds) {
            const float *pr = part + tid * pstride;
            for (uint32_t k = 0; k < U; k++) t1 = t1 + pr[k];
            for (uint32_t k = U; k < Ut; k++) t2 = t2 + pr[k];
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

// Block 320 threads (wave 0 adds, waves 1-4 produce), R = g.pad = 64 / Ut
// rows per workgroup (Ut <= 64); LDS: x (xpad_floats(cols)), R * (Ut | 1)
// unit sums rounded up to 4, then max(2 * R * Ut * 68, norm ? cols : 0)
// floats.
extern "C" __global__ void __launch_bounds__(320)
mynah_gemv_pc_q4k(const GemvGroup grp) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    __shared__ double shd[16];
    if (gemv_prefetch_tail(grp.pf)) return;
    const uint32_t t = blockIdx.x;
    uint32_t i = 0;
    while (i + 1 < grp.n && t >= grp.d[i + 1].tile0) i++;
    group_pc<PcQ4K>(grp.d[i], t, lds, shd);
}
