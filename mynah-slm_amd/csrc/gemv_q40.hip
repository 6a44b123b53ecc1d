// gemv_q40.hip — Q4_0 products bit-identical to the reference.
//
// Q4_0 (third_party/ingot/src/kernels.c:2332-2514): 32 weights in 18 bytes,
// d f16 @0 and qs[16] @2; weight i (i < 16) = d * ((qs[i] & 15) - 8), weight
// 16 + i = d * ((qs[i] >> 4) - 8). Each weight is exact in f32 (11 + 4
// significant bits). The as-built matvec (kernels.c:2467-2484) keeps ONE
// running f32 sum over the whole row — sum += w[i] * x[i], product and sum
// rounded separately, blocks in order, no per-block partials — and the
// batched product has no kernel of its own: ingot_matmat's generic path
// (generic.c:76-93) decodes the row and runs the same chain per token. So
// every output is one serial chain of cols adds that cannot be split or
// reordered without changing its bits.
//
// Layout (batched, and the matvec with MYNAH_Q40_PC=0; the matvec's default
// kernel is mynah_q40_chain_pc below): lane = row (64 rows per one-wave
// workgroup), T tokens per lane as T
// independent chains interleaved (T = 1 for the matvec; 2, 4 or 8 batched,
// the most that still leaves enough waves to fill the chip), grid.y
// over token groups; res (may be NULL or equal y) is added to each finished
// chain, the residual add of the batched prefill. The row is streamed in chunks of 8 blocks (256 values,
// 144 bytes): a chunk's words are loaded one chunk ahead of their use, and
// the matching 256 x values of each token are staged in LDS and read as
// broadcasts. The chains are latency-bound (cols dependent adds each); the
// chunk prefetch keeps the loads off that path.
//
// SPDX-License-Identifier: MIT
#include "common.hip.h"

#define Q40_CHUNK 8u            // blocks per chunk
#define Q40_WORDS 37            // dwords covering a chunk at either 2-byte skew

template <int T>
MYNAH_DEV void q40_chain(const uint8_t *__restrict__ w, const float *__restrict__ x, float *y,
                         uint32_t rows, uint32_t cols, uint32_t tokens, uint32_t row_bytes,
                         const float *res) {
#pragma clang fp contract(off)
    __shared__ float4 xs[T][64];
    const uint32_t lane = threadIdx.x;
    const uint32_t row = blockIdx.x * 64u + lane;
    const uint32_t t0 = blockIdx.y * (uint32_t)T;
    const uint8_t *wr = w + (size_t)(row < rows ? row : rows - 1u) * row_bytes;
    const uint32_t nb = cols / 32u;
    // Row starts are 2-byte aligned: the chunk is read as the aligned dwords
    // that hold it, and realigned by the skew s (0 or 2 bytes).
    const uint32_t s = (uint32_t)(uintptr_t)wr & 3u;
    const uint32_t *wa = (const uint32_t *)(wr - s);

    uint32_t raw[Q40_WORDS];
    float4 xn[T];
    // Loads chunk c's words and x slices; only dwords holding chunk bytes and
    // x values inside the row are read.
    auto fetch = [&](uint32_t b0) {
        const uint32_t n = nb - b0 < Q40_CHUNK ? nb - b0 : Q40_CHUNK;
        const uint32_t *p = wa + (18u * b0) / 4u;
        const uint32_t lim = s + 18u * n;
        if (n == Q40_CHUNK) {
            // Dwords 0..35 hold chunk bytes (or, at skew 2, the two bytes
            // before it in the same dword); dword 36 only at skew 2.
            __builtin_memcpy(raw, p, (Q40_WORDS - 1) * sizeof(uint32_t));
            raw[Q40_WORDS - 1] = s ? p[Q40_WORDS - 1] : 0u;
        } else {
#pragma unroll
            for (int k = 0; k < Q40_WORDS; k++) raw[k] = 4u * (uint32_t)k < lim ? p[k] : 0u;
        }
#pragma unroll
        for (int t = 0; t < T; t++) {
            const uint32_t tt = t0 + (uint32_t)t;
            xn[t] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (tt < tokens && 4u * lane < 32u * n)
                xn[t] = *(const float4 *)(x + (size_t)tt * cols + 32u * b0 + 4u * lane);
        }
    };

    float acc[T];
#pragma unroll
    for (int t = 0; t < T; t++) acc[t] = 0.0f;

    fetch(0);
    for (uint32_t b0 = 0; b0 < nb; b0 += Q40_CHUNK) {
        const uint32_t n = nb - b0 < Q40_CHUNK ? nb - b0 : Q40_CHUNK;
        __syncthreads();                        // the previous chunk's x is consumed
#pragma unroll
        for (int t = 0; t < T; t++) xs[t][lane] = xn[t];
        // Chunk byte 4k .. 4k + 3 as v[k]; 18 * b0 is even, so the chunk keeps
        // the row's skew.
        uint32_t v[Q40_WORDS - 1];
        const uint32_t sh = (s + 18u * b0) & 3u;
#pragma unroll
        for (int k = 0; k < Q40_WORDS - 1; k++) v[k] = align_bytes(raw[k + 1], raw[k], sh);
        if (b0 + Q40_CHUNK < nb) fetch(b0 + Q40_CHUNK);
        __syncthreads();                        // this chunk's x is in LDS
#pragma unroll
        for (int k = 0; k < (int)Q40_CHUNK; k++) {
            if ((uint32_t)k >= n) break;
            // Block k at chunk byte 18k: d, then 16 quant bytes.
            const int o = 18 * k;
            const uint32_t dbits = (o & 3) ? (v[o >> 2] >> 16) : (v[o >> 2] & 0xffffu);
            const float d = f16_to_f32(dbits);
            uint32_t q[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int b = o + 2 + 4 * j;
                q[j] = (b & 3) ? align_bytes(v[(b >> 2) + 1], v[b >> 2], 2u) : v[b >> 2];
            }
#pragma unroll
            for (int hf = 0; hf < 2; hf++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t nib = hf ? ((q[j] >> 4) & 0x0f0f0f0fu) : (q[j] & 0x0f0f0f0fu);
                    const float wv[4] = {d * (ubyte_f<0>(nib) - 8.0f), d * (ubyte_f<1>(nib) - 8.0f),
                                         d * (ubyte_f<2>(nib) - 8.0f), d * (ubyte_f<3>(nib) - 8.0f)};
                    // weights 16 hf + 4 j .. + 3 of the block
#pragma unroll
                    for (int t = 0; t < T; t++) {
                        const float4 x4 = xs[t][8 * k + 4 * hf + j];
                        acc[t] = acc[t] + wv[0] * x4.x;
                        acc[t] = acc[t] + wv[1] * x4.y;
                        acc[t] = acc[t] + wv[2] * x4.z;
                        acc[t] = acc[t] + wv[3] * x4.w;
                    }
                }
        }
    }
    if (row < rows) {
#pragma unroll
        for (int t = 0; t < T; t++)
            if (t0 + (uint32_t)t < tokens) {
                const size_t o = (size_t)(t0 + (uint32_t)t) * rows + row;
                y[o] = res ? res[o] + acc[t] : acc[t];
            }
    }
}

// ── the matvec with the products computed beside the chain ────────────────
// One token: the chain is the whole cost, and a wave that decodes, converts
// and multiplies every weight before adding it issues ~5 instructions per
// weight of its chain. Here wave 0 of a 256-thread workgroup only adds: for
// its 64 rows (lane = row) it reads the products w_i * x_i, four at a time,
// from LDS and extends each row's running sum in the reference's order.
// Waves 1..3 produce them: at step s wave p decodes block 3 s + p - 1 of its
// lane's row and writes its 32 products (the reference's f32 roundings) into
// one of two LDS buffers; one barrier per step hands a buffer over. Each
// producer keeps its next four blocks in flight (a ring of four register
// sets, indexed statically by unrolling the steps by four).
#define QP_AHEAD 4

struct Q40Blk {
    uint32_t raw[5], s;
};

MYNAH_DEV void q40_fetch(Q40Blk &bk, const uint8_t *row, uint32_t b, uint32_t nb) {
    if (b < nb) {
        const uint8_t *p = row + 18u * b;
        bk.s = (uint32_t)(uintptr_t)p & 3u;
        const uint32_t *a = (const uint32_t *)(p - bk.s);
        // 18 block bytes at skew 0 or 2 lie in dwords 0..4 (at skew 0 dword 4
        // holds the last two quant bytes and two bytes past the block).
#pragma unroll
        for (int k = 0; k < 5; k++) bk.raw[k] = a[k];
    }
}

// The 32 products of a block (kernels.c:2353-2360 values times x, one
// rounding each) into quads 8 p .. 8 p + 7 of buffer `dst`.
MYNAH_DEV void q40_products(const Q40Blk &bk, const float *__restrict__ xb, float4 (*dst)[64],
                            uint32_t p, uint32_t lane) {
#pragma clang fp contract(off)
    const float d = f16_to_f32(bk.s ? (bk.raw[0] >> 16) : bk.raw[0]);
    uint32_t q[4];
#pragma unroll
    for (int j = 0; j < 4; j++) q[j] = bk.s ? bk.raw[j + 1] : align_bytes(bk.raw[j + 1], bk.raw[j], 2u);
#pragma unroll
    for (int hf = 0; hf < 2; hf++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t nib = hf ? ((q[j] >> 4) & 0x0f0f0f0fu) : (q[j] & 0x0f0f0f0fu);
            const float4 x4 = *(const float4 *)(xb + 16 * hf + 4 * j);
            float4 pr;
            pr.x = (d * (ubyte_f<0>(nib) - 8.0f)) * x4.x;
            pr.y = (d * (ubyte_f<1>(nib) - 8.0f)) * x4.y;
            pr.z = (d * (ubyte_f<2>(nib) - 8.0f)) * x4.z;
            pr.w = (d * (ubyte_f<3>(nib) - 8.0f)) * x4.w;
            dst[8u * p + 4u * (uint32_t)hf + (uint32_t)j][lane] = pr;
        }
}

extern "C" __global__ void __launch_bounds__(256)
mynah_q40_chain_pc(const uint8_t *__restrict__ w, const float *__restrict__ x,
                   float *__restrict__ y, uint32_t rows, uint32_t cols, uint32_t row_bytes) {
#pragma clang fp contract(off)
    __shared__ float4 pr[2][24][64];          // [buffer][quad of the step][row]
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t row = blockIdx.x * 64u + lane;
    const uint8_t *wr = w + (size_t)(row < rows ? row : rows - 1u) * row_bytes;
    const uint32_t nb = cols / 32u, nsteps = (nb + 2u) / 3u;
    const uint32_t p = wave - 1u;             // producer index (waves 1..3)
    Q40Blk ring[QP_AHEAD];
    if (wave != 0u) {
#pragma unroll
        for (int k = 0; k < QP_AHEAD; k++) q40_fetch(ring[k], wr, 3u * (uint32_t)k + p, nb);
        if (p < nb) q40_products(ring[0], x + 32u * p, pr[0], p, lane);
        q40_fetch(ring[0], wr, 3u * QP_AHEAD + p, nb);
    }
    __syncthreads();
    float acc = 0.0f;
    // Step s: the consumer adds buffer s & 1 while the producers fill buffer
    // (s + 1) & 1 with step s + 1, whose block sits in ring[(s + 1) % 4].
    for (uint32_t s0 = 0; s0 < nsteps; s0 += QP_AHEAD) {
#pragma unroll
        for (int j = 0; j < QP_AHEAD; j++) {
            const uint32_t st = s0 + (uint32_t)j;
            if (st >= nsteps) break;
            if (wave == 0u) {
                const uint32_t nq = 8u * (nb - 3u * st < 3u ? nb - 3u * st : 3u);
#pragma unroll
                for (uint32_t q = 0; q < 24u; q++) {
                    if (q >= nq) break;
                    const float4 v = pr[st & 1u][q][lane];
                    acc = acc + v.x;
                    acc = acc + v.y;
                    acc = acc + v.z;
                    acc = acc + v.w;
                }
            } else if (st + 1u < nsteps) {
                const uint32_t b = 3u * (st + 1u) + p;
                const int slot = (j + 1) % QP_AHEAD;   // static once unrolled
                if (b < nb) q40_products(ring[slot], x + 32u * b, pr[(st + 1u) & 1u], p, lane);
                q40_fetch(ring[slot], wr, b + 3u * QP_AHEAD, nb);
            }
            __syncthreads();
        }
    }
    if (wave == 0u && row < rows) y[row] = acc;
}

extern "C" __global__ void __launch_bounds__(64)
mynah_q40_chain1(const uint8_t *__restrict__ w, const float *__restrict__ x, float *y,
                 uint32_t rows, uint32_t cols, uint32_t tokens, uint32_t row_bytes,
                 const float *res) {
    q40_chain<1>(w, x, y, rows, cols, tokens, row_bytes, res);
}

extern "C" __global__ void __launch_bounds__(64)
mynah_q40_chain2(const uint8_t *__restrict__ w, const float *__restrict__ x, float *y,
                 uint32_t rows, uint32_t cols, uint32_t tokens, uint32_t row_bytes,
                 const float *res) {
    q40_chain<2>(w, x, y, rows, cols, tokens, row_bytes, res);
}

extern "C" __global__ void __launch_bounds__(64)
mynah_q40_chain4(const uint8_t *__restrict__ w, const float *__restrict__ x, float *y,
                 uint32_t rows, uint32_t cols, uint32_t tokens, uint32_t row_bytes,
                 const float *res) {
    q40_chain<4>(w, x, y, rows, cols, tokens, row_bytes, res);
}

extern "C" __global__ void __launch_bounds__(64)
mynah_q40_chain8(const uint8_t *__restrict__ w, const float *__restrict__ x, float *y,
                 uint32_t rows, uint32_t cols, uint32_t tokens, uint32_t row_bytes,
                 const float *res) {
    q40_chain<8>(w, x, y, rows, cols, tokens, row_bytes, res);
}
