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
// Layout: lane = row (64 rows per one-wave workgroup), T tokens per lane as T
// independent chains interleaved (T = 1 for the matvec, 8 batched), grid.y
// over token groups. The row is streamed in chunks of 8 blocks (256 values,
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
MYNAH_DEV void q40_chain(const uint8_t *__restrict__ w, const float *__restrict__ x,
                         float *__restrict__ y, uint32_t rows, uint32_t cols, uint32_t tokens,
                         uint32_t row_bytes) {
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
            if (t0 + (uint32_t)t < tokens) y[(size_t)(t0 + (uint32_t)t) * rows + row] = acc[t];
    }
}

extern "C" __global__ void __launch_bounds__(64)
mynah_q40_chain1(const uint8_t *__restrict__ w, const float *__restrict__ x, float *__restrict__ y,
                 uint32_t rows, uint32_t cols, uint32_t tokens, uint32_t row_bytes) {
    q40_chain<1>(w, x, y, rows, cols, tokens, row_bytes);
}

extern "C" __global__ void __launch_bounds__(64)
mynah_q40_chain8(const uint8_t *__restrict__ w, const float *__restrict__ x, float *__restrict__ y,
                 uint32_t rows, uint32_t cols, uint32_t tokens, uint32_t row_bytes) {
    q40_chain<8>(w, x, y, rows, cols, tokens, row_bytes);
}
