// decode.hip — the non-GEMV kernels of the resident Qwen3 decode step.
//
// Each follows the f32 operator of the reference decoder it replaces
// (src/kernels.c, src/arch_qwen3.c, src/sampler.c) operation for operation:
// same products and sums, no contraction, double accumulators where the
// reference keeps them. Parallel reductions change only the order of
// double-precision sums (of exactly representable terms) and of
// order-independent maxima; expf is the GPU's.
//
// The step position lives in device memory (`pos`, the reference's n_past),
// so one captured launch sequence advances itself when replayed.
//
// SPDX-License-Identifier: MIT
#include "common.hip.h"

#define DEC_WG 256

// Wave-wide double sum / float max (all lanes get the result).
MYNAH_DEV double wave_sum_d(double v) {
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

MYNAH_DEV float wave_max_f(float v) {
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}

// Per-head RMSNorm then split-half RoPE of one head vector by one wave
// (src/kernels.c:130-137, 173-189): s from the double sum of squares,
// x = x * (s * w), then x[i] = a c - b s, x[i + hd/2] = b c + a s. src may
// equal dst (the key is rotated in place in the cache slot).
MYNAH_DEV void head_norm_rope(const float *src, float *dst, const float *__restrict__ w,
                              const float *__restrict__ cs, const float *__restrict__ sn,
                              uint32_t hd, float eps, float *tmp) {
#pragma clang fp contract(off)
    const uint32_t lane = threadIdx.x & 63u;
    double acc = 0.0;
    for (uint32_t i = lane; i < hd; i += 64) acc += (double)src[i] * (double)src[i];
    const double sum = wave_sum_d(acc);
    const float s = (float)(1.0 / sqrt(sum / (double)hd + (double)eps));
    for (uint32_t i = lane; i < hd; i += 64) tmp[i] = src[i] * (s * w[i]);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    const uint32_t half = hd / 2;
    for (uint32_t i = lane; i < half; i += 64) {
        const float a = tmp[i], b = tmp[i + half], c = cs[i], si = sn[i];
        dst[i] = a * c - b * si;
        dst[i + half] = b * c + a * si;
    }
}

// Attention scores for one key head and a chunk of 64 positions
// (src/kernels.c:228-250 first loop, with src/arch_qwen3.c:209-218 folded in):
// every thread first fetches its key row k_t into registers; then wave g
// normalises and rotates query head kvh * group + g into LDS, and the
// workgroup whose chunk holds `pos` normalises and rotates the new key in the
// cache slot (the only writer of that slot; its own score uses the rotated
// key from LDS); then thread (g, j) computes dot(q, k_t) * scale for
// t = chunk * 64 + j. Grid (n_kv_heads, ceil(n_ctx / 64)), block 64 * group;
// group <= 8, hd == 128.
extern "C" __global__ void __launch_bounds__(512)
mynah_attn_scores(const float *__restrict__ q, float *__restrict__ k_layer,
                  const float *__restrict__ q_norm, const float *__restrict__ k_norm,
                  const float *__restrict__ rope_cos, const float *__restrict__ rope_sin,
                  const uint32_t *__restrict__ pos_ptr, float *__restrict__ scores,
                  uint32_t n_ctx, uint32_t hd, uint32_t kv_dim, uint32_t group, float eps,
                  float scale) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) float qn[8][128];
    __shared__ __attribute__((aligned(16))) float kn[128];
    __shared__ float tmp[9][128];
    const uint32_t pos = pos_ptr[0], n_kv = pos + 1u;
    const uint32_t kvh = blockIdx.x, t0 = blockIdx.y * 64u;
    if (t0 >= n_kv) return;
    const uint32_t g = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t t = t0 + lane;
    const bool live = t < pos;                      // the new key is rotated below
    float4 kr[32];
    const float4 *krow = (const float4 *)(k_layer + (size_t)(live ? t : 0u) * kv_dim + (size_t)kvh * 128u);
#pragma unroll
    for (int i = 0; i < 32; i++) kr[i] = krow[i];
    const uint32_t half = 64u;
    const float *cs = rope_cos + (size_t)pos * half, *sn = rope_sin + (size_t)pos * half;
    head_norm_rope(q + (size_t)(kvh * group + g) * 128u, qn[g], q_norm, cs, sn, 128u, eps, tmp[g]);
    float *kpos = k_layer + (size_t)pos * kv_dim + (size_t)kvh * 128u;
    if (g == 0 && pos < t0 + 64u) {
        head_norm_rope(kpos, kn, k_norm, cs, sn, 128u, eps, tmp[8]);
        __builtin_amdgcn_wave_barrier();
        for (uint32_t i = lane; i < 128u; i += 64u) kpos[i] = kn[i];
    }
    __syncthreads();
    if (t < n_kv) {
        if (!live) {
#pragma unroll
            for (int i = 0; i < 32; i++) kr[i] = *(const float4 *)(kn + 4 * i);
        }
        float s0[8], s1[8];
#pragma unroll
        for (int l = 0; l < 8; l++) { s0[l] = 0.0f; s1[l] = 0.0f; }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float kv[16] = {kr[4 * j].x, kr[4 * j].y, kr[4 * j].z, kr[4 * j].w,
                                  kr[4 * j + 1].x, kr[4 * j + 1].y, kr[4 * j + 1].z, kr[4 * j + 1].w,
                                  kr[4 * j + 2].x, kr[4 * j + 2].y, kr[4 * j + 2].z, kr[4 * j + 2].w,
                                  kr[4 * j + 3].x, kr[4 * j + 3].y, kr[4 * j + 3].z, kr[4 * j + 3].w};
            const float *qq = qn[g] + 16 * j;
#pragma unroll
            for (int l = 0; l < 8; l++) {
                s0[l] = __builtin_fmaf(qq[l], kv[l], s0[l]);
                s1[l] = __builtin_fmaf(qq[8 + l], kv[8 + l], s1[l]);
            }
        }
        // src/kernels.c:56-62: lanes s0 + s1, halves, two pair-adds.
        float tt[8], v[4];
#pragma unroll
        for (int l = 0; l < 8; l++) tt[l] = s0[l] + s1[l];
#pragma unroll
        for (int l = 0; l < 4; l++) v[l] = tt[l] + tt[l + 4];
        const float dot = (v[0] + v[1]) + (v[2] + v[3]);
        scores[(size_t)(kvh * group + g) * n_ctx + t] = dot * scale;
    }
}

// Softmax and weighted sum of V for one key head and 16 output dimensions
// (src/kernels.c:207-220, 244-249): wave g % 4 turns the scores of query
// head kvh * group + g into probabilities in LDS (f32 max, expf, double sum,
// times the f32 reciprocal); the V columns stream through LDS in chunks of
// AO_CH positions, double-buffered (the whole workgroup loads chunk c + 1
// while the chain threads consume chunk c); thread (g, j) accumulates
// o = fma(v_t[d], p_t, o) for t = 0 .. n_kv - 1 in order, d = 16 * chunk + j.
// Grid (n_kv_heads, hd / 16), block 256; group <= 16; dynamic LDS group *
// n_ctx floats.
#define AO_CH 256
extern "C" __global__ void __launch_bounds__(256)
mynah_attn_out(const float *__restrict__ v_layer, const float *__restrict__ scores,
               const uint32_t *__restrict__ pos_ptr, float *__restrict__ out, uint32_t n_ctx,
               uint32_t hd, uint32_t kv_dim, uint32_t group) {
#pragma clang fp contract(off)
    extern __shared__ float p_all[];
    __shared__ __attribute__((aligned(16))) float vb[2][AO_CH][16];
    const uint32_t n_kv = pos_ptr[0] + 1u;
    const uint32_t kvh = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    for (uint32_t gw = wave; gw < group; gw += 4u) {
        const uint32_t h = kvh * group + gw;
        float *p = p_all + (size_t)gw * n_ctx;
        const float *sc = scores + (size_t)h * n_ctx;
        float m = -__builtin_inff();
        for (uint32_t t = lane; t < n_kv; t += 64) m = fmaxf(m, sc[t]);
        m = wave_max_f(m);
        double acc = 0.0;
        for (uint32_t t = lane; t < n_kv; t += 64) {
            const float e = expf(sc[t] - m);
            p[t] = e;
            acc += (double)e;
        }
        const double sum = wave_sum_d(acc);
        const float inv = (float)(1.0 / sum);
        for (uint32_t t = lane; t < n_kv; t += 64) p[t] = p[t] * inv;
    }
    // Chunk loader: row r of the chunk (16 floats = 4 float4) -> vb.
    const float *vcol = v_layer + (size_t)kvh * hd + 16u * blockIdx.y;
    const uint32_t nc = (n_kv + AO_CH - 1u) / AO_CH;
    float4 reg[4];
    auto fetch = [&](uint32_t c) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t idx = threadIdx.x + 256u * (uint32_t)k;   // float4 index in the chunk
            const uint32_t t = c * AO_CH + idx / 4u;
            reg[k] = t < n_kv ? *(const float4 *)(vcol + (size_t)t * kv_dim + 4u * (idx % 4u))
                              : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    };
    auto stash = [&](uint32_t buf) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t idx = threadIdx.x + 256u * (uint32_t)k;
            *(float4 *)(&vb[buf][idx / 4u][4u * (idx % 4u)]) = reg[k];
        }
    };
    fetch(0);
    stash(0);
    __syncthreads();
    const uint32_t g = threadIdx.x >> 4, j = threadIdx.x & 15u;
    const bool chain = g < group;
    const float *p = p_all + (size_t)(chain ? g : 0u) * n_ctx;
    float o = 0.0f;
    for (uint32_t c = 0; c < nc; c++) {
        if (c + 1 < nc) fetch(c + 1);
        if (chain) {
            const uint32_t tn = n_kv - c * AO_CH < AO_CH ? n_kv - c * AO_CH : AO_CH;
            const float *pc = p + c * AO_CH;
            const uint32_t b = c & 1u;
            uint32_t t = 0;
            for (; t + 16 <= tn; t += 16) {
                float vv[16], pp[16];
#pragma unroll
                for (int k = 0; k < 16; k++) { vv[k] = vb[b][t + k][j]; pp[k] = pc[t + k]; }
#pragma unroll
                for (int k = 0; k < 16; k++) o = __builtin_fmaf(vv[k], pp[k], o);
            }
            for (; t < tn; t++) o = __builtin_fmaf(vb[b][t][j], pc[t], o);
        }
        if (c + 1 < nc) stash((c + 1) & 1u);
        __syncthreads();
    }
    if (chain) out[(size_t)(kvh * group + g) * hd + 16u * blockIdx.y + j] = o;
}

// src/kernels.c:118-128 (the final norm before the head,
// src/arch_qwen3.c:239): s = (float)(1 / sqrt(sum(x^2) / n + eps)) with the
// sum in double; out = (x * s) * w. One workgroup.
extern "C" __global__ void __launch_bounds__(1024)
mynah_rmsnorm(const float *__restrict__ x, const float *__restrict__ w, float *__restrict__ out,
              uint32_t n, float eps) {
#pragma clang fp contract(off)
    __shared__ double sh[16];
    double acc = 0.0;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) acc += (double)x[i] * (double)x[i];
    const double sum = block_sum_d(acc, sh);
    const float s = (float)(1.0 / sqrt(sum / (double)n + (double)eps));
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) out[i] = x[i] * s * w[i];
}

// src/sampler.c:122-129 finishes here: each workgroup of the head GEMV left
// one 64-bit key (orderable logit << 32 | ~row) for the first maximum of its
// rows; the largest key is the first index of the maximum logit. Writes the
// token, appends it to tokens[step], and advances pos and step (the
// reference's n_past++). One workgroup.
extern "C" __global__ void __launch_bounds__(1024)
mynah_argmax_advance(const unsigned long long *__restrict__ keys, uint32_t n_keys,
                     uint32_t *__restrict__ token, uint32_t *__restrict__ tokens,
                     uint32_t *__restrict__ pos, uint32_t *__restrict__ step, uint32_t max_steps) {
    __shared__ unsigned long long wk[16];
    unsigned long long best = 0ull;
    for (uint32_t i = threadIdx.x; i < n_keys; i += blockDim.x) best = keys[i] > best ? keys[i] : best;
    best = wave_max_u64(best);
    if ((threadIdx.x & 63u) == 0) wk[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t k = 1; k < (blockDim.x + 63u) / 64u; k++) best = wk[k] > best ? wk[k] : best;
        const uint32_t idx = ~(uint32_t)(best & 0xffffffffull);
        token[0] = idx;
        const uint32_t s = step[0];
        if (s < max_steps) tokens[s] = idx;
        step[0] = s + 1u;
        pos[0] = pos[0] + 1u;
    }
}

// src/arch_qwen3.c:160-176: dequantise embedding row `token` into x (no
// scaling). type 0 = f32 rows; otherwise the exact block decoders. One
// thread per 32 values.
extern "C" __global__ void __launch_bounds__(DEC_WG)
mynah_embed_row(const uint8_t *__restrict__ table, const uint32_t *__restrict__ token_ptr,
                float *__restrict__ x, uint32_t d, uint32_t type, uint32_t row_bytes) {
#pragma clang fp contract(off)
    const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;   // 32-value group
    if (c >= d / 32u) return;
    const uint8_t *row = table + (size_t)token_ptr[0] * row_bytes;
    float *dst = x + 32u * c;
    if (type == 0u) {
        const float *f = (const float *)row + 32u * c;
        for (int i = 0; i < 32; i++) dst[i] = f[i];
    } else if (type == 12u) {
        const uint8_t *blk = row + (c / 8u) * 144u;
        const uint32_t j = c % 8u, g = j >> 1;
        const float dd = f16_to_f32(blk[0] | (blk[1] << 8)), dmin = f16_to_f32(blk[2] | (blk[3] << 8));
        const uint8_t *s = blk + 4;
        uint32_t sc, m;
        if (j < 4) { sc = s[j] & 63u; m = s[j + 4] & 63u; }
        else {
            sc = (s[j + 4] & 15u) | ((s[j - 4] >> 6) << 4);
            m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
        }
        const float a = dd * (float)sc, o = dmin * (float)m;
        for (int i = 0; i < 32; i++) {
            const uint32_t q = (j & 1u) ? (blk[16 + 32 * g + i] >> 4) : (blk[16 + 32 * g + i] & 15u);
            dst[i] = a * (float)q - o;
        }
    } else if (type == 14u) {
        const uint8_t *blk = row + (c / 8u) * 210u;
        const uint32_t qq = c % 8u, h = qq >> 2, k = qq & 3u;
        const float dd = f16_to_f32(blk[208] | (blk[209] << 8));
        const int8_t *sc = (const int8_t *)(blk + 192);
        const uint8_t *ql = blk + 64u * h + 32u * (k & 1u), *qh = blk + 128u + 32u * h;
        for (int i = 0; i < 32; i++) {
            const uint32_t lo = (k < 2) ? (ql[i] & 15u) : (ql[i] >> 4);
            const int q = (int)(lo | (((qh[i] >> (2u * k)) & 3u) << 4)) - 32;
            dst[i] = dd * (float)sc[8u * h + 2u * k + (uint32_t)i / 16u] * (float)q;
        }
    } else {
        const uint8_t *blk = row + c * 34u;
        const float dd = f16_to_f32(blk[0] | (blk[1] << 8));
        for (int i = 0; i < 32; i++) dst[i] = (float)(int8_t)blk[2 + i] * dd;
    }
}

