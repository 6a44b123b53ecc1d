// decode.hip — the non-GEMV kernels of the resident Qwen3 decode step.
//
// Each follows the f32 operator of the reference decoder it replaces
// (src/kernels.c, src/arch_qwen3.c, src/sampler.c) operation for operation:
// same products and sums, no contraction, double accumulators where the
// reference keeps them. Parallel reductions change only the order of
// order-independent maxima and of double-precision sums of exactly
// representable terms, whose f32 results (the softmax reciprocal, the RMS
// scale) are kept only where sum_settled (sum_settle.h) shows that the
// reference's index order gives the same; elsewhere the terms are added
// again in index order. expf is the C library's (mynah_expf.h).
//
// The step position lives in device memory (`pos`, the reference's n_past),
// so one captured launch sequence advances itself when replayed.
//
// SPDX-License-Identifier: MIT
#include "common.hip.h"

// The value of lane i + N of the same 16-lane row (DPP row_shl:N; past the
// row end 0, which no caller uses).
template <int N>
MYNAH_DEV float row_down(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + N, 0xf, 0xf, false));
}

// Lane 0 of each 16-lane row: the sum of the row's 16 partial dots in the
// horizontal order of the reference's AVX2 dot (src/kernels.c:39-62): the
// two 8-lane halves, then 4, then 1, then 2 apart.
MYNAH_DEV float row16_dot(float acc) {
    const float tt = acc + row_down<8>(acc);
    const float v = tt + row_down<4>(tt);
    const float w = v + row_down<1>(v);
    return w + row_down<2>(w);
}

#define DEC_WG 256

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
    const float s = rms_scale_settled(wave_sum_d(acc), src, hd, eps);
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

// Per-head RMSNorm + RoPE of a 128-vector held by one wave, lane i holding
// x[i] and x[i + 64] (src/kernels.c:130-137, 173-189): the same operations as
// head_norm_rope, with the pair (i, i + 64) rotated in registers. The sum of
// squares is the wave's (seq = false) or the reference's index order
// (seq = true: x[0 .. 63] from the lanes' x0, then x[64 .. 127]); returns
// the double scale r, s = (float)r, for the caller's check (sum_settled).
MYNAH_DEV double norm_rope_reg(float x0, float x1, float w0, float w1, float c, float sn,
                               float eps, bool seq, float &y0, float &y1) {
#pragma clang fp contract(off)
    double sum;
    if (!seq) {
        sum = wave_sum_d((double)x0 * (double)x0 + (double)x1 * (double)x1);
    } else {
        sum = 0.0;
#pragma nounroll
        for (int j = 0; j < 64; j++) {
            const double v = (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(x0), j));
            sum += v * v;
        }
#pragma nounroll
        for (int j = 0; j < 64; j++) {
            const double v = (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(x1), j));
            sum += v * v;
        }
    }
    const double r = rms_inv(sum, 128u, eps);
    const float s = (float)r;
    const float a = x0 * (s * w0), b = x1 * (s * w1);
    y0 = a * c - b * sn;
    y1 = b * c + a * sn;
    return r;
}

// Attention scores for one key head and a chunk of SC_POS positions
// (src/kernels.c:228-250 first loop, with src/arch_qwen3.c:209-218 folded in).
// Lane (r, l) of wave w handles position t = t0 + 4 w + r and the dot-product
// lane l of the reference's 8-wide FMA dot (src/kernels.c:39-62): it holds
// k_t[16 j + l] for j = 0..7 and accumulates fma(q[16 j + l], k_t[16 j + l])
// over j, which is s0[l] for l < 8 and s1[l - 8] otherwise; the 16 lanes of a
// position then combine exactly as the reference does: tt = s0 + s1, v[l] =
// tt[l] + tt[l + 4], dot = (v0 + v1) + (v2 + v3). The query heads kvh * group
// + h are normalised and rotated (src/kernels.c:130-137, 173-189) in
// registers by wave h % 4 into LDS, and the workgroup whose chunk holds `pos`
// normalises and rotates the new key in the cache slot (the only writer of
// that slot; its own score uses the rotated key from LDS). Nothing before the
// position's arrival depends on it: chunks below spec_chunks (those live when
// the launch was enqueued; the position only grows) load their key rows
// (clamped into the cache) at once, the query heads, their norm weights and
// the rotation of the position (rope_now, its cos and sin rows, copied there
// by the launch that set the position) likewise; the other chunks first learn
// whether they hold any position. Scores rows are `sstride` floats apart.
// Grid (n_kv_heads, ceil(n_ctx / SC_POS)), block 256; group <= 8, hd == 128.
#define SC_POS 16
MYNAH_DEV void attn_scores_body(const float *__restrict__ q, float *__restrict__ k_layer,
                                const float *__restrict__ q_norm, const float *__restrict__ k_norm,
                                const float *__restrict__ rope_now,
                                const uint32_t *__restrict__ pos_ptr, float *__restrict__ scores,
                                uint32_t n_ctx, uint32_t sstride, uint32_t kv_dim, uint32_t group,
                                float eps, float scale, uint32_t spec_chunks) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) float qn[8][128];
    __shared__ __attribute__((aligned(16))) float kn[128];
    __shared__ double nr[9];
    const uint32_t forced = index_sums_forced();
    const uint32_t kvh = blockIdx.x, c = blockIdx.y, t0 = c * SC_POS;
    if (c >= spec_chunks && t0 >= pos_ptr[0] + 1u) return;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t r = lane >> 4, l = lane & 15u;
    const uint32_t t = t0 + 4u * wave + r;
    const uint32_t row = t < n_ctx ? t : n_ctx - 1u;
    const float *krow = k_layer + (size_t)row * kv_dim + (size_t)kvh * 128u + l;
    float kv[8];
#pragma unroll
    for (int j = 0; j < 8; j++) kv[j] = krow[16 * j];
    // Query heads wave and wave + 4 (those below group), their norm weights
    // and the rotation of the position.
    float x0[2], x1[2];
    const float w0 = q_norm[lane], w1 = q_norm[lane + 64u];
    const float cs = rope_now[lane], sn = rope_now[64u + lane];
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const uint32_t h = wave + 4u * (uint32_t)e;
        const float *src = q + (size_t)(kvh * group + (h < group ? h : 0u)) * 128u;
        x0[e] = src[lane];
        x1[e] = src[lane + 64u];
    }
    const uint32_t pos = pos_ptr[0], n_kv = pos + 1u;
    if (t0 >= n_kv) return;       // a speculative chunk past the position (after a reset)
    const bool has_pos = pos < t0 + SC_POS;
    // The new key: wave group % 4 (after its query heads, if any).
    const uint32_t kw = group % 4u;
    float *kpos = k_layer + (size_t)pos * kv_dim + (size_t)kvh * 128u;
    float k0 = 0.0f, k1 = 0.0f, kw0 = 0.0f, kw1 = 0.0f;
    if (has_pos && wave == kw) {
        k0 = kpos[lane];
        k1 = kpos[lane + 64u];
        kw0 = k_norm[lane];
        kw1 = k_norm[lane + 64u];
    }
    // The norms, then the scores; each norm's double scale goes to nr (the
    // query heads' at h, the key's at 8) for the check after the scores.
    auto norms = [&](bool seq) __attribute__((always_inline)) {
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const uint32_t h = wave + 4u * (uint32_t)e;
            if (h < group) {
                float y0, y1;
                const double rs = norm_rope_reg(x0[e], x1[e], w0, w1, cs, sn, eps, seq, y0, y1);
                qn[h][lane] = y0;
                qn[h][lane + 64u] = y1;
                if (lane == 0) nr[h] = rs;
            }
        }
        if (has_pos && wave == kw) {
            float y0, y1;
            const double rs = norm_rope_reg(k0, k1, kw0, kw1, cs, sn, eps, seq, y0, y1);
            kn[lane] = y0;
            kn[lane + 64u] = y1;
            kpos[lane] = y0;
            kpos[lane + 64u] = y1;
            if (lane == 0) nr[8] = rs;
        }
    };
    auto dots = [&]() __attribute__((always_inline)) {
        if (t < n_kv) {
            if (t >= pos) {
#pragma unroll
                for (int j = 0; j < 8; j++) kv[j] = kn[16 * j + l];
            }
            for (uint32_t h = 0; h < group; h++) {
                float acc = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; j++) acc = __builtin_fmaf(qn[h][16 * j + l], kv[j], acc);
                const float dot = row16_dot(acc);
                if (l == 0) scores[(size_t)(kvh * group + h) * sstride + t] = dot * scale;
            }
        }
    };
    norms(false);
    __syncthreads();
    dots();
    // The check, after the scores are out (off the path to them): lane h <
    // group tests query head h's scale, lane 8 the key's; every wave reads
    // the same nr, so the workgroup decides as one. Where a scale does not
    // settle (or under the test switch), the norms are taken again in index
    // order and the scores (and the cache slot) written again.
    bool bad = false;
    if (lane < group || (lane == 8u && has_pos)) bad = !sum_settled(nr[lane], 128u, 1u, 0u);
    if (forced != 0u || __ballot(bad) != 0ull) {
        __syncthreads();
        norms(true);
        __syncthreads();
        dots();
    }
}

extern "C" __global__ void __launch_bounds__(256)
mynah_attn_scores(const float *__restrict__ q, float *__restrict__ k_layer,
                  const float *__restrict__ q_norm, const float *__restrict__ k_norm,
                  const float *__restrict__ rope_now, const uint32_t *__restrict__ pos_ptr,
                  float *__restrict__ scores, uint32_t n_ctx, uint32_t sstride, uint32_t kv_dim,
                  uint32_t group, float eps, float scale, uint32_t spec_chunks) {
    attn_scores_body(q, k_layer, q_norm, k_norm, rope_now, pos_ptr, scores, n_ctx, sstride,
                     kv_dim, group, eps, scale, spec_chunks);
}

// Softmax and weighted sum of V for one key head and AO_DV = 8 output
// dimensions (src/kernels.c:207-220, 244-249). Wave g turns the scores of
// query head kvh * group + g into probabilities: the scores are loaded into
// registers (lane l holds positions 4 l + 256 k .. + 3), then the f32 max,
// expf, the double sum and the product with the f32 reciprocal of the sum,
// and the probabilities land in LDS. The V slice (32 contiguous bytes of each
// position: two lanes per row) streams through LDS, transposed to
// dimension-major, in chunks of AO_CH positions, chunk c + 1 fetched into
// registers while chunk c is consumed; lane j < AO_DV of wave g accumulates
// o = fma(v_t[d], p_t, o) for t = 0 .. n_kv - 1 in order, d = AO_DV *
// blockIdx.y + j. Scores rows are `sstride` floats apart (a multiple of 4).
// Grid (n_kv_heads, hd / AO_DV), block 64 * group, group in 2..8; n_kv <= 64
// * 4 * AO_SK; dynamic LDS group * sstride floats.
#define AO_DV 8
#define AO_CH 1024
#define AO_SK 16
#define AO_VR (AO_CH * 2 / 128)

// Chunk c of the V slice: row t = c * AO_CH + (i >> 1), half i & 1, for
// i = threadIdx.x + nthr * k (nthr = blockDim.x >= 128); only the passes
// that hold rows below n_kv are issued.
MYNAH_DEV void ao_fetch(float4 *vr, const float *vcol, uint32_t c, uint32_t n_kv, uint32_t kv_dim,
                        uint32_t nthr) {
    const uint32_t rows = n_kv - c * AO_CH < AO_CH ? n_kv - c * AO_CH : AO_CH;
    const uint32_t npass = (2u * rows + nthr - 1u) / nthr;
#pragma unroll
    for (int k = 0; k < AO_VR; k++) {
        if ((uint32_t)k < npass) {
            const uint32_t i = threadIdx.x + nthr * (uint32_t)k;
            const uint32_t r = i >> 1;
            vr[k] = r < rows ? *(const float4 *)(vcol + (size_t)(c * AO_CH + r) * kv_dim + 4u * (i & 1u))
                             : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
}

MYNAH_DEV float ao_fma4(float4 v, float4 p, float o) {
    o = __builtin_fmaf(v.x, p.x, o);
    o = __builtin_fmaf(v.y, p.y, o);
    o = __builtin_fmaf(v.z, p.z, o);
    return __builtin_fmaf(v.w, p.w, o);
}

// Softmax of one scores row over positions 0 .. n_kv - 1 by one wave
// (src/kernels.c:207-220), in two parts. softmax_load: lane l takes the
// float4s l, l + 64, ... (KS of them, n_kv <= 256 KS) into registers, the
// index clamped to the row's last float4 that holds a position; straight-line
// loads, so the wave waits for them once and not behind each other.
// softmax_finish: positions past n_kv become -inf, then the f32 max, expf
// (2^(i/32) table at `tab`), the double sum and the product with the f32
// reciprocal of the sum; p gets the probabilities of the float4s that hold
// positions < n_kv (positions past n_kv in the last float4 get 0). p may
// equal sc_row (every score is read before any probability is written).
template <int KS = AO_SK>
MYNAH_DEV void softmax_load(float4 *sv, const float *sc_row, uint32_t n_kv) {
    const uint32_t lane = threadIdx.x & 63u;
    const float4 *sc = (const float4 *)sc_row;
    const uint32_t n4 = (n_kv + 3u) / 4u;
#pragma unroll
    for (int k = 0; k < KS; k++) {
        const uint32_t i = lane + 64u * (uint32_t)k;
        sv[k] = sc[i < n4 ? i : n4 - 1u];
    }
}

template <int KS = AO_SK>
MYNAH_DEV void softmax_finish(float4 *sv, uint32_t n_kv, float *p, const uint64_t *tab) {
#pragma clang fp contract(off)
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t n4 = (n_kv + 3u) / 4u, kmax = (n4 + 63u) / 64u;
    const float ninf = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < KS; k++) {
        if ((uint32_t)k < kmax) {
            const uint32_t i = lane + 64u * (uint32_t)k, t = 4u * i;
            float4 v = i < n4 ? sv[k] : make_float4(ninf, ninf, ninf, ninf);
            if (t + 1u >= n_kv) v.y = ninf;
            if (t + 2u >= n_kv) v.z = ninf;
            if (t + 3u >= n_kv) v.w = ninf;
            sv[k] = v;
        }
    }
    float m = ninf;
#pragma unroll
    for (int k = 0; k < KS; k++)
        if ((uint32_t)k < kmax)
            m = fmaxf(fmaxf(fmaxf(m, sv[k].x), fmaxf(sv[k].y, sv[k].z)), sv[k].w);
    m = wave_max_f(m);
    double acc = 0.0;
#pragma unroll
    for (int k = 0; k < KS; k++) {
        if ((uint32_t)k < kmax) {
            float4 e;
            e.x = mynah_expf_t(sv[k].x - m, tab);
            e.y = mynah_expf_t(sv[k].y - m, tab);
            e.z = mynah_expf_t(sv[k].z - m, tab);
            e.w = mynah_expf_t(sv[k].w - m, tab);
            acc += (double)e.x;
            acc += (double)e.y;
            acc += (double)e.z;
            acc += (double)e.w;
            sv[k] = e;
        }
    }
    double r = 1.0 / wave_sum_d(acc);
    if (MYNAH_UNSETTLED(r, n_kv, 2u, index_sums_forced())) {
        // The exponentials into p, then every lane adds them in index order.
#pragma unroll
        for (int k = 0; k < KS; k++) {
            const uint32_t i = lane + 64u * (uint32_t)k;
            if ((uint32_t)k < kmax && i < n4) *(float4 *)(p + 4u * i) = sv[k];
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
        __builtin_amdgcn_wave_barrier();
        r = 1.0 / seq_sum(p, n_kv);
    }
    const float inv = (float)r;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int k = 0; k < KS; k++) {
        if ((uint32_t)k < kmax) {
            const uint32_t i = lane + 64u * (uint32_t)k;
            const float4 e = sv[k];
            if (i < n4)
                *(float4 *)(p + 4u * i) = make_float4(e.x * inv, e.y * inv, e.z * inv, e.w * inv);
        }
    }
}

MYNAH_DEV void softmax_row(const float *sc_row, uint32_t n_kv, float *p) {
    float4 sv[AO_SK];
    softmax_load(sv, sc_row, n_kv);
    softmax_finish(sv, n_kv, p, mynah_exp2_tab);
}

// softmax_row for rows of any length, by one wave, through memory instead of
// registers: the same float4-to-lane assignment (lane l takes float4s l,
// l + 64, ...), the same masking of the last float4, the same order of each
// lane's double sum and the same wave reduction, so its results are
// bit-identical to softmax_row's wherever both apply. Three passes: the
// maximum; e = expf(s - m) written over p (p may equal sc_row: each float4
// is read, then written, by the same lane) with the double sum; p = e *
// inv.
MYNAH_DEV void softmax_row_long(const float *sc_row, uint32_t n_kv, float *p) {
#pragma clang fp contract(off)
    const uint32_t lane = threadIdx.x & 63u;
    const float4 *sc = (const float4 *)sc_row;
    float4 *p4 = (float4 *)p;
    const uint32_t n4 = (n_kv + 3u) / 4u;
    const float ninf = -__builtin_inff();
    auto masked = [&](uint32_t i) {
        float4 v = sc[i];
        const uint32_t t = 4u * i;
        if (t + 1u >= n_kv) v.y = ninf;
        if (t + 2u >= n_kv) v.z = ninf;
        if (t + 3u >= n_kv) v.w = ninf;
        return v;
    };
    float m = ninf;
    for (uint32_t i = lane; i < n4; i += 64u) {
        const float4 v = masked(i);
        m = fmaxf(fmaxf(fmaxf(m, v.x), fmaxf(v.y, v.z)), v.w);
    }
    m = wave_max_f(m);
    double acc = 0.0;
    for (uint32_t i = lane; i < n4; i += 64u) {
        const float4 v = masked(i);
        float4 e;
        e.x = mynah_expf(v.x - m);
        e.y = mynah_expf(v.y - m);
        e.z = mynah_expf(v.z - m);
        e.w = mynah_expf(v.w - m);
        acc += (double)e.x;
        acc += (double)e.y;
        acc += (double)e.z;
        acc += (double)e.w;
        p4[i] = e;
    }
    double r = 1.0 / wave_sum_d(acc);
    if (MYNAH_UNSETTLED(r, n_kv, 2u, index_sums_forced())) {
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
        __builtin_amdgcn_wave_barrier();
        r = 1.0 / seq_sum(p, n_kv);
    }
    const float inv = (float)r;
    for (uint32_t i = lane; i < n4; i += 64u) {
        const float4 e = p4[i];
        p4[i] = make_float4(e.x * inv, e.y * inv, e.z * inv, e.w * inv);
    }
}

// Rows up to 4096 positions in registers, longer ones through memory (the
// same bits either way).
MYNAH_DEV void softmax_any(const float *sc_row, uint32_t n_kv, float *p) {
    if (n_kv <= 64u * 4u * AO_SK) softmax_row(sc_row, n_kv, p);
    else softmax_row_long(sc_row, n_kv, p);
}

MYNAH_DEV void attn_out_body(const float *__restrict__ v_layer, const float *__restrict__ scores,
                             uint32_t pos, float *__restrict__ out, uint32_t sstride,
                             uint32_t kv_dim, uint32_t group) {
#pragma clang fp contract(off)
    extern __shared__ __attribute__((aligned(16))) float p_all[];
    __shared__ __attribute__((aligned(16))) float vt[AO_DV][AO_CH + 4];
    const uint32_t n_kv = pos + 1u;
    const uint32_t kvh = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t nthr = blockDim.x;
    const float *vcol = v_layer + (size_t)kvh * 128u + AO_DV * blockIdx.y;
    const uint32_t nc = (n_kv + AO_CH - 1u) / AO_CH;
    float4 vr[AO_VR];
    ao_fetch(vr, vcol, 0, n_kv, kv_dim, nthr);

    // Softmax of head g = wave into LDS.
    float *p = p_all + (size_t)wave * sstride;
    softmax_any(scores + (size_t)(kvh * group + wave) * sstride, n_kv, p);

    const bool chain = lane < AO_DV;
    float o = 0.0f;
    for (uint32_t c = 0; c < nc; c++) {
        const uint32_t tn = n_kv - c * AO_CH < AO_CH ? n_kv - c * AO_CH : AO_CH;
        const uint32_t npass = (2u * tn + nthr - 1u) / nthr;
#pragma unroll
        for (int k = 0; k < AO_VR; k++) {
            const uint32_t i = threadIdx.x + nthr * (uint32_t)k;
            const uint32_t r = i >> 1, d = 4u * (i & 1u);
            if ((uint32_t)k < npass && r < AO_CH) {
                vt[d][r] = vr[k].x; vt[d + 1][r] = vr[k].y; vt[d + 2][r] = vr[k].z; vt[d + 3][r] = vr[k].w;
            }
        }
        __syncthreads();
        if (c + 1 < nc) ao_fetch(vr, vcol, c + 1, n_kv, kv_dim, nthr);
        if (chain) {
            const float *pc = p + c * AO_CH, *vc = vt[lane];
            uint32_t t = 0;
            for (; t + 16 <= tn; t += 16) {
                float4 va[4], pa[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    va[k] = *(const float4 *)(vc + t + 4 * k);
                    pa[k] = *(const float4 *)(pc + t + 4 * k);
                }
#pragma unroll
                for (int k = 0; k < 4; k++) o = ao_fma4(va[k], pa[k], o);
            }
            for (; t < tn; t++) o = __builtin_fmaf(vc[t], pc[t], o);
        }
        __syncthreads();
    }
    if (chain) out[(size_t)(kvh * group + wave) * 128u + AO_DV * blockIdx.y + lane] = o;
}

extern "C" __global__ void __launch_bounds__(512)
mynah_attn_out(const float *__restrict__ v_layer, const float *__restrict__ scores,
               const uint32_t *__restrict__ pos_ptr, float *__restrict__ out, uint32_t sstride,
               uint32_t kv_dim, uint32_t group) {
    attn_out_body(v_layer, scores, pos_ptr[0], out, sstride, kv_dim, group);
}

// ── exact attention for contexts whose score rows outgrow the LDS ─────────
// The same operations as mynah_attn_out in two launches: the softmax of
// every head's scores in place (one wave per head, softmax_row_long, the
// bits of softmax_row), then the ordered PV chains of mynah_attn_out with
// the probabilities staged per chunk of AO_CH positions beside the V slice.
extern "C" __global__ void __launch_bounds__(64)
mynah_attn_softmax(float *scores, const uint32_t *__restrict__ pos_ptr, uint32_t sstride) {
    float *row = scores + (size_t)blockIdx.x * sstride;
    softmax_row_long(row, pos_ptr[0] + 1u, row);
}

extern "C" __global__ void __launch_bounds__(512)
mynah_attn_out_long(const float *__restrict__ v_layer, const float *__restrict__ probs,
                    const uint32_t *__restrict__ pos_ptr, float *__restrict__ out,
                    uint32_t sstride, uint32_t kv_dim, uint32_t group) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) float vt[AO_DV][AO_CH + 4];
    extern __shared__ __attribute__((aligned(16))) float pcd[];     // [group][AO_CH]
    const uint32_t n_kv = pos_ptr[0] + 1u;
    const uint32_t kvh = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t nthr = blockDim.x;
    const float *vcol = v_layer + (size_t)kvh * 128u + AO_DV * blockIdx.y;
    const float4 *prow = (const float4 *)(probs + (size_t)(kvh * group + wave) * sstride);
    const uint32_t nc = (n_kv + AO_CH - 1u) / AO_CH;
    float4 vr[AO_VR];
    ao_fetch(vr, vcol, 0, n_kv, kv_dim, nthr);
    const bool chain = lane < AO_DV;
    float o = 0.0f;
    for (uint32_t c = 0; c < nc; c++) {
        const uint32_t tn = n_kv - c * AO_CH < AO_CH ? n_kv - c * AO_CH : AO_CH;
        const uint32_t npass = (2u * tn + nthr - 1u) / nthr;
#pragma unroll
        for (int k = 0; k < AO_VR; k++) {
            const uint32_t i = threadIdx.x + nthr * (uint32_t)k;
            const uint32_t r = i >> 1, d = 4u * (i & 1u);
            if ((uint32_t)k < npass && r < AO_CH) {
                vt[d][r] = vr[k].x; vt[d + 1][r] = vr[k].y; vt[d + 2][r] = vr[k].z; vt[d + 3][r] = vr[k].w;
            }
        }
        // This wave's probabilities of the chunk (softmax_row wrote whole
        // float4s, 0 past n_kv in the last one).
        for (uint32_t i = lane; i < (tn + 3u) / 4u; i += 64u)
            *(float4 *)&pcd[wave * AO_CH + 4u * i] = prow[c * (AO_CH / 4u) + i];
        __syncthreads();
        if (c + 1 < nc) ao_fetch(vr, vcol, c + 1, n_kv, kv_dim, nthr);
        if (chain) {
            const float *pcw = pcd + wave * AO_CH, *vc = vt[lane];
            uint32_t t = 0;
            for (; t + 16 <= tn; t += 16) {
                float4 va[4], pa[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    va[k] = *(const float4 *)(vc + t + 4 * k);
                    pa[k] = *(const float4 *)(pcw + t + 4 * k);
                }
#pragma unroll
                for (int k = 0; k < 4; k++) o = ao_fma4(va[k], pa[k], o);
            }
            for (; t < tn; t++) o = __builtin_fmaf(vc[t], pcw[t], o);
        }
        __syncthreads();
    }
    if (chain) out[(size_t)(kvh * group + wave) * 128u + AO_DV * blockIdx.y + lane] = o;
}

// Calls f(Index<C>), f(Index<C + 1>), ... while the index is below n (and
// N): a run of steps written out, each with its constants, that stops at n.
template <uint32_t C, uint32_t N, class F>
MYNAH_DEV void steps_until(uint32_t n, F &&f) {
    if constexpr (C < N) {
        if (C >= n) return;
        f(Index<C>{});
        steps_until<C + 1u, N>(n, f);
    }
}

// ── exact attention: a PV chain in every lane ──────────────────────────────
// The reference's weighted sum (src/kernels.c:83-100, 252-272) is, for every
// (query head, dimension), one chain o = fma(v_t[d], p_t, o) over t = 0 ..
// n_kv - 1 in order: n_kv dependent FMAs that no reordering may shorten (a
// dependent v_fmac_f32 costs about 8.7 cycles on gfx950). A workgroup takes
// one query head and a slice of DPV_SW = 16 of its dimensions: lane l of wave
// 0 carries the chain of dimension l % DPV_SW (lanes DPV_SW and up repeat the
// first ones and are not stored), reading four positions of its dimension
// (V in LDS dimension-major, rows padded by four floats so the loaders'
// transposing stores and the chain's reads hit 64 distinct banks) and their
// four probabilities (every lane the same address) with one ds_read_b128
// each, eight groups of four positions ahead: the chain's wave issues two LDS
// reads per four FMAs, whose issue cycles add to the chain. V of the slice streams through a
// ring of three LDS chunks of DPV_CH positions, filled by four loader waves
// that keep up to DPV_WIN chunks in flight in registers, one barrier per
// chunk; narrow slices keep each CU's share of V (and its load issue) small
// beside the chain. The probabilities are either computed by the loader
// waves into LDS (PMEM = false, n_kv <= 256 DPV_LW KS: the softmax of
// src/kernels.c:207-220 over the four waves — f32 max, expf, a double sum
// per lane, per wave (wave_sum_d) and then of the four waves in order, kept
// where sum_settled shows the reference's index order gives the same f32
// reciprocal and otherwise taken again in index order, product with the
// f32 reciprocal) or read, normalised by
// mynah_attn_softmax, from the scores rows and staged per chunk beside V
// (PMEM = true, any length). Grid n_heads * 128 / DPV_SW: workgroup b takes
// key head kvh = b % n_kv_heads, query head kvh * group + (b / n_kv_heads) %
// group and slice b / (n_kv_heads * group), so every workgroup of a key head
// runs on the XCD b % 8 names when n_kv_heads is 8 and shares its V rows in
// that L2; block 64 (1 + DPV_LW); hd == 128.
#define DPV_SW 16
#define DPV_CH (4096 / DPV_SW)
#ifndef DPV_LW
#define DPV_LW 4                                          // loader waves (= MYNAH_PV_LW)
#endif
#define DPV_NBUF 3
#define DPV_WIN 4
// A native 4-float vector: arrays of it stay in registers (copies of the
// HIP float4 struct become memcpy calls that can pin an array in scratch).
typedef float v4f __attribute__((ext_vector_type(4)));

// v_layer and sp carry no __restrict__: loads from restrict-qualified
// read-only memory may be moved across barriers, which would undo the
// loaders' placement of their fetches.
template <bool PMEM, int KS>
MYNAH_DEV void attn_pv_body(const float *v_layer, const float *sp, uint32_t pos,
                            float *__restrict__ out, uint32_t sstride, uint32_t kv_dim,
                            uint32_t n_kv_heads, uint32_t group) {
#pragma clang fp contract(off)
    constexpr uint32_t RQ = DPV_SW / 4u;                    // float4 per row of the slice
    constexpr uint32_t NL = 64u * DPV_LW;                    // loader threads
    constexpr uint32_t NV = DPV_CH * DPV_SW / 4u / NL;      // float4 of V per loader thread per chunk
    constexpr uint32_t VST = DPV_CH + 4u;                   // floats per dimension row
    __shared__ __attribute__((aligned(16))) float vbuf[DPV_NBUF][DPV_SW * VST];   // [dim][t]
    __shared__ __attribute__((aligned(16))) float pl[PMEM ? DPV_NBUF * DPV_CH : 4u * NL * KS];
    __shared__ uint64_t etab[DPV_LW][32];
    __shared__ float wmax[DPV_LW];
    __shared__ double wsum[DPV_LW];
    const uint32_t forced = index_sums_forced();
    const uint32_t n_kv = pos + 1u;
    const uint32_t b = blockIdx.x, kvh = b % n_kv_heads, rest = b / n_kv_heads;
    const uint32_t head = kvh * group + rest % group, slice = rest / group;
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
    const uint32_t nc = (n_kv + DPV_CH - 1u) / DPV_CH;
    const float *prow = sp + (size_t)head * sstride;
    if (wave == 0) {
        bool refix = false;
        float fix = 0.0f, mx = 0.0f;
        if constexpr (!PMEM) {
            __syncthreads();                              // wave maxima
            __syncthreads();                              // wave sums
            // The loaders keep the reciprocal of the four waves' double sum
            // in wave order. This wave, idle until the probabilities are
            // staged, checks it (sum_settled); where it does not settle it
            // adds the exponentials again in index order — lane j
            // recomputes position 64 c + j from the scores row with the
            // loaders' expf and maximum, the wave adds each c's 64 values in
            // lane order — and, if that reciprocal differs, rewrites the
            // probabilities before its chain reads them (always, under the
            // test switch).
            double lsum = wsum[0];
#pragma unroll
            for (uint32_t w = 1; w < DPV_LW; w++) lsum = lsum + wsum[w];
            const double r = 1.0 / lsum;
            if (MYNAH_UNSETTLED(r, n_kv, 2u, forced)) {
                mx = wmax[0];
#pragma unroll
                for (uint32_t w = 1; w < DPV_LW; w++) mx = fmaxf(mx, wmax[w]);
                double seq = 0.0;
                for (uint32_t c0 = 0; c0 < n_kv; c0 += 64u) {
                    const uint32_t t = c0 + lane, cnt = n_kv - c0 < 64u ? n_kv - c0 : 64u;
                    const float e = t < n_kv ? mynah_expf_t(prow[t] - mx, etab[0]) : 0.0f;
#pragma nounroll
                    for (uint32_t j = 0; j < cnt; j++)
                        seq += (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), j));
                }
                fix = (float)(1.0 / seq);
                refix = forced != 0u || __float_as_uint(fix) != __float_as_uint((float)r);
            }
        }
        __syncthreads();                                  // p, chunks 0 and 1 staged
        if constexpr (!PMEM) {
            if (refix) {
                for (uint32_t t = lane; t < n_kv; t += 64u)
                    pl[t] = mynah_expf_t(prow[t] - mx, etab[0]) * fix;
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
            }
        }
        const uint32_t d = lane % DPV_SW;
        float acc = 0.0f;
        // Group m of chunk c: positions DPV_CH c + 4 m .. + 3 of this lane's
        // dimension and their probabilities.
        auto vsrc = [&](uint32_t c, uint32_t m) __attribute__((always_inline)) {
            return *(const float4 *)(vbuf[c % DPV_NBUF] + d * VST + 4u * m);
        };
        auto psrc = [&](uint32_t c, uint32_t m) __attribute__((always_inline)) {
            return *(const float4 *)(PMEM ? pl + (c % DPV_NBUF) * DPV_CH + 4u * m
                                          : pl + c * DPV_CH + 4u * m);
        };
        auto fma4 = [&](const float4 v, const float4 p) __attribute__((always_inline)) {
            acc = __builtin_fmaf(v.x, p.x, acc);
            acc = __builtin_fmaf(v.y, p.y, acc);
            acc = __builtin_fmaf(v.z, p.z, acc);
            acc = __builtin_fmaf(v.w, p.w, acc);
        };
        // Full chunks: eight groups of reads in flight, ahead into chunk
        // c + 1, whose buffer was staged before the last barrier (for c + 1
        // past the end the reads are of a stale buffer and unused).
        float4 rv[8], rp[8];
#pragma unroll
        for (uint32_t m = 0; m < 8u; m++) {
            rv[m] = vsrc(0, m);
            rp[m] = psrc(0, m);
        }
        for (uint32_t c = 0; c < nc; c++) {
            const uint32_t tn = n_kv - c * DPV_CH < DPV_CH ? n_kv - c * DPV_CH : DPV_CH;
            if (tn == DPV_CH) {
                static_for<DPV_CH / 4u>([&](auto mi) __attribute__((always_inline)) {
                    constexpr uint32_t m = decltype(mi)::value, r = m % 8u;
                    __builtin_amdgcn_sched_barrier(0);
                    fma4(rv[r], rp[r]);
                    if constexpr (m + 8u < DPV_CH / 4u) {
                        rv[r] = vsrc(c, m + 8u);
                        rp[r] = psrc(c, m + 8u);
                    } else {
                        rv[r] = vsrc(c + 1u, m + 8u - DPV_CH / 4u);
                        rp[r] = psrc(c + 1u, m + 8u - DPV_CH / 4u);
                    }
                });
                __builtin_amdgcn_sched_barrier(0);
            } else {
                // The last chunk, partial: straight from LDS.
                const float *vc = vbuf[c % DPV_NBUF] + d * VST;
                const float *pc = PMEM ? pl + (c % DPV_NBUF) * DPV_CH : pl + c * DPV_CH;
                for (uint32_t t = 0; t < tn; t++) acc = __builtin_fmaf(vc[t], pc[t], acc);
            }
            __syncthreads();
        }
        if (lane < DPV_SW) out[(size_t)head * 128u + slice * DPV_SW + lane] = acc;
        return;
    }

    // Loader waves 1 .. DPV_LW: chunk c is fetched into register slot c % DPV_WIN
    // DPV_WIN chunks before it is stored into buffer c % DPV_NBUF (two
    // iterations before the chain reads it). Rows past the position read the
    // last row, whose copies the chain never reads, so the loads have no
    // branch and the waits count them exactly.
    const uint32_t lt = tid - 64u, lw = wave - 1u;
    const float *vcol = v_layer + (size_t)kvh * 128u + slice * DPV_SW;
    v4f vr[DPV_WIN][NV], pr[DPV_WIN];
    auto fetch = [&](v4f *v4, v4f &p4, uint32_t c) __attribute__((always_inline)) {
#pragma unroll
        for (uint32_t q = 0; q < NV; q++) {
            const uint32_t i = lt + NL * q, t = c * DPV_CH + i / RQ;
            const uint32_t tt = t < n_kv ? t : n_kv - 1u;
            v4[q] = *(const v4f *)(vcol + (size_t)tt * kv_dim + 4u * (i % RQ));
        }
        if constexpr (PMEM) {
            const uint32_t t4 = c * DPV_CH + 4u * (lt % (DPV_CH / 4u)), last = (n_kv - 1u) & ~3u;
            p4 = *(const v4f *)(prow + (t4 < n_kv ? t4 : last));
        }
    };
    auto store = [&](const v4f *v4, const v4f &p4, uint32_t c) __attribute__((always_inline)) {
#pragma unroll
        for (uint32_t q = 0; q < NV; q++) {
            const uint32_t i = lt + NL * q, t = i / RQ, d0 = 4u * (i % RQ);
            float *dst = vbuf[c % DPV_NBUF] + d0 * VST + t;
            dst[0] = v4[q].x;
            dst[VST] = v4[q].y;
            dst[2u * VST] = v4[q].z;
            dst[3u * VST] = v4[q].w;
        }
        if constexpr (PMEM) {
            if (lt < DPV_CH / 4u) *(v4f *)(pl + (c % DPV_NBUF) * DPV_CH + 4u * lt) = p4;
        }
    };
    if constexpr (!PMEM) {
        // The expf table, the scores (float4 lt + NL k of the row, index
        // clamped into the row's positions) and the first two chunks of V go
        // out first; the rest of V once the scores are in.
        const float4 *sc = (const float4 *)prow;
        const uint32_t n4 = (n_kv + 3u) / 4u;
        const float ninf = -__builtin_inff();
        float4 sv[KS];
        const uint64_t tv = mynah_exp2_tab[lane & 31u];
#pragma unroll
        for (int k = 0; k < KS; k++) {
            const uint32_t i = lt + NL * (uint32_t)k;
            sv[k] = sc[i < n4 ? i : n4 - 1u];
        }
        fetch(vr[0], pr[0], 0);
        fetch(vr[1], pr[1], 1);
        etab[lw][lane & 31u] = tv;                        // lanes l and l + 32 write the same value
        // Every column at once, no branch: positions at or past n_kv are
        // -inf, whose exponential is 0 and adds nothing to the sums.
        float m = ninf;
#pragma unroll
        for (int k = 0; k < KS; k++) {
            const uint32_t t = 4u * (lt + NL * (uint32_t)k);
            float4 v = sv[k];
            v.x = t < n_kv ? v.x : ninf;
            v.y = t + 1u < n_kv ? v.y : ninf;
            v.z = t + 2u < n_kv ? v.z : ninf;
            v.w = t + 3u < n_kv ? v.w : ninf;
            sv[k] = v;
            m = fmaxf(fmaxf(fmaxf(m, v.x), fmaxf(v.y, v.z)), v.w);
        }
        m = wave_max_dpp(m);
        if (lane == 0) wmax[lw] = m;
        __syncthreads();
        static_for<DPV_WIN - 2u>([&](auto w) __attribute__((always_inline)) {
            constexpr uint32_t W = decltype(w)::value + 2u;
            fetch(vr[W], pr[W], W);
        });
        m = wmax[0];
#pragma unroll
        for (uint32_t w = 1; w < DPV_LW; w++) m = fmaxf(m, wmax[w]);
        double acc = 0.0;
#pragma unroll
        for (int k = 0; k < KS; k++) {
            float4 e;
            e.x = mynah_expf_t(sv[k].x - m, etab[lw]);
            e.y = mynah_expf_t(sv[k].y - m, etab[lw]);
            e.z = mynah_expf_t(sv[k].z - m, etab[lw]);
            e.w = mynah_expf_t(sv[k].w - m, etab[lw]);
            sv[k] = e;
        }
#pragma unroll
        for (int k = 0; k < KS; k++) {
            acc += (double)sv[k].x;
            acc += (double)sv[k].y;
            acc += (double)sv[k].z;
            acc += (double)sv[k].w;
        }
        acc = wave_sum_d(acc);
        if (lane == 0) wsum[lw] = acc;
        __syncthreads();
        // The double sum of the four waves in wave order (the chain's wave
        // checks its reciprocal against the reference's index order).
        double lsum = wsum[0];
#pragma unroll
        for (uint32_t w = 1; w < DPV_LW; w++) lsum = lsum + wsum[w];
        const float inv = (float)(1.0 / lsum);
#pragma unroll
        for (int k = 0; k < KS; k++) {
            const uint32_t i = lt + NL * (uint32_t)k;
            if (i < n4) {
                const float4 e = sv[k];
                *(float4 *)(pl + 4u * i) = make_float4(e.x * inv, e.y * inv, e.z * inv, e.w * inv);
            }
        }
    } else {
        static_for<DPV_WIN>([&](auto w) __attribute__((always_inline)) {
            constexpr uint32_t W = decltype(w)::value;
            fetch(vr[W], pr[W], W);
        });
    }
    store(vr[0], pr[0], 0);
    store(vr[1], pr[1], 1);
    fetch(vr[0], pr[0], DPV_WIN);
    fetch(vr[1], pr[1], DPV_WIN + 1u);
    __syncthreads();
    // One barrier per chunk of the chain (nc in all); chunk c + 2 goes where
    // chunk c - 1 was and its slot takes chunk c + 2 + DPV_WIN. With the
    // probabilities in LDS the chunks are at most 4 KS and the steps are
    // written out one by one (a loop's back edge would make the compiler
    // wait for every fetch in flight at its head); otherwise a loop of
    // rounds of DPV_WIN steps, each slot index a constant.
    auto step = [&](auto wi, uint32_t c) __attribute__((always_inline)) {
        constexpr uint32_t S = (decltype(wi)::value + 2u) % DPV_WIN;
        store(vr[S], pr[S], c + 2u);
        fetch(vr[S], pr[S], c + 2u + DPV_WIN);
        __syncthreads();
    };
    if constexpr (!PMEM) {
        steps_until<0, 4u * NL * KS / DPV_CH>(nc, [&](auto ci) __attribute__((always_inline)) {
            constexpr uint32_t c = decltype(ci)::value;
            step(Index<c % DPV_WIN>{}, c);
        });
    } else {
        for (uint32_t c0 = 0;; c0 += DPV_WIN) {
            bool more = true;
            static_for<DPV_WIN>([&](auto wi) __attribute__((always_inline)) {
                const uint32_t c = c0 + decltype(wi)::value;
                if (more && c >= nc) more = false;
                if (more) step(wi, c);
            });
            if (!more) return;
        }
    }
}

#define DPV_KERNEL(PMEM, KS, NAME)                                                             \
    extern "C" __global__ void __launch_bounds__(64 * (1 + DPV_LW))                           \
    NAME(const float *v_layer, const float *sp, const uint32_t *__restrict__ pos_ptr,         \
         float *__restrict__ out, uint32_t sstride, uint32_t kv_dim, uint32_t n_kv_heads,     \
         uint32_t group) {                                                                    \
        attn_pv_body<PMEM, KS>(v_layer, sp, pos_ptr[0], out, sstride, kv_dim, n_kv_heads,     \
                               group);                                                        \
    }
// Probabilities in LDS: KS float4 of scores per loader thread cover n_ctx <= 256 DPV_LW KS.
DPV_KERNEL(false, 1, mynah_attn_pv_1)
DPV_KERNEL(false, 2, mynah_attn_pv_2)
DPV_KERNEL(false, 3, mynah_attn_pv_3)
DPV_KERNEL(false, 4, mynah_attn_pv_4)
// Probabilities from memory (any length).
DPV_KERNEL(true, 1, mynah_attn_pv_m)

// ── attention with the positions split across workgroups ───────────────────
// The same operations as mynah_attn_scores + mynah_attn_out, except that the
// softmax is taken per chunk of CH positions and the chunks are combined
// afterwards (the split form of src/kernels.c:228-250). mynah_attn_split:
// workgroup (kvh, c) computes the scores of positions c * CH .. for the
// group's query heads (same lane order as the reference dot), its chunk max
// m_c, e_t = expf(s_t - m_c), the double sum l_c of the e_t and the partial
// o_c = sum e_t v_t (fma chain in t order), and stores (m_c, l_c, o_c).
// mynah_attn_combine: M = max m_c, w_c = expf(m_c - M), inv = (float)(1 /
// sum_c w_c l_c), o = sum_c (w_c * inv) o_c in chunk order. Differences from
// the reference are f32 rounding of the exponentials and of the order of the
// weighted sum. Split: grid (n_kv_heads, ceil(n_ctx / CH)), block 128 *
// group; group <= 8, hd == 128. Partials: pm, pl [n_kv][nch_max][group], po
// [n_kv][nch_max][group][128].
// CH positions per workgroup; G query heads per key head fixed at compile
// time (block 128 G, K rows loaded in CH / (8 G) passes of 8 G rows), or
// G = 0: the group given at run time (2 .. 8, block 128 group, CH = 32).
template <uint32_t CH, uint32_t G>
MYNAH_DEV void attn_split_body(const float *__restrict__ q, float *__restrict__ k_layer,
                               const float *__restrict__ v_layer, const float *__restrict__ q_norm,
                               const float *__restrict__ k_norm, const float *__restrict__ rope_now,
                               const uint32_t *__restrict__ pos_ptr,
                               float *__restrict__ pm, double *__restrict__ pl, float *__restrict__ po,
                               uint32_t nch_max, uint32_t kv_dim, uint32_t group_rt, float eps,
                               float scale, uint32_t n_ctx, uint32_t spec_chunks) {
#pragma clang fp contract(off)
    constexpr uint32_t GM = G ? G : 8u;                       // most query heads per key head
    constexpr uint32_t G1 = G ? G : 1u;
    constexpr uint32_t PASSES = G ? CH / (8u * G1) : (CH + 15u) / 16u;
    constexpr uint32_t VR = G ? CH / (4u * G1) : (CH * 32u + 255u) / 256u;
    static_assert(G == 0 || (CH % (8u * G1) == 0 && CH % (4u * G1) == 0), "chunk and group");
    __shared__ __attribute__((aligned(16))) float qn[GM][128];
    __shared__ __attribute__((aligned(16))) float kn[128];
    __shared__ __attribute__((aligned(16))) float vs[CH][128];
    __shared__ __attribute__((aligned(16))) float es[GM][CH];
    __shared__ __attribute__((aligned(16))) float ee[GM][CH];
    const uint32_t group = G ? G : group_rt;
    const uint32_t pos = pos_ptr[0], n_kv = pos + 1u;
    const uint32_t kvh = blockIdx.x, c = blockIdx.y, t0 = c * CH;
    // Chunks below spec_chunks were live when the launch was enqueued and the
    // position only grows, so their K/V loads go out before the position
    // arrives; the others first learn whether they hold any position at all.
    const bool spec = c < spec_chunks;
    if (!spec && t0 >= n_kv) return;
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
    const uint32_t nthr = G ? 128u * G : blockDim.x;
    const uint32_t nw = nthr >> 6;                  // 2 * group waves
    // The K rows of the dot lanes and the V rows of the chunk are loaded
    // first (rows clamped into the cache; positions at or past pos are
    // masked below), then for wave w < group query head w with its norm
    // weights; after the position, the new key (wave group, when this chunk
    // holds pos) and the rotation of position pos.
    const uint32_t r = lane >> 4, l = lane & 15u;
    const uint32_t ppp = 4u * nw;                   // positions per pass
    float kv[PASSES][8];
#pragma unroll
    for (uint32_t ps = 0; ps < PASSES; ps++) {
        const uint32_t t = t0 + ppp * ps + 4u * wave + r;
        const uint32_t row = t < n_ctx ? t : n_ctx - 1u;
        const float *krow = k_layer + (size_t)row * kv_dim + (size_t)kvh * 128u + l;
#pragma unroll
        for (int j = 0; j < 8; j++) kv[ps][j] = krow[16 * j];
    }
    float4 vr[VR];
#pragma unroll
    for (uint32_t k = 0; k < VR; k++) {
        const uint32_t i = tid + nthr * k;
        const uint32_t tr = i >> 5, q4 = i & 31u, t = t0 + tr;
        const uint32_t row = t < n_ctx ? t : n_ctx - 1u;
        vr[k] = (G || i < CH * 32u)
                    ? *(const float4 *)(v_layer + (size_t)row * kv_dim + (size_t)kvh * 128u + 4u * q4)
                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    // The query heads, their norm weights and the rotation of the position
    // (rope_now: its cos and sin rows, copied there by the launch that set
    // the position) do not depend on the position's value either.
    const bool qwave = wave < group;
    float x0 = 0.0f, x1 = 0.0f, w0 = 0.0f, w1 = 0.0f, cs = 0.0f, sn = 0.0f;
    if (qwave) {
        const float *src = q + (size_t)(kvh * group + wave) * 128u;
        x0 = src[lane];
        x1 = src[lane + 64u];
        w0 = q_norm[lane];
        w1 = q_norm[lane + 64u];
    }
    if (wave <= group) {
        cs = rope_now[lane];
        sn = rope_now[64u + lane];
    }
    if (t0 >= n_kv) return;       // a speculative chunk past the position (after a reset)
    const bool has_pos = pos < t0 + CH;
#pragma unroll
    for (uint32_t k = 0; k < VR; k++) {
        const uint32_t t = t0 + ((tid + nthr * k) >> 5);
        if (t >= n_kv) vr[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    const bool kwave = wave == group && has_pos;
    float *kpos = k_layer + (size_t)pos * kv_dim + (size_t)kvh * 128u;
    if (kwave) {
        x0 = kpos[lane];
        x1 = kpos[lane + 64u];
        w0 = k_norm[lane];
        w1 = k_norm[lane + 64u];
    }
#pragma unroll
    for (uint32_t k = 0; k < VR; k++) {
        const uint32_t i = tid + nthr * k;
        if (G || i < CH * 32u) *(float4 *)(&vs[i >> 5][4u * (i & 31u)]) = vr[k];
    }
    if (qwave || kwave) {
        float y0, y1;
        // The wave's order of the sum of squares, unchecked: the split
        // attention rounds differently from the reference anyway.
        norm_rope_reg(x0, x1, w0, w1, cs, sn, eps, false, y0, y1);
        float *dst = qwave ? qn[wave] : kn;
        dst[lane] = y0;
        dst[lane + 64u] = y1;
        if (kwave) {
            kpos[lane] = y0;
            kpos[lane + 64u] = y1;
        }
    }
    __syncthreads();
    // Scores, reference dot order, into es[h][t - t0].
#pragma unroll
    for (uint32_t ps = 0; ps < PASSES; ps++) {
        const uint32_t tl = ppp * ps + 4u * wave + r, t = t0 + tl;
        if ((G || tl < CH) && t < n_kv) {
            float kk[8];
#pragma unroll
            for (int j = 0; j < 8; j++) kk[j] = t < pos ? kv[ps][j] : kn[16 * j + l];
#pragma unroll
            for (uint32_t h = 0; h < GM; h++) {
                if (G == 0 && h >= group) break;
                float acc = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; j++) acc = __builtin_fmaf(qn[h][16 * j + l], kk[j], acc);
                const float dot = row16_dot(acc);
                if (l == 0) es[h][tl] = dot * scale;
            }
        }
    }
    __syncthreads();
    // Chunk softmax: thread (h, d) with d < CH turns position d into e.
    const uint32_t h = tid >> 7, d = tid & 127u;
    const uint32_t tn = n_kv - t0 < CH ? n_kv - t0 : CH;
    float m = -__builtin_inff();
    if (h < group) {
#pragma unroll
        for (uint32_t k = 0; k < CH / 4; k++) {
            const float4 v = *(const float4 *)(&es[h][4 * k]);
            if (4u * k < tn) m = fmaxf(m, v.x);
            if (4u * k + 1u < tn) m = fmaxf(m, v.y);
            if (4u * k + 2u < tn) m = fmaxf(m, v.z);
            if (4u * k + 3u < tn) m = fmaxf(m, v.w);
        }
        if (d < CH) ee[h][d] = d < tn ? mynah_expf(es[h][d] - m) : 0.0f;
    }
    __syncthreads();
    // Partial weighted sum (fma chain in t order) and the chunk's exp sum.
    // Positions past n_kv have e = 0 and v = 0, so they leave both sums
    // unchanged; the exp sum runs as four interleaved double chains.
    if (h < group) {
        float o = 0.0f;
        double l4[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (uint32_t k = 0; k < CH / 4; k++) {
            const float4 e = *(const float4 *)(&ee[h][4 * k]);
            const float ev[4] = {e.x, e.y, e.z, e.w};
#pragma unroll
            for (uint32_t u = 0; u < 4; u++) {
                o = __builtin_fmaf(vs[4 * k + u][d], ev[u], o);
                l4[u] += (double)ev[u];
            }
        }
        const double lsum = (l4[0] + l4[1]) + (l4[2] + l4[3]);
        const size_t slot = ((size_t)kvh * nch_max + c) * group + h;
        po[slot * 128u + d] = o;
        if (d == 0) {
            pm[slot] = m;
            pl[slot] = lsum;
        }
    }
}

#define AS_ARGS                                                                                    \
    const float *__restrict__ q, float *__restrict__ k_layer, const float *__restrict__ v_layer,   \
        const float *__restrict__ q_norm, const float *__restrict__ k_norm,                        \
        const float *__restrict__ rope_now, const uint32_t *__restrict__ pos_ptr,                  \
        float *__restrict__ pm, double *__restrict__ pl, float *__restrict__ po, uint32_t nch_max, \
        uint32_t kv_dim, uint32_t group, float eps, float scale, uint32_t n_ctx,                   \
        uint32_t spec_chunks
#define AS_PASS_ARGS q, k_layer, v_layer, q_norm, k_norm, rope_now, pos_ptr, pm, pl, po, nch_max, \
                     kv_dim, group, eps, scale, n_ctx, spec_chunks

extern "C" __global__ void __launch_bounds__(1024) mynah_attn_split(AS_ARGS) {
    attn_split_body<AS_CH, 0>(AS_PASS_ARGS);
}
#define AS_KERNEL(G, CH)                                                                           \
    extern "C" __global__ void __launch_bounds__(128 * G) mynah_attn_split_g##G##_##CH(AS_ARGS) { \
        attn_split_body<CH, G>(AS_PASS_ARGS);                                                      \
    }
AS_KERNEL(2, 32)
AS_KERNEL(2, 64)
AS_KERNEL(2, 128)
AS_KERNEL(4, 32)
AS_KERNEL(4, 64)
AS_KERNEL(4, 128)

// Grid n_heads, block 256: four waves combine the chunks of one query head.
// Thread c (and c + 256, ...) takes chunk c's max and exp sum: M = max m_c,
// w_c = expf(m_c - M) (kept in LDS), L = sum_c w_c l_c in double (each
// wave's share, then the four shares in wave order); inv = (float)(1 / L).
// Up to 128 chunks wave 0 computes M and L alone (lane l holding chunks l
// and 64 + l; same values: its two double sums are the first two waves'
// sums, the others contribute -inf and 0.0), one barrier fewer. Wave w then sums o_w = fma(w_c * inv, o_c, o_w) over its chunks c = w,
// w + 4, ... in order, lane l holding dimensions l and l + 64, and the four
// partial vectors are added in wave order. The first AC_PRE chunks of every
// wave are loaded before the position arrives (every slot below nch_max is
// in bounds), so nearly all partials are in flight at once. Dynamic LDS:
// nch_max floats.
#define AC_WAVES 4
#define AC_PRE 16
extern "C" __global__ void __launch_bounds__(256)
mynah_attn_combine(const uint32_t *__restrict__ pos_ptr, const float *__restrict__ pm,
                   const double *__restrict__ pl, const float *__restrict__ po,
                   float *__restrict__ out, uint32_t nch_max, uint32_t group, uint32_t wave0_max,
                   uint32_t ch) {
#pragma clang fp contract(off)
    extern __shared__ float wsc[];
    __shared__ float smax[AC_WAVES];
    __shared__ double ssum[AC_WAVES];
    __shared__ float sinv;
    __shared__ float spart[AC_WAVES - 1][128];
    const uint32_t head = blockIdx.x, kvh = head / group, h = head - kvh * group;
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
    const size_t base = (size_t)kvh * nch_max * group + h;    // slot of chunk c: base + c * group
    const float *pob = po + base * 128u + lane;
    const size_t cstride = (size_t)group * 128u;
    float pv[AC_PRE][2];
#pragma unroll
    for (uint32_t k = 0; k < AC_PRE; k++) {
        const uint32_t c = wave + AC_WAVES * k;
        pv[k][0] = c < nch_max ? pob[(size_t)c * cstride] : 0.0f;
        pv[k][1] = c < nch_max ? pob[(size_t)c * cstride + 64u] : 0.0f;
    }
    // Chunk tid's max and exp sum, also in flight before the position.
    const float pm0 = tid < nch_max ? pm[base + (size_t)tid * group] : 0.0f;
    const double pl0 = tid < nch_max ? pl[base + (size_t)tid * group] : 0.0;
    // Wave 0 also holds chunk 64 + lane for the max and sum.
    const uint32_t c1 = 64u + lane;
    const float pm1 = wave == 0u && c1 < nch_max ? pm[base + (size_t)c1 * group] : 0.0f;
    const double pl1 = wave == 0u && c1 < nch_max ? pl[base + (size_t)c1 * group] : 0.0;
    const uint32_t n_kv = pos_ptr[0] + 1u, nch = (n_kv + ch - 1u) / ch;
    float inv;
    if (nch <= wave0_max) {          // wave0_max <= 128
        // Wave 0 alone finds M and L: lane l holds chunks l and 64 + l, whose
        // double sums are the combine's first two wave sums (the other
        // waves' maxima being -inf and their sums 0, added all the same).
        if (wave == 0u) {
            float m = -__builtin_inff();
            if (lane < nch) m = fmaxf(m, pm0);
            if (64u + lane < nch) m = fmaxf(m, pm1);
            const float M = wave_max_dpp(m);
            double l = 0.0, l1 = 0.0;
            if (lane < nch) {
                const float w = mynah_expf(pm0 - M);
                wsc[lane] = w;
                l += (double)w * pl0;
            }
            if (64u + lane < nch) {
                const float w = mynah_expf(pm1 - M);
                wsc[64u + lane] = w;
                l1 += (double)w * pl1;
            }
            l = wave_sum_d(l);
            l1 = wave_sum_d(l1);
            if (lane == 0) sinv = (float)(1.0 / (((l + l1) + 0.0) + 0.0));
        }
        __syncthreads();
        inv = sinv;
    } else {
        float m = -__builtin_inff();
        if (tid < nch) m = fmaxf(m, pm0);
        for (uint32_t c = tid + 256u; c < nch; c += 256u) m = fmaxf(m, pm[base + (size_t)c * group]);
        m = wave_max_f(m);
        if (lane == 0) smax[wave] = m;
        __syncthreads();
        const float M = fmaxf(fmaxf(smax[0], smax[1]), fmaxf(smax[2], smax[3]));
        double l = 0.0;
        if (tid < nch) {
            const float w = mynah_expf(pm0 - M);
            wsc[tid] = w;
            l += (double)w * pl0;
        }
        for (uint32_t c = tid + 256u; c < nch; c += 256u) {
            const float w = mynah_expf(pm[base + (size_t)c * group] - M);
            wsc[c] = w;
            l += (double)w * pl[base + (size_t)c * group];
        }
        l = wave_sum_d(l);
        if (lane == 0) ssum[wave] = l;
        __syncthreads();
        inv = (float)(1.0 / (((ssum[0] + ssum[1]) + ssum[2]) + ssum[3]));
    }
    float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < AC_PRE; k++) {     // static indices keep pv in registers
        const uint32_t c = wave + AC_WAVES * k;
        if (c < nch) {
            const float sc = wsc[c] * inv;
            o0 = __builtin_fmaf(sc, pv[k][0], o0);
            o1 = __builtin_fmaf(sc, pv[k][1], o1);
        }
    }
    uint32_t c = wave + AC_WAVES * AC_PRE;
    for (; c + AC_WAVES * 3u < nch; c += AC_WAVES * 4u) {
        float a[4], b[4];
#pragma unroll
        for (uint32_t u = 0; u < 4; u++) {
            a[u] = pob[(size_t)(c + AC_WAVES * u) * cstride];
            b[u] = pob[(size_t)(c + AC_WAVES * u) * cstride + 64u];
        }
#pragma unroll
        for (uint32_t u = 0; u < 4; u++) {
            const float sc = wsc[c + AC_WAVES * u] * inv;
            o0 = __builtin_fmaf(sc, a[u], o0);
            o1 = __builtin_fmaf(sc, b[u], o1);
        }
    }
    for (; c < nch; c += AC_WAVES) {
        const float sc = wsc[c] * inv;
        o0 = __builtin_fmaf(sc, pob[(size_t)c * cstride], o0);
        o1 = __builtin_fmaf(sc, pob[(size_t)c * cstride + 64u], o1);
    }
    if (wave > 0) {
        spart[wave - 1][lane] = o0;
        spart[wave - 1][lane + 64u] = o1;
    }
    __syncthreads();
    if (wave == 0) {
        o0 = ((o0 + spart[0][lane]) + spart[1][lane]) + spart[2][lane];
        o1 = ((o1 + spart[0][lane + 64u]) + spart[1][lane + 64u]) + spart[2][lane + 64u];
        out[(size_t)head * 128u + lane] = o0;
        out[(size_t)head * 128u + 64u + lane] = o1;
    }
}


// The combine of one query head without a barrier, for launches of at most
// MAXC chunks: the operations of mynah_attn_combine in the same order.
// Chunk c's max and exp sum sit in lane c % 64 (set c / 64) of every wave:
// M by wave maxima, L = ((s_0 + s_1) + 0.0) + 0.0 with s_k the wave's double
// sum over set k (the combine's per-wave sums; its third and fourth waves
// hold no chunk), then the four fma chains over the chunks c = 0, 1, 2, 3
// mod 4 with weights w_c * inv (read from their lanes), added in that order.
// DPL dimensions per lane: 2 (one wave per head, dimensions l and l + 64)
// or 1 (two waves, wave w dimension 64 w + l, each on its own). Every
// partial of the launch's chunks is loaded before the position arrives.
// Grid n_heads, block 128 / DPL.
template <int MAXC, int DPL>
MYNAH_DEV void attn_combine_waves(const uint32_t *__restrict__ pos_ptr, const float *__restrict__ pm,
                                  const double *__restrict__ pl, const float *__restrict__ po,
                                  float *__restrict__ out, uint32_t nch_max, uint32_t group,
                                  uint32_t ch) {
#pragma clang fp contract(off)
    constexpr uint32_t SETS = (MAXC + 63) / 64;
    const uint32_t head = blockIdx.x, kvh = head / group, h = head - kvh * group;
    const uint32_t lane = threadIdx.x & 63u, dim0 = DPL == 1 ? 64u * (threadIdx.x >> 6) : 0u;
    const size_t base = (size_t)kvh * nch_max * group + h;
    const float *pob = po + base * 128u + dim0 + lane;
    const size_t cstride = (size_t)group * 128u;
    float pv[MAXC][DPL];
    static_for<MAXC>([&](auto C) {
        constexpr uint32_t c = decltype(C)::value;
        static_for<DPL>([&](auto D) {
            constexpr uint32_t e = decltype(D)::value;
            pv[c][e] = c < nch_max ? pob[(size_t)c * cstride + 64u * e] : 0.0f;
        });
    });
    float pmv[SETS];
    double plv[SETS];
    static_for<SETS>([&](auto K) {
        constexpr uint32_t k = decltype(K)::value;
        const uint32_t c = 64u * k + lane;
        pmv[k] = c < nch_max ? pm[base + (size_t)c * group] : 0.0f;
        plv[k] = c < nch_max ? pl[base + (size_t)c * group] : 0.0;
    });
    const uint32_t n_kv = pos_ptr[0] + 1u, nch = (n_kv + ch - 1u) / ch;
    float m = -__builtin_inff();
    static_for<SETS>([&](auto K) {
        constexpr uint32_t k = decltype(K)::value;
        if (64u * k + lane < nch) m = fmaxf(m, pmv[k]);
    });
    const float M = wave_max_dpp(m);
    float w[SETS];
    double L = 0.0;
    static_for<SETS>([&](auto K) {
        constexpr uint32_t k = decltype(K)::value;
        double l = 0.0;
        w[k] = 0.0f;
        if (64u * k + lane < nch) {
            w[k] = mynah_expf(pmv[k] - M);
            l += (double)w[k] * plv[k];
        }
        const double sk = wave_sum_d(l);
        L = k == 0 ? sk : L + sk;
    });
    for (uint32_t k = SETS; k < 4u; k++) L = L + 0.0;
    const float inv = (float)(1.0 / L);
    float o[4][DPL];
    static_for<4>([&](auto K) {
        static_for<DPL>([&](auto D) { o[decltype(K)::value][decltype(D)::value] = 0.0f; });
    });
    static_for<MAXC>([&](auto C) {
        constexpr uint32_t c = decltype(C)::value;
        if (c < nch) {
            const float wc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w[c / 64u]), c % 64u));
            const float sc = wc * inv;
            static_for<DPL>([&](auto D) {
                constexpr uint32_t e = decltype(D)::value;
                o[c & 3u][e] = __builtin_fmaf(sc, pv[c][e], o[c & 3u][e]);
            });
        }
    });
    static_for<DPL>([&](auto D) {
        constexpr uint32_t e = decltype(D)::value;
        out[(size_t)head * 128u + dim0 + 64u * e + lane] = ((o[0][e] + o[1][e]) + o[2][e]) + o[3][e];
    });
}

// One wave per query head up to AC1_MAX chunks. (Two waves, one dimension
// per lane, up to 128 chunks, measured slower than the four-wave combine at
// the 4B's 69 chunks: 459 -> 452 tok/s.)
#define AC1_MAX 32                                 // = MYNAH_AC1_MAX (runtime_internal.h)
extern "C" __global__ void __launch_bounds__(64)
mynah_attn_combine1(const uint32_t *__restrict__ pos_ptr, const float *__restrict__ pm,
                    const double *__restrict__ pl, const float *__restrict__ po,
                    float *__restrict__ out, uint32_t nch_max, uint32_t group, uint32_t ch) {
    attn_combine_waves<AC1_MAX, 2>(pos_ptr, pm, pl, po, out, nch_max, group, ch);
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
    const float s = rms_scale_settled(block_sum_d(acc, sh), x, n, eps);
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) out[i] = x[i] * s * w[i];
}

// src/arch_qwen3.c:160-176: dequantise the 32 values of group c of
// embedding row `token` into x (no scaling). type 0 = f32 rows; otherwise
// the exact block decoders.
MYNAH_DEV void embed_group(const uint8_t *__restrict__ table, uint32_t token, float *__restrict__ x,
                           uint32_t c, uint32_t type, uint32_t row_bytes) {
#pragma clang fp contract(off)
    const uint8_t *row = table + (size_t)token * row_bytes;
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
    } else if (type == 13u) {
        // Q5_K: Q4_K's scales, quants at 48, fifth bits in qh[i] bit j.
        const uint8_t *blk = row + (c / 8u) * 176u;
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
            const uint32_t b = blk[48 + 32 * g + i];
            const uint32_t q = ((j & 1u) ? (b >> 4) : (b & 15u)) + (((blk[16 + i] >> j) & 1u) << 4);
            dst[i] = a * (float)q - o;
        }
    } else if (type == 2u) {
        // Q4_0 (kernels.c:2353-2360): d f16 @0, qs[16] @2; weight i is the low
        // nibble of qs[i] minus 8, weight i + 16 the high nibble minus 8.
        const uint8_t *blk = row + c * 18u;
        const float dd = f16_to_f32(blk[0] | (blk[1] << 8));
        for (int i = 0; i < 16; i++) {
            dst[i] = dd * ((float)(blk[2 + i] & 15u) - 8.0f);
            dst[i + 16] = dd * ((float)(blk[2 + i] >> 4) - 8.0f);
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

// src/sampler.c:122-129 finishes here: each workgroup of the head GEMV left
// one 64-bit key (orderable logit << 32 | ~row) for the first maximum of its
// rows; the largest key is the first index of the maximum logit. Appends it
// to tokens[step], advances pos and step (the reference's n_past++), picks
// the next token — forced[step + 1] while step + 1 < n_forced[0] (a prompt
// being prefilled, src/generate.c:13-86), the argmax after — and
// dequantises its embedding row into x for the next step
// (src/arch_qwen3.c:160-176). One workgroup.
extern "C" __global__ void __launch_bounds__(1024)
mynah_argmax_advance(const unsigned long long *__restrict__ keys, uint32_t n_keys,
                     uint32_t *__restrict__ token, uint32_t *__restrict__ tokens,
                     uint32_t *__restrict__ pos, uint32_t *__restrict__ step, uint32_t max_steps,
                     const uint8_t *__restrict__ table, float *__restrict__ x, uint32_t d,
                     uint32_t type, uint32_t row_bytes, const uint32_t *__restrict__ forced,
                     const uint32_t *__restrict__ n_forced, uint32_t vocab,
                     const float *__restrict__ rope_cos, const float *__restrict__ rope_sin,
                     float *__restrict__ rope_now) {
    __shared__ unsigned long long wk[16];
    __shared__ uint32_t sidx, spos;
    // The counters go out with the keys.
    uint32_t s = 0, nf = 0, p = 0;
    if (threadIdx.x == 0) {
        s = step[0];
        nf = n_forced[0];
        p = pos[0];
    }
    unsigned long long best = 0ull;
    for (uint32_t i = threadIdx.x; i < n_keys; i += blockDim.x) best = keys[i] > best ? keys[i] : best;
    best = wave_max_u64(best);
    if ((threadIdx.x & 63u) == 0) wk[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t k = 1; k < (blockDim.x + 63u) / 64u; k++) best = wk[k] > best ? wk[k] : best;
        const uint32_t idx = ~(uint32_t)(best & 0xffffffffull);
        uint32_t next = s + 1u < nf ? forced[s + 1u] : idx;
        if (next >= vocab) next = 0u;       // no keys (a prefill step) and nothing forced
        token[0] = next;
        if (s < max_steps) tokens[s] = idx;
        step[0] = s + 1u;
        pos[0] = p + 1u;
        sidx = next;
        spos = p + 1u;
    }
    __syncthreads();
    const uint32_t idx = sidx, np = spos;
    // The rotation of the next position for the next step's attention
    // (max_steps = the context length = the rope tables' rows).
    if (threadIdx.x < 64u && np < max_steps) {
        rope_now[threadIdx.x] = rope_cos[(size_t)np * 64u + threadIdx.x];
        rope_now[64u + threadIdx.x] = rope_sin[(size_t)np * 64u + threadIdx.x];
    }
    for (uint32_t c = threadIdx.x; c < d / 32u; c += blockDim.x) embed_group(table, idx, x, c, type, row_bytes);
}

// The embedding row of the current token into x (the first step of a
// sequence; later steps get theirs from mynah_argmax_advance). One thread per
// 32 values.
extern "C" __global__ void __launch_bounds__(DEC_WG)
mynah_embed_row(const uint8_t *__restrict__ table, const uint32_t *__restrict__ token_ptr,
                float *__restrict__ x, uint32_t d, uint32_t type, uint32_t row_bytes,
                const uint32_t *__restrict__ pos_ptr, const float *__restrict__ rope_cos,
                const float *__restrict__ rope_sin, float *__restrict__ rope_now, uint32_t n_ctx) {
    const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;   // 32-value group
    // The rotation of the current position, for the split attention.
    if (c < 64u) {
        const uint32_t p = pos_ptr[0];
        if (p < n_ctx) {
            rope_now[c] = rope_cos[(size_t)p * 64u + c];
            rope_now[64u + c] = rope_sin[(size_t)p * 64u + c];
        }
    }
    if (c >= d / 32u) return;
    embed_group(table, token_ptr[0], x, c, type, row_bytes);
}

// ── batched prompt prefill ─────────────────────────────────────────────────
// The prompt's tokens fill the cache T at a time (positions p0 .. p0 + T - 1)
// with the same operations, in the same order, as T decode steps: every
// value a kernel here writes is bit-identical to the one the decode step
// writes for that token (same device functions, same reduction orders).
// Rows are tokens: X[t][d], Q[t][q_dim], scores[t][head][sstride].

// Input RMSNorm of row t (src/kernels.c:118-128), reduced exactly as the
// fused norm of a grouped GEMV launch with blockDim.x threads (stage_x):
// thread i accumulates the float4s i, i + blockDim.x, ... in order, then
// block_sum_d. Grid: rows; the caller passes the decode launch's block size.
extern "C" __global__ void __launch_bounds__(1024)
mynah_rmsnorm_rows(const float *__restrict__ x, const float *__restrict__ w, float *__restrict__ out,
                   uint32_t cols, float eps) {
#pragma clang fp contract(off)
    __shared__ double shd[16];
    const float4 *x4 = (const float4 *)(x + (size_t)blockIdx.x * cols);
    const float4 *w4 = (const float4 *)w;
    float4 *o4 = (float4 *)(out + (size_t)blockIdx.x * cols);
    const uint32_t n4 = cols / 4u;
    double acc = 0.0;
#pragma unroll 4
    for (uint32_t q = threadIdx.x; q < n4; q += blockDim.x) {
        const float4 v = x4[q];
        acc = __builtin_fma((double)v.x, (double)v.x, acc);
        acc = __builtin_fma((double)v.y, (double)v.y, acc);
        acc = __builtin_fma((double)v.z, (double)v.z, acc);
        acc = __builtin_fma((double)v.w, (double)v.w, acc);
    }
    const float sc = rms_scale_settled(block_sum_d(acc, shd), x + (size_t)blockIdx.x * cols,
                                       cols, eps);
    for (uint32_t q = threadIdx.x; q < n4; q += blockDim.x) {
        float4 v = x4[q];
        const float4 wv = w4[q];
        v.x = v.x * sc * wv.x; v.y = v.y * sc * wv.y; v.z = v.z * sc * wv.z; v.w = v.w * sc * wv.w;
        o4[q] = v;
    }
}

// act = (g * sigmoid(g)) * u elementwise (src/kernels.c:193-205, the
// grouped GEMV's gate/up epilogue); act may alias g.
extern "C" __global__ void __launch_bounds__(256)
mynah_swiglu_rows(const float *g, const float *__restrict__ u, float *act, uint32_t n) {
#pragma clang fp contract(off)
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float gv = g[i];
    act[i] = gv * sigmoid_ref(gv) * u[i];
}

// Embedding rows of T tokens: grid (ceil(d / 32 / 256), T), one thread per
// 32 values (src/arch_qwen3.c:160-176).
extern "C" __global__ void __launch_bounds__(DEC_WG)
mynah_embed_rows(const uint8_t *__restrict__ table, const uint32_t *__restrict__ tokens,
                 float *__restrict__ x, uint32_t d, uint32_t type, uint32_t row_bytes) {
    const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= d / 32u) return;
    embed_group(table, tokens[blockIdx.y], x + (size_t)blockIdx.y * d, c, type, row_bytes);
}

// Per-head RMSNorm + RoPE of the T new tokens (src/arch_qwen3.c:209-218):
// grid (T, n_heads + n_kv_heads), one wave; head h < n_heads rotates query
// head h of row t in q, the others key head h - n_heads of position p0 + t in
// the layer's cache, both in place.
extern "C" __global__ void __launch_bounds__(64)
mynah_prefill_rope(float *__restrict__ q, float *__restrict__ k_layer,
                   const float *__restrict__ q_norm, const float *__restrict__ k_norm,
                   const float *__restrict__ rope_cos, const float *__restrict__ rope_sin,
                   uint32_t p0, uint32_t n_heads, uint32_t kv_dim, float eps) {
    __shared__ float tmp[128];
    const uint32_t t = blockIdx.x, h = blockIdx.y, pos = p0 + t;
    const float *cs = rope_cos + (size_t)pos * 64u, *sn = rope_sin + (size_t)pos * 64u;
    if (h < n_heads) {
        float *qh = q + ((size_t)t * n_heads + h) * 128u;
        head_norm_rope(qh, qh, q_norm, cs, sn, 128u, eps, tmp);
    } else {
        float *kh = k_layer + (size_t)pos * kv_dim + (size_t)(h - n_heads) * 128u;
        head_norm_rope(kh, kh, k_norm, cs, sn, 128u, eps, tmp);
    }
}

// Scores of PS_Q consecutive query rows q0 .. q0 + PS_Q - 1 (positions
// p0 + q0 + i) against a chunk of PS_POS positions, each lane one position:
// lane l of wave w holds the whole key row of position t = t0 + 64 w + l in
// registers and computes, for every (query, head) pair of the tile, the
// reference's AVX2 dot (src/kernels.c:39-62) in its own registers: the 16
// FMA chains a[i] = fma(q[16 j + i], k_t[16 j + i], a[i]) over j = 0..7 (a[i]
// is s0[i] for i < 8, s1[i - 8] otherwise), then tt[i] = a[i] + a[i + 8],
// v[i] = tt[i] + tt[i + 4], dot = (v0 + v1) + (v2 + v3) -- the operations of
// the decode kernel's 16-lane form (row16_dot), bit for bit. The query
// values are wave-uniform LDS reads; the scores of a wave are 64 consecutive
// floats. A query scores only positions up to its own. Grid (n_kv_heads,
// ceil((p0 + T) / PS_POS), ceil(T / PS_Q)), block 256; group <= 8.
#define PS_Q 16
#define PS_POS 256
extern "C" __global__ void __launch_bounds__(256)
mynah_prefill_scores(const float *__restrict__ qn, const float *__restrict__ k_layer,
                     float *__restrict__ scores, uint32_t p0, uint32_t T, uint32_t sstride,
                     uint32_t kv_dim, uint32_t group, float scale) {
#pragma clang fp contract(off)
    // Queries of the tile, [query][head][128]: PS_Q * group * 512 bytes of
    // dynamic LDS.
    extern __shared__ __attribute__((aligned(16))) float ql[];
    const uint32_t kvh = blockIdx.x, t0 = blockIdx.y * PS_POS, q0 = blockIdx.z * PS_Q;
    const uint32_t nq = T - q0 < PS_Q ? T - q0 : PS_Q;
    const uint32_t last = p0 + q0 + nq - 1u;          // position of the tile's last query
    if (t0 > last) return;
    const uint32_t n_heads = gridDim.x * group, q_dim = n_heads * 128u;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t tw = t0 + 64u * wave, t = tw + lane;
    // Rows past the tile's last query read row 0 (finite, never stored).
    const float4 *krow = (const float4 *)(k_layer + (size_t)(t <= last ? t : 0u) * kv_dim +
                                          (size_t)kvh * 128u);
    float4 k4[32];
    static_for<32>([&](auto I) { k4[decltype(I)::value] = krow[decltype(I)::value]; });
    for (uint32_t i = threadIdx.x; i < nq * group * 32u; i += blockDim.x) {
        const uint32_t qi = i / (group * 32u), rem = i % (group * 32u);
        *(float4 *)&ql[(qi * group + (rem >> 5)) * 128u + 4u * (rem & 31u)] =
            *(const float4 *)&qn[(size_t)(q0 + qi) * q_dim + (size_t)kvh * group * 128u + 4u * rem];
    }
    __syncthreads();
    for (uint32_t qi = 0; qi < nq; qi++) {
        const uint32_t pos = p0 + q0 + qi;
        if (tw > pos) continue;                         // wave-uniform
        float *srow = scores + (size_t)(q0 + qi) * n_heads * sstride;
        for (uint32_t h = 0; h < group; h++) {
            const float4 *qh = (const float4 *)&ql[(qi * group + h) * 128u];
            float a[16];
            static_for<16>([&](auto I) { a[decltype(I)::value] = 0.0f; });
            static_for<8>([&](auto J) {
                constexpr uint32_t j = decltype(J)::value;
                static_for<4>([&](auto M) {
                    constexpr uint32_t m = decltype(M)::value;
                    const float4 qv = qh[4u * j + m], kv = k4[4u * j + m];
                    a[4u * m + 0u] = __builtin_fmaf(qv.x, kv.x, a[4u * m + 0u]);
                    a[4u * m + 1u] = __builtin_fmaf(qv.y, kv.y, a[4u * m + 1u]);
                    a[4u * m + 2u] = __builtin_fmaf(qv.z, kv.z, a[4u * m + 2u]);
                    a[4u * m + 3u] = __builtin_fmaf(qv.w, kv.w, a[4u * m + 3u]);
                });
            });
            float tt[8];
            static_for<8>([&](auto I) {
                constexpr uint32_t i = decltype(I)::value;
                tt[i] = a[i] + a[i + 8u];
            });
            const float v0 = tt[0] + tt[4], v1 = tt[1] + tt[5], v2 = tt[2] + tt[6],
                        v3 = tt[3] + tt[7];
            const float dot = (v0 + v1) + (v2 + v3);
            if (t <= pos) srow[(size_t)(kvh * group + h) * sstride + t] = dot * scale;
        }
    }
}

// Softmax of query row t = blockIdx.x, head 4 blockIdx.y + wave (positions
// 0 .. p0 + t), written back over its scores: grid (T, ceil(n_heads / 4)),
// four waves, one row each.
extern "C" __global__ void __launch_bounds__(256)
mynah_prefill_softmax(float *scores, uint32_t p0, uint32_t sstride, uint32_t n_heads) {
    const uint32_t h = blockIdx.y * 4u + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (h >= n_heads) return;
    float *row = scores + ((size_t)blockIdx.x * n_heads + h) * sstride;
    softmax_any(row, p0 + blockIdx.x + 1u, row);
}

// Weighted V sums of PV_Q consecutive query rows for one key head
// (src/kernels.c:244-249): out[t][h][d] = fma(v_j[d], p_t,h[j], o) for
// j = 0 .. p0 + t in order, each chain one thread's register. Thread
// (d = tid % 128, c = tid / 128) owns the chains (query, head) = pairs
// c, c + 4, ... of the tile. Per chunk of PV_CH positions the probabilities
// (0 past each query's own last position, which leaves its chain unchanged:
// fma(v, 0, o) = o for finite v and o != -0, and o never becomes -0 from
// +0) and the V rows (rows past the tile's last position hold row 0, finite)
// are staged in LDS; the next chunk's V rows and probabilities are fetched
// into registers while this one is summed. Grid (n_kv_heads,
// ceil(T / PV_Q)), block 512.
#define PV_Q 8
#define PV_CH 64
// G = group (2 .. 8, the decoder's limits): each thread owns NPT = 2 G
// (query, head) pairs, all compile-time indices; pairs of a short last tile
// have probabilities 0 (their outputs are not stored).
template <uint32_t G>
MYNAH_DEV void prefill_pv_tile(const float *__restrict__ v_layer, const float *__restrict__ probs,
                               float *__restrict__ out, uint32_t p0, uint32_t T, uint32_t sstride,
                               uint32_t kv_dim, float (*pl)[PV_CH], float (*vl)[128]) {
#pragma clang fp contract(off)
    constexpr uint32_t NPT = PV_Q * G / 4u, NPR = PV_Q * G * PV_CH / 512u;
    const uint32_t kvh = blockIdx.x, q0 = blockIdx.y * PV_Q;
    const uint32_t nq = T - q0 < PV_Q ? T - q0 : PV_Q;
    const uint32_t npair = nq * G, n_heads = gridDim.x * G;
    const uint32_t tid = threadIdx.x, d = tid & 127u, c = tid >> 7;
    const uint32_t n_end = p0 + q0 + nq;            // positions of the last query
    const float *vbase = v_layer + (size_t)kvh * 128u;
    // V fetch role: float4 f = tid + 512 k of the chunk: row f / 32, column
    // 4 (f % 32); rows past n_end read row 0 (never used). Probability fetch
    // role: entry i = tid + 512 k of the chunk's PV_Q G x PV_CH (pair i /
    // PV_CH, position i % PV_CH), 0 past the pair's query or past npair.
    // Four named registers rather than an array: an array of float4 written
    // through the compile-time loop stays in private memory.
    float4 vr0, vr1, vr2, vr3;
    auto vr = [&](auto K) -> float4 & {
        constexpr uint32_t k = decltype(K)::value;
        if constexpr (k == 0) return vr0;
        else if constexpr (k == 1) return vr1;
        else if constexpr (k == 2) return vr2;
        else return vr3;
    };
    float pr_r[NPR];
    float o[NPT];
    static_for<NPT>([&](auto K) { o[decltype(K)::value] = 0.0f; });
    for (uint32_t t0 = 0; t0 < n_end; t0 += PV_CH) {
        if (t0 == 0) {
            static_for<4>([&](auto K) {
                constexpr uint32_t k = decltype(K)::value;
                const uint32_t f = tid + 512u * k, r = f >> 5;
                vr(K) = *(const float4 *)(vbase + (size_t)(r < n_end ? r : 0u) * kv_dim + 4u * (f & 31u));
            });
            static_for<NPR>([&](auto K) {
                constexpr uint32_t k = decltype(K)::value;
                const uint32_t i = tid + 512u * k, pr = i / PV_CH, t = i % PV_CH;
                const uint32_t qi = pr / G, h = pr % G;
                pr_r[k] = pr < npair && t < p0 + q0 + qi + 1u
                              ? probs[((size_t)(q0 + qi) * n_heads + kvh * G + h) * sstride + t]
                              : 0.0f;
            });
        }
        __syncthreads();
        static_for<4>([&](auto K) {
            constexpr uint32_t k = decltype(K)::value;
            const uint32_t f = tid + 512u * k;
            *(float4 *)&vl[f >> 5][4u * (f & 31u)] = vr(K);
        });
        static_for<NPR>([&](auto K) {
            constexpr uint32_t k = decltype(K)::value;
            const uint32_t i = tid + 512u * k;
            pl[i / PV_CH][i % PV_CH] = pr_r[k];
        });
        __syncthreads();
        const uint32_t t1 = t0 + PV_CH;
        if (t1 < n_end) {
            static_for<4>([&](auto K) {
                constexpr uint32_t k = decltype(K)::value;
                const uint32_t f = tid + 512u * k, r = t1 + (f >> 5);
                vr(K) = *(const float4 *)(vbase + (size_t)(r < n_end ? r : 0u) * kv_dim + 4u * (f & 31u));
            });
            static_for<NPR>([&](auto K) {
                constexpr uint32_t k = decltype(K)::value;
                const uint32_t i = tid + 512u * k, pr = i / PV_CH, t = t1 + i % PV_CH;
                const uint32_t qi = pr / G, h = pr % G;
                pr_r[k] = pr < npair && t < p0 + q0 + qi + 1u
                              ? probs[((size_t)(q0 + qi) * n_heads + kvh * G + h) * sstride + t]
                              : 0.0f;
            });
        }
        // Four positions per step (rounded up: the padding has p = 0).
        const uint32_t tn = n_end - t0 < PV_CH ? n_end - t0 : PV_CH;
        for (uint32_t j = 0; j < tn; j += 4) {
            const float v0 = vl[j][d], v1 = vl[j + 1][d], v2 = vl[j + 2][d], v3 = vl[j + 3][d];
            static_for<NPT>([&](auto K) {
                constexpr uint32_t k = decltype(K)::value;
                const float4 pp = *(const float4 *)&pl[c + 4u * k][j];
                float acc = o[k];
                acc = __builtin_fmaf(v0, pp.x, acc);
                acc = __builtin_fmaf(v1, pp.y, acc);
                acc = __builtin_fmaf(v2, pp.z, acc);
                o[k] = __builtin_fmaf(v3, pp.w, acc);
            });
        }
    }
    static_for<NPT>([&](auto K) {
        constexpr uint32_t k = decltype(K)::value;
        const uint32_t pr = c + 4u * k;
        if (pr < npair) {
            const uint32_t qi = pr / G, h = pr % G;
            out[((size_t)(q0 + qi) * n_heads + kvh * G + h) * 128u + d] = o[k];
        }
    });
}

extern "C" __global__ void __launch_bounds__(512)
mynah_prefill_pv(const float *__restrict__ v_layer, const float *__restrict__ probs,
                 float *__restrict__ out, uint32_t p0, uint32_t T, uint32_t sstride,
                 uint32_t kv_dim, uint32_t group) {
    __shared__ __attribute__((aligned(16))) float pl[PV_Q * 8][PV_CH];
    __shared__ __attribute__((aligned(16))) float vl[PV_CH][128];
    switch (group) {
    case 2u: prefill_pv_tile<2>(v_layer, probs, out, p0, T, sstride, kv_dim, pl, vl); break;
    case 3u: prefill_pv_tile<3>(v_layer, probs, out, p0, T, sstride, kv_dim, pl, vl); break;
    case 4u: prefill_pv_tile<4>(v_layer, probs, out, p0, T, sstride, kv_dim, pl, vl); break;
    case 5u: prefill_pv_tile<5>(v_layer, probs, out, p0, T, sstride, kv_dim, pl, vl); break;
    case 6u: prefill_pv_tile<6>(v_layer, probs, out, p0, T, sstride, kv_dim, pl, vl); break;
    case 7u: prefill_pv_tile<7>(v_layer, probs, out, p0, T, sstride, kv_dim, pl, vl); break;
    default: prefill_pv_tile<8>(v_layer, probs, out, p0, T, sstride, kv_dim, pl, vl); break;
    }
}
