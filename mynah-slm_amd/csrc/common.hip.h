// common.hip.h — device helpers shared by the gfx950 kernels.
//
// SPDX-License-Identifier: MIT
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mynah_expf.h"
#include "sum_settle.h"

#define MYNAH_DEV static __device__ __forceinline__

// Exact f16 -> f32 (v_cvt_f32_f16; HIP keeps f16 subnormals by default).
MYNAH_DEV float f16_to_f32(uint32_t bits16) {
    const unsigned short s = (unsigned short)(bits16 & 0xffffu);
    _Float16 h;
    __builtin_memcpy(&h, &s, 2);
    return (float)h;
}

// Byte K of a dword as float: one v_cvt_f32_ubyte{K}. Written as inline asm
// because the compiler otherwise folds a preceding nibble mask into a v_bfe
// and converts byte 0, which costs an extra instruction per weight.
template <int K>
MYNAH_DEV float ubyte_f(uint32_t v) {
    float r;
    if (K == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(r) : "v"(v));
    else if (K == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(r) : "v"(v));
    else if (K == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(r) : "v"(v));
    else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// ubyte_f (ASM) or the plain conversion (the backend picks the instruction).
// Kernels with MFMA take the plain form: inline asm in a kernel makes the
// compiler keep MFMA results in the accumulation registers, which costs a
// v_accvgpr_read per result before it can be used.
template <bool ASM, int K>
MYNAH_DEV float ubyte_sel(uint32_t v) {
    if constexpr (ASM) return ubyte_f<K>(v);
    else return (float)((v >> (8 * K)) & 0xffu);
}

// Byte k of a dword as float (plain C; the backend picks the conversion).
MYNAH_DEV float byte_f(uint32_t v, int k) { return (float)((v >> (8 * k)) & 0xffu); }

// {hi:lo} >> (8 * shift), low dword (v_alignbyte_b32).
MYNAH_DEV uint32_t align_bytes(uint32_t hi, uint32_t lo, uint32_t shift) {
    return __builtin_amdgcn_alignbyte(hi, lo, shift);
}

// Sum over the 8 lanes of an aligned 8-lane group (xor butterfly).
MYNAH_DEV float group8_sum(float v) {
    v += __shfl_xor(v, 1, 64);
    v += __shfl_xor(v, 2, 64);
    v += __shfl_xor(v, 4, 64);
    return v;
}

MYNAH_DEV float wave_sum(float v) {
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// A double moved across lanes by one DPP control (both halves).
template <int CTRL>
MYNAH_DEV double dpp_d(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)b, CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(b >> 32), CTRL, 0xf, 0xf, false);
    return __longlong_as_double(((long long)hi << 32) | (long long)(unsigned)lo);
}

MYNAH_DEV double readlane_d(double v, int lane) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)b, lane);
    const int hi = __builtin_amdgcn_readlane((int)(b >> 32), lane);
    return __longlong_as_double(((long long)hi << 32) | (long long)(unsigned)lo);
}

// Positions per workgroup of the generic split decode attention (= MYNAH_AS_CH
// in runtime_internal.h).
#define AS_CH 32

// Wave-wide float max (all lanes get the result).
MYNAH_DEV float wave_max_f(float v) {
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}

// Calls f(Index<0>), ..., f(Index<N - 1>): register arrays indexed by
// these stay in registers from the start (no loop to unroll first).
template <uint32_t I> struct Index { static constexpr uint32_t value = I; };
template <uint32_t N, class F>
MYNAH_DEV void static_for(F &&f) {
    if constexpr (N > 0) {
        static_for<N - 1>(f);
        f(Index<N - 1>{});
    }
}

// A float moved across lanes by one DPP control.
template <int CTRL>
MYNAH_DEV float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Wave-wide float max by DPP within rows, then the four row maxima (a max
// is the same in any order).
MYNAH_DEV float wave_max_dpp(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x124>(v));
    v = fmaxf(v, dpp_f<0x128>(v));
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// A 64-bit key moved across lanes by one DPP control (both halves).
template <int CTRL>
MYNAH_DEV unsigned long long dpp_u64(unsigned long long v) {
    const unsigned lo = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)v, CTRL, 0xf, 0xf, false);
    const unsigned hi =
        (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)(v >> 32), CTRL, 0xf, 0xf, false);
    return ((unsigned long long)hi << 32) | lo;
}

MYNAH_DEV unsigned long long readlane_u64(unsigned long long v, int lane) {
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)v, lane);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(v >> 32), lane);
    return ((unsigned long long)hi << 32) | lo;
}

// Wave-wide 64-bit max of a fully active wave, every lane receiving it: DPP
// within quads and rows, then the four row maxima read as scalars (no LDS
// round trip, unlike wave_max_u64's shuffles).
MYNAH_DEV unsigned long long wave_max_u64_dpp(unsigned long long v) {
    unsigned long long o = dpp_u64<0xB1>(v);
    v = o > v ? o : v;
    o = dpp_u64<0x4E>(v);
    v = o > v ? o : v;
    o = dpp_u64<0x124>(v);
    v = o > v ? o : v;
    o = dpp_u64<0x128>(v);
    v = o > v ? o : v;
    const unsigned long long a = readlane_u64(v, 0), b = readlane_u64(v, 16);
    const unsigned long long c = readlane_u64(v, 32), d = readlane_u64(v, 48);
    const unsigned long long ab = a > b ? a : b, cd = c > d ? c : d;
    return ab > cd ? ab : cd;
}

// Sum over the 64 lanes of a (fully active) wave in double, every lane
// receiving the total: DPP within quads (xor 1, xor 2) and rows (rotate by
// 4, 8), then the four row sums read as scalars.
MYNAH_DEV double wave_sum_d(double v) {
    v += dpp_d<0xB1>(v);     // quad_perm(1, 0, 3, 2)
    v += dpp_d<0x4E>(v);     // quad_perm(2, 3, 0, 1)
    v += dpp_d<0x124>(v);    // row_ror:4
    v += dpp_d<0x128>(v);    // row_ror:8
    return ((readlane_d(v, 0) + readlane_d(v, 16)) + readlane_d(v, 32)) + readlane_d(v, 48);
}

// Workgroup-wide double sum; every thread gets the result. `sh` holds one
// double per wave (blockDim.x <= 1024) and is written with no barrier in
// front: a kernel calls this at most once per `sh` (every caller does).
MYNAH_DEV double block_sum_d(double v, double *sh) {
    v = wave_sum_d(v);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    double t = 0.0;
    const uint32_t nw = (blockDim.x + 63u) >> 6;
    for (uint32_t k = 0; k < nw; k++) t += sh[k];
    return t;
}

// ── the reference's double sums, from a parallel order ─────────────────────
// The test that keeps a parallel-order double sum, and when it holds, is in
// sum_settle.h. mynah_index_sums != 0 makes every such sum take the
// index-order path (a test switch: mynah_hip_set_index_order_sums).
// The hot kernels read it once, early, beside their other first loads
// (index_sums_forced), and hand it to every test; protected visibility
// addresses it directly, without a load of its address first.
extern "C" {
__device__ __attribute__((used, visibility("protected"))) uint32_t mynah_index_sums;
}

MYNAH_DEV uint32_t index_sums_forced() { return mynah_index_sums; }

// The test on r's bits (every lane holds the same r), in the vector unit.
MYNAH_DEV bool sum_settled(double r, uint32_t n, uint32_t k2, uint32_t forced) {
    const uint64_t bits = (uint64_t)__double_as_longlong(r);
    return (forced == 0u) & (mynah_sum_settled((uint32_t)(bits >> 32), (uint32_t)bits, n, k2) != 0);
}

// The branch to a sum's index-order path, marked unlikely so that the path
// is laid out after the kernel's main path, which stays one straight run of
// code (a taken branch over it would start a new instruction fetch).
#define MYNAH_UNSETTLED(r, n, k2, forced) __builtin_expect(!sum_settled((r), (n), (k2), (forced)), 0)

// src/kernels.c:119-120 itself: the squares of x[0 .. n) added in index
// order. Every calling lane computes the whole sum (the addresses are the
// same across the wave, so each load is one broadcast).
MYNAH_DEV double seq_sumsq(const float *x, uint32_t n) {
#pragma clang fp contract(off)
    double acc = 0.0;
#pragma nounroll
    for (uint32_t i = 0; i < n; i++) acc += (double)x[i] * (double)x[i];
    return acc;
}

// src/kernels.c:213-217's sum itself: e[0 .. n) added in index order, by
// every calling lane.
MYNAH_DEV double seq_sum(const float *e, uint32_t n) {
#pragma clang fp contract(off)
    double acc = 0.0;
#pragma nounroll
    for (uint32_t i = 0; i < n; i++) acc += (double)e[i];
    return acc;
}

// src/kernels.c:121 before its conversion to f32.
MYNAH_DEV double rms_inv(double sum, uint32_t n, float eps) {
#pragma clang fp contract(off)
    return 1.0 / sqrt(sum / (double)n + (double)eps);
}

// The RMS scale (float)(1 / sqrt(sum / n + eps)) of x[0 .. n) as the
// reference computes it, from the sum of squares `sum` in a parallel order;
// x is read again only when that sum cannot settle it.
MYNAH_DEV float rms_scale_settled(double sum, const float *x, uint32_t n, float eps) {
    double r = rms_inv(sum, n, eps);
    if (MYNAH_UNSETTLED(r, n, 1u, index_sums_forced())) r = rms_inv(seq_sumsq(x, n), n, eps);
    return (float)r;
}

MYNAH_DEV unsigned long long wave_max_u64(unsigned long long v) {
    for (int m = 32; m >= 1; m >>= 1) {
        const unsigned long long o = __shfl_xor(v, m, 64);
        v = o > v ? o : v;
    }
    return v;
}

// Key ordering logits like the reference's greedy choice (src/sampler.c:
// 124-129): a larger value wins, and among equal values the smaller index
// (hence ~index in the low word). -0 is folded onto +0 so they compare equal.
// The reference starts from logits[0] and moves on a strict `>`, so a NaN
// is never picked past index 0, and a NaN at index 0 is never left (no
// comparison with it holds): NaN keys are 0 (below every number's key, all
// of which are > 0) except at index 0, whose NaN key is the largest key.
MYNAH_DEV unsigned long long argmax_key(float v, uint32_t index) {
    if (v != v) return index == 0u ? ~0ull : 0ull;
    uint32_t b = __float_as_uint(v == 0.0f ? 0.0f : v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)b << 32) | (unsigned long long)(~index);
}
