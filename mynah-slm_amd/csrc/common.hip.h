// common.hip.h — device helpers shared by the gfx950 kernels.
//
// SPDX-License-Identifier: MIT
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

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

// Workgroup-wide double sum; every thread gets the result. `sh` holds one
// double per wave (blockDim.x <= 1024).
MYNAH_DEV double block_sum_d(double v, double *sh) {
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    double t = 0.0;
    const uint32_t nw = (blockDim.x + 63u) >> 6;
    for (uint32_t k = 0; k < nw; k++) t += sh[k];
    return t;
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
MYNAH_DEV unsigned long long argmax_key(float v, uint32_t index) {
    uint32_t b = __float_as_uint(v == 0.0f ? 0.0f : v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((unsigned long long)b << 32) | (unsigned long long)(~index);
}
