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
