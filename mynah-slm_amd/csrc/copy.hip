// copy.hip — a plain streaming device copy (16-byte vector loads and stores).
//
// It is the yardstick for the HBM traffic counters: FETCH_SIZE and WRITE_SIZE
// of a copy of known size give the factor that turns the counters of the GEMV
// kernels into bytes.
//
// SPDX-License-Identifier: MIT
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

extern "C" __global__ void __launch_bounds__(256)
mynah_copy16(const uint4 *__restrict__ src, uint4 *__restrict__ dst, uint64_t n16) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
        dst[i] = src[i];
}

// A read-only stream: every 16-byte chunk of src is loaded once and folded
// into a per-thread XOR, written only in the (practically impossible) case
// that all its bits are set, so the kernel moves the bytes a GEMV reads and
// almost nothing else: the yardstick of what one launch can read at a size.
// Four loads per thread are in flight at a time.
extern "C" __global__ void __launch_bounds__(256)
mynah_read16(const uint4 *__restrict__ src, uint64_t n16, uint32_t *__restrict__ sink) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint4 acc = {0u, 0u, 0u, 0u};
    for (; i + 3u * stride < n16; i += 4u * stride) {
        const uint4 a = src[i], b = src[i + stride], c = src[i + 2u * stride],
                    e = src[i + 3u * stride];
        acc.x ^= a.x ^ b.x ^ c.x ^ e.x;
        acc.y ^= a.y ^ b.y ^ c.y ^ e.y;
        acc.z ^= a.z ^ b.z ^ c.z ^ e.z;
        acc.w ^= a.w ^ b.w ^ c.w ^ e.w;
    }
    for (; i < n16; i += stride) {
        const uint4 a = src[i];
        acc.x ^= a.x;
        acc.y ^= a.y;
        acc.z ^= a.z;
        acc.w ^= a.w;
    }
    if ((acc.x & acc.y & acc.z & acc.w) == 0xffffffffu) sink[0] = acc.x ^ acc.y;
}

// y[i] = expf(x[i]) with the reference's C library bits (mynah_expf.h), for
// callers that compute softmaxes beside the library and for its tests.
extern "C" __global__ void __launch_bounds__(256)
mynah_expf_map(const float *__restrict__ x, float *__restrict__ y, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        y[i] = mynah_expf(x[i]);
}

// The VALU yardstick: every lane runs eight independent chains of `iters`
// dependent v_add_f32 (non-packed), so with eight waves per SIMD the SIMD
// issues nothing but f32 adds: the time per wave64 add is what the exact
// summation orders (one add per product, in a fixed order) pay per product.
// The result is stored only in the (impossible) case that it equals `never`.
extern "C" __global__ void __launch_bounds__(256)
mynah_valu_add_rate(uint32_t iters, float c, float never, float *__restrict__ sink) {
#pragma clang fp contract(off)
    float a[8];
#pragma unroll
    for (int i = 0; i < 8; i++) a[i] = (float)threadIdx.x * 0.001f + (float)i;
    for (uint32_t it = 0; it < iters; it++) {
#pragma unroll
        for (int i = 0; i < 8; i++) a[i] = a[i] + c;
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) s = s + a[i];
    if (s == never) sink[0] = s;
}
