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

// y[i] = expf(x[i]) with the reference's C library bits (mynah_expf.h), for
// callers that compute softmaxes beside the library and for its tests.
extern "C" __global__ void __launch_bounds__(256)
mynah_expf_map(const float *__restrict__ x, float *__restrict__ y, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        y[i] = mynah_expf(x[i]);
}
