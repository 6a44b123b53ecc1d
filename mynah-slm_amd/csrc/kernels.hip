// kernels.hip — the one gfx950 code object of the library (every kernel
// translation unit is included here and compiled by a single hipcc --genco).
//
// SPDX-License-Identifier: MIT
#include "dequant.hip"
#include "gemv_exact.hip"
#include "gemv_pc.hip"
#include "gemv_stream.hip"
#include "gemv_q40.hip"
#include "gemv_fast.hip"
#include "gemm_exact.hip"
#include "gemm_mfma.hip"
#include "decode.hip"
#include "sample.hip"
#include "copy.hip"
#include "int8.hip"
