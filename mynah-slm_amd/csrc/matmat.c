/* matmat.c — batched Y[tokens][rows] = X[tokens][cols] · W^T.
 *
 * Replaces ingot_matmat (third_party/ingot/src/generic.c:107-124) and the
 * per-type batched kernels (kernels.c:1742-1751, 2597-2606, 2627-2648). Exact f32 for
 * every width unless the int8 lane is on (int8.c), like the reference's exact
 * path: the tiled kernel of
 * gemm_exact.hip keeps the batched reference's own summation order (natural
 * weight order per 256-value unit, kernels.c:1017-1039 and 2635-2648), so
 * every output is bit-identical to ingot's exact matmat. tokens == 1 is the
 * matvec, as in the reference (kernels.c:1726); the callers route it.
 *
 * SPDX-License-Identifier: MIT */
#include "kernels_hip.h"
#include "runtime_internal.h"

int mynah_matmat_launch(mynah_device *d, int type, const void *w, size_t rows, size_t cols,
                        const float *x, float *y, size_t tokens, int exact, hipStream_t stream) {
    size_t rb;
    if (mynah_geometry(type, rows, cols, &rb) != 0) return -1;
    /* The batched Q4_K and Q5_K products take the int8 lane when it is on,
     * exactly where the reference's do (kernels.c:1723-1751, 2573-2595;
     * tokens >= 2). */
    if (!exact && (type == MYNAH_Q4_K || type == MYNAH_Q5_K) && tokens >= 2 &&
        mynah_int8_mode() != MYNAH_INT8_OFF)
        return mynah_int8_product(d, type, w, rows, cols, x, y, tokens, stream);
    /* Q4_0 has no batched kernel in the reference: its generic path runs the
     * matvec's chain per token (generic.c:76-93), and so does this one. */
    if (type == MYNAH_Q4_0) return mynah_q40_launch(d, w, rows, cols, x, y, tokens, stream);
    /* The reference's batched core works in 256-wide units for every type
     * and refuses anything else (kernels.c:1087-1088, 2641-2648). */
    if (cols % 256 != 0) {
        mynah_set_error("batched matmat needs cols to be a multiple of 256");
        return -1;
    }
    if (tokens == 0 || tokens > 0xffffffffu || rb > 0xffffffffu) {
        mynah_set_error("bad token count");
        return -1;
    }
    if (((uintptr_t)x & 15u) != 0 || mynah_w_misaligned(type, w)) {
        mynah_set_error("misaligned operand for the batched GEMM");
        return -1;
    }
    const int k = type == MYNAH_Q4_K   ? MYNAH_K_Q4K_GEMM
                  : type == MYNAH_Q5_K ? MYNAH_K_Q5K_GEMM
                  : type == MYNAH_Q6_K ? MYNAH_K_Q6K_GEMM
                                       : MYNAH_K_Q80_GEMM;
    uint32_t r32 = (uint32_t)rows, c32 = (uint32_t)cols, t32 = (uint32_t)tokens, rb32 = (uint32_t)rb;
    void *args[] = {&w, &x, &y, &r32, &c32, &t32, &rb32};
    return mynah_launch(d, k, (unsigned)((rows + 63) / 64), (unsigned)((tokens + 63) / 64), 256, 0,
                        stream, args);
}

int mynah_matmat_mv_launch(mynah_device *d, int type, const void *w, size_t rows, size_t cols,
                           const float *x, float *y, size_t tokens, const float *res,
                           hipStream_t stream) {
    size_t rb;
    if (mynah_geometry(type, rows, cols, &rb) != 0) return -1;
    if (type == MYNAH_Q4_0) {
        mynah_set_error("no matvec-order GEMM for Q4_0");
        return -1;
    }
    if (cols % 256 != 0 || tokens == 0 || tokens > 0xffffffffu || rb > 0xffffffffu) {
        mynah_set_error("matvec-order GEMM needs cols %% 256 == 0 and 1 <= tokens < 2^32");
        return -1;
    }
    if (((uintptr_t)x & 15u) != 0 || mynah_w_misaligned(type, w)) {
        mynah_set_error("misaligned operand for the matvec-order GEMM");
        return -1;
    }
    const int k = type == MYNAH_Q4_K   ? MYNAH_K_Q4K_GEMM_MV
                  : type == MYNAH_Q5_K ? MYNAH_K_Q5K_GEMM_MV
                  : type == MYNAH_Q6_K ? MYNAH_K_Q6K_GEMM_MV
                                       : MYNAH_K_Q80_GEMM_MV;
    uint32_t r32 = (uint32_t)rows, c32 = (uint32_t)cols, t32 = (uint32_t)tokens, rb32 = (uint32_t)rb;
    void *args[] = {&w, &x, &y, &r32, &c32, &t32, &rb32, &res};
    return mynah_launch(d, k, (unsigned)((rows + 63) / 64), (unsigned)((tokens + 63) / 64), 256, 0,
                        stream, args);
}
