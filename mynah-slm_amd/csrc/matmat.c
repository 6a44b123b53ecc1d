/* matmat.c — batched Y[tokens][rows] = X[tokens][cols] · W^T.
 *
 * Replaces ingot_matmat (third_party/ingot/src/generic.c:107-124) and the
 * per-type batched kernels (kernels.c:1742-1751, 2627-2648). Exact f32 for
 * every width, like the reference's exact path.
 *
 * This form runs the exact GEMV once per token in the batched reference's own
 * summation order (natural weight order per 256-value unit, kernels.c:1017-
 * 1039 and 2635-2648), so every output is bit-identical to ingot's exact
 * matmat; tokens == 1 is the matvec, as in the reference (kernels.c:1726).
 *
 * SPDX-License-Identifier: MIT */
#include "runtime_internal.h"

int mynah_matmat_launch(mynah_device *d, int type, const void *w, size_t rows, size_t cols,
                        const float *x, float *y, size_t tokens, hipStream_t stream) {
    size_t rb;
    if (mynah_geometry(type, rows, cols, &rb) != 0) return -1;
    /* The reference's batched core works in 256-wide units for every type
     * and refuses anything else (kernels.c:1087-1088, 2641-2648). */
    if (cols % 256 != 0) {
        mynah_set_error("batched matmat needs cols to be a multiple of 256");
        return -1;
    }
    for (size_t t = 0; t < tokens; t++) {
        if (mynah_gemv_seq_launch(d, type, w, rows, cols, x + t * cols, y + t * rows, stream) != 0)
            return -1;
    }
    return 0;
}
