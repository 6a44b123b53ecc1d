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

#include <stdlib.h>

static long env_long(const char *name, long dflt) {
    const char *e = getenv(name);
    return (e != NULL && e[0] != '\0') ? strtol(e, NULL, 10) : dflt;
}

/* The exact GEMM with its products on MFMA (gemm_mfma.hip): the default;
 * MYNAH_GEMM_MFMA=0 runs the VALU kernels of gemm_exact.hip instead (same
 * bits). A launch of at most one 64 x 64 tile per CU splits the
 * super-blocks over gridDim.z, up to MYNAH_GEMM_WGS_PER_CU (default 4)
 * workgroups per CU (MYNAH_GEMM_SPLIT=0 never, N at most N ways), and folds
 * the first split's running total and the later per-super-block sums in
 * order afterwards (mynah_gemm_fold). */
static int gemm_mfma_launch(mynah_device *d, int type, int ord, const void *w, size_t rows,
                            size_t cols, size_t rb, const float *x, float *y, size_t tokens,
                            const float *res, hipStream_t stream) {
    static const int kid[2][4] = {
        {MYNAH_K_Q4K_GEMM_MFMA, MYNAH_K_Q5K_GEMM_MFMA, MYNAH_K_Q6K_GEMM_MFMA,
         MYNAH_K_Q80_GEMM_MFMA},
        {MYNAH_K_Q4K_GEMM_MV_MFMA, MYNAH_K_Q5K_GEMM_MV_MFMA, MYNAH_K_Q6K_GEMM_MV_MFMA,
         MYNAH_K_Q80_GEMM_MV_MFMA}};
    const int ti = type == MYNAH_Q4_K ? 0 : type == MYNAH_Q5_K ? 1 : type == MYNAH_Q6_K ? 2 : 3;
    const uint32_t units = (uint32_t)(cols / 256);
    const unsigned gx = (unsigned)((rows + 63) / 64), gy = (unsigned)((tokens + 63) / 64);
    const uint64_t tiles = (uint64_t)gx * gy;
    uint32_t nz = 1;
    const char *env = getenv("MYNAH_GEMM_SPLIT");
    const long cap = env ? strtol(env, NULL, 10) : 64;
    const long per_cu = env_long("MYNAH_GEMM_WGS_PER_CU", 4);
    const uint64_t want = (uint64_t)(per_cu > 0 ? per_cu : 1) * (uint64_t)d->cus;
    if (!(ord == 1 && type == MYNAH_Q8_0) && cap > 1 && tiles <= (uint64_t)d->cus) {
        nz = (uint32_t)((want + tiles - 1) / tiles);
        if (nz > units) nz = units;
        if (nz > (uint32_t)cap) nz = (uint32_t)cap;
    }
    uint32_t r32 = (uint32_t)rows, c32 = (uint32_t)cols, t32 = (uint32_t)tokens,
             rb32 = (uint32_t)rb;
    if (nz <= 1) {
        float *part = NULL;
        void *args[] = {&w, &x, &y, &r32, &c32, &t32, &rb32, &res, &part};
        return mynah_launch3(d, kid[ord][ti], gx, gy, 1, 256, 0, stream, args);
    }
    const size_t n = rows * tokens, bytes = (size_t)units * n * sizeof(float);
    float *part = NULL;
    hipError_t e = hipMallocAsync((void **)&part, bytes, stream);
    if (e != hipSuccess) {
        mynah_set_error("hipMallocAsync(split-K partials, %zu bytes): %s", bytes,
                        hipGetErrorString(e));
        return -1;
    }
    void *args[] = {&w, &x, &y, &r32, &c32, &t32, &rb32, &res, &part};
    int rc = mynah_launch3(d, kid[ord][ti], gx, gy, nz, 256, 0, stream, args);
    if (rc == 0) {
        uint32_t u32 = units, first = units / nz;   /* the units of split 0 */
        void *fargs[] = {&part, &res, &y, &r32, &t32, &first, &u32};
        rc = mynah_launch(d, MYNAH_K_GEMM_FOLD, (unsigned)((n + 255) / 256), 1, 256, 0, stream,
                          fargs);
    }
    e = hipFreeAsync(part, stream);
    if (rc == 0 && e != hipSuccess) {
        mynah_set_error("hipFreeAsync(split-K partials): %s", hipGetErrorString(e));
        return -1;
    }
    return rc;
}

static int gemm_mfma_on(void) {
    const char *env = getenv("MYNAH_GEMM_MFMA");
    return env == NULL || env[0] != '0';
}

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
    if (type == MYNAH_Q4_0) return mynah_q40_launch(d, w, rows, cols, x, y, tokens, NULL, stream);
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
    if (gemm_mfma_on())
        return gemm_mfma_launch(d, type, 0, w, rows, cols, rb, x, y, tokens, NULL, stream);
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
    /* Q4_0's matvec and batched product share one order (a single running
     * sum per output, kernels.c:2467-2484, generic.c:76-93): the batched
     * chains are the matvec-order GEMM. */
    if (type == MYNAH_Q4_0) {
        if (tokens == 0 || tokens > 0xffffffffu) {
            mynah_set_error("matvec-order GEMM needs 1 <= tokens < 2^32");
            return -1;
        }
        return mynah_q40_launch(d, w, rows, cols, x, y, tokens, res, stream);
    }
    if (cols % 256 != 0 || tokens == 0 || tokens > 0xffffffffu || rb > 0xffffffffu) {
        mynah_set_error("matvec-order GEMM needs cols %% 256 == 0 and 1 <= tokens < 2^32");
        return -1;
    }
    if (((uintptr_t)x & 15u) != 0 || mynah_w_misaligned(type, w)) {
        mynah_set_error("misaligned operand for the matvec-order GEMM");
        return -1;
    }
    if (gemm_mfma_on())
        return gemm_mfma_launch(d, type, 1, w, rows, cols, rb, x, y, tokens, res, stream);
    const int k = type == MYNAH_Q4_K   ? MYNAH_K_Q4K_GEMM_MV
                  : type == MYNAH_Q5_K ? MYNAH_K_Q5K_GEMM_MV
                  : type == MYNAH_Q6_K ? MYNAH_K_Q6K_GEMM_MV
                                       : MYNAH_K_Q80_GEMM_MV;
    uint32_t r32 = (uint32_t)rows, c32 = (uint32_t)cols, t32 = (uint32_t)tokens, rb32 = (uint32_t)rb;
    void *args[] = {&w, &x, &y, &r32, &c32, &t32, &rb32, &res};
    return mynah_launch(d, k, (unsigned)((rows + 63) / 64), (unsigned)((tokens + 63) / 64), 256, 0,
                        stream, args);
}
