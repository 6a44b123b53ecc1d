/* runtime_internal.h — shared by the C11 host files of the library.
 *
 * SPDX-License-Identifier: MIT */
#ifndef MYNAH_RUNTIME_INTERNAL_H
#define MYNAH_RUNTIME_INTERNAL_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

enum { MYNAH_Q8_0 = 8, MYNAH_Q4_K = 12, MYNAH_Q6_K = 14 };

/* Every kernel of the embedded code object: id and symbol name. */
#define MYNAH_KERNEL_LIST(X)                          \
    X(MYNAH_K_Q4K_R1, "mynah_q4k_gemv_r1")            \
    X(MYNAH_K_Q4K_R2, "mynah_q4k_gemv_r2")            \
    X(MYNAH_K_Q4K_R4, "mynah_q4k_gemv_r4")            \
    X(MYNAH_K_Q6K_R1, "mynah_q6k_gemv_r1")            \
    X(MYNAH_K_Q6K_R2, "mynah_q6k_gemv_r2")            \
    X(MYNAH_K_Q6K_R4, "mynah_q6k_gemv_r4")            \
    X(MYNAH_K_Q80_R1, "mynah_q80_gemv_r1")            \
    X(MYNAH_K_Q80_R2, "mynah_q80_gemv_r2")            \
    X(MYNAH_K_Q80_R4, "mynah_q80_gemv_r4")            \
    X(MYNAH_K_DEQUANT, "mynah_dequant")                 \
    X(MYNAH_K_Q4K_EXACT, "mynah_q4k_gemv_exact")        \
    X(MYNAH_K_Q6K_EXACT, "mynah_q6k_gemv_exact")        \
    X(MYNAH_K_Q80_EXACT, "mynah_q80_gemv_exact")        \
    X(MYNAH_K_Q4K_EXACT_SEQ, "mynah_q4k_gemv_exact_seq") \
    X(MYNAH_K_Q80_EXACT_SEQ, "mynah_q80_gemv_exact_seq")

enum {
#define X(id, name) id,
    MYNAH_KERNEL_LIST(X)
#undef X
    MYNAH_K_COUNT
};

#define MYNAH_MAX_DEVICES 16

typedef struct {
    int loaded;
    hipModule_t module;
    hipFunction_t fn[MYNAH_K_COUNT];
    hipStream_t stream;
} mynah_device;

void mynah_set_error(const char *fmt, ...);
mynah_device *mynah_dev(void);
hipStream_t mynah_stream_or_default(mynah_device *d, void *stream);
int mynah_launch(mynah_device *d, int kernel, unsigned gx, unsigned gy, unsigned block,
                 size_t shmem, hipStream_t stream, void **args);
int mynah_geometry(int type, size_t rows, size_t cols, size_t *row_bytes);

int mynah_gemv_launch(mynah_device *d, int type, const void *w, size_t rows, size_t cols,
                      const float *x, float *y, hipStream_t stream);
/* The exact GEMV in the batched reference's summation order (one token of
 * the exact matmat). cols must be a multiple of 256. */
int mynah_gemv_seq_launch(mynah_device *d, int type, const void *w, size_t rows, size_t cols,
                          const float *x, float *y, hipStream_t stream);
int mynah_dequant_launch(mynah_device *d, int type, const void *w, size_t rows, size_t cols,
                         float *y, hipStream_t stream);
int mynah_matmat_launch(mynah_device *d, int type, const void *w, size_t rows, size_t cols,
                        const float *x, float *y, size_t tokens, hipStream_t stream);

#endif
