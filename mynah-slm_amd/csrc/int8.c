/* int8.c — host side of the int8 activation lane of Q4_K products and of
 * batched Q5_K products (int8.hip): the lane switch, the launches and the
 * per-call workspace.
 *
 * The reference has this lane only in an AVX2 + FMA (or Arm dotprod) build of
 * ingot. There, INGOT_SDOT selects it (third_party/ingot/src/kernels.c:
 * 812-838 for the matvec, 1704-1721 for the batched form):
 *   - the batched Q4_K and Q5_K matmat (tokens >= 2) is int8 unless
 *     INGOT_SDOT=0 (kernels.c:1742-1751, 2573-2595);
 *   - the Q4_K matvec is int8 only with INGOT_SDOT=1;
 *   - ingot_matmat_is_exact(tokens) says which path a width takes.
 * The as-built reference (ingot's -O2, no -march) has no int8 lane, and this
 * library follows it by default: MYNAH_INT8_OFF. mynah_hip_set_int8() or
 * INGOT_SDOT=1 in the environment (read once, at the first call that asks)
 * turn it on.
 *
 * SPDX-License-Identifier: MIT */
#include "kernels_hip.h"
#include "runtime_internal.h"

#include <pthread.h>
#include <math.h>
#include <stdlib.h>

static int int8_mode = -1;
static pthread_mutex_t mode_mu = PTHREAD_MUTEX_INITIALIZER;

int mynah_int8_mode(void) {
    pthread_mutex_lock(&mode_mu);
    if (int8_mode < 0) {
        const char *v = getenv("INGOT_SDOT");
        int8_mode = (v != NULL && v[0] == '1') ? MYNAH_INT8_ALL : MYNAH_INT8_OFF;
    }
    const int m = int8_mode;
    pthread_mutex_unlock(&mode_mu);
    return m;
}

int mynah_hip_set_int8(int mode) {
    if (mode != MYNAH_INT8_OFF && mode != MYNAH_INT8_BATCHED && mode != MYNAH_INT8_ALL) {
        mynah_set_error("unknown int8 mode %d", mode);
        return -1;
    }
    pthread_mutex_lock(&mode_mu);
    int8_mode = mode;
    pthread_mutex_unlock(&mode_mu);
    return 0;
}

int mynah_hip_int8(void) { return mynah_int8_mode(); }

/* The reference's batched core walks tokens in tiles of
 * clamp(4 MiB / (4 cols), 32, 128), rounded down to even (kernels.c:893-920,
 * no INGOT_QK_TILE override); the epilogue of a token depends on where it
 * falls in its tile. */
static uint32_t token_tile(size_t cols) {
    size_t tile = ((size_t)4 << 20) / (cols * sizeof(float));
    if (tile > 128) tile = 128;
    if (tile < 32) tile = 32;
    tile &= ~(size_t)1;
    return (uint32_t)tile;
}

static int check_kq(int type, const void *w, size_t rows, size_t cols, size_t tokens) {
    size_t rb;
    if (type != MYNAH_Q4_K && type != MYNAH_Q5_K) {
        mynah_set_error("the int8 lane takes Q4_K and Q5_K only");
        return -1;
    }
    if (mynah_geometry(type, rows, cols, &rb) != 0) return -1;
    if (tokens == 0 || tokens > 0xffffffffu || rows > 0xffffffffu ||
        tokens > SIZE_MAX / cols || cols / 256 > 0xffffffffu / tokens) {
        mynah_set_error("bad token count");
        return -1;
    }
    if (((uintptr_t)w & 15u) != 0) {
        mynah_set_error("Q4_K / Q5_K weights must be 16-byte aligned");
        return -1;
    }
    if (type == MYNAH_Q5_K && tokens < 2) {
        mynah_set_error("Q5_K has no int8 matvec (the reference's lane is batched only)");
        return -1;
    }
    return 0;
}

int mynah_q8_quantize_launch(mynah_device *d, const float *x, size_t tokens, size_t cols,
                             int8_t *xq, float *xs, int32_t *xsum, hipStream_t stream) {
    if (x == NULL || xq == NULL || xs == NULL || xsum == NULL) {
        mynah_set_error("null argument");
        return -1;
    }
    if (cols == 0 || cols % 256 != 0 || tokens == 0 || tokens > SIZE_MAX / cols ||
        tokens * (cols / 256) > 0xffffffffu - 3u || cols > 0xffffffffu) {
        mynah_set_error("quantiser needs cols a multiple of 256 and a sane token count");
        return -1;
    }
    if (((uintptr_t)x & 15u) != 0 || ((uintptr_t)xq & 3u) != 0 || ((uintptr_t)xs & 3u) != 0 ||
        ((uintptr_t)xsum & 3u) != 0) {
        mynah_set_error("misaligned quantiser operand");
        return -1;
    }
    uint32_t units = (uint32_t)(tokens * (cols / 256)), nb = (uint32_t)(cols / 256),
             c32 = (uint32_t)cols;
    void *args[] = {&x, &xq, &xs, &xsum, &units, &nb, &c32};
    return mynah_launch(d, MYNAH_K_Q8_QUANTIZE, (units + 3u) / 4u, 1, 256, 0, stream, args);
}

int mynah_q4k_int8_launch(mynah_device *d, int type, const void *w, size_t rows, size_t cols,
                          const int8_t *xq, const float *xs, const int32_t *xsum, float *y,
                          size_t tokens, hipStream_t stream) {
    if (w == NULL || xq == NULL || xs == NULL || xsum == NULL || y == NULL) {
        mynah_set_error("null argument");
        return -1;
    }
    if (check_kq(type, w, rows, cols, tokens) != 0) return -1;
    if (((uintptr_t)xq & 15u) != 0 || ((uintptr_t)xsum & 15u) != 0 || ((uintptr_t)xs & 3u) != 0) {
        mynah_set_error("int8 operands must be 16-byte aligned");
        return -1;
    }
    uint32_t r32 = (uint32_t)rows, nb = (uint32_t)(cols / 256);
    if (tokens == 1) {
        uint32_t rpw = nb >= 256 ? 1u : 256u / nb;
        const size_t shmem = (size_t)rpw * nb * sizeof(float);
        if (shmem > 64 * 1024) {
            mynah_set_error("row too long for the int8 matvec");
            return -1;
        }
        void *args[] = {&w, &xq, &xs, &xsum, &y, &r32, &nb, &rpw};
        return mynah_launch(d, MYNAH_K_Q4K_GEMV_INT8, (unsigned)((rows + rpw - 1) / rpw), 1, 256,
                            shmem, stream, args);
    }
    uint32_t c32 = (uint32_t)cols, t32 = (uint32_t)tokens, tile = token_tile(cols);
    void *args[] = {&w, &xq, &xs, &xsum, &y, &r32, &c32, &t32, &nb, &tile};
    /* Workgroup tile (32 tr) rows x (32 tt) tokens: the largest tile whose
     * workgroups fill whole rounds of the chip (>= 90 % of the last round
     * busy), given how many of each fit a CU (LDS: the double-buffered
     * operands, 60 KiB for 2 x 2 down to 30 KiB for 1 x 1); else the tile
     * with the fullest last round. */
    static const int cand[4][3] = {{2, 2, 2}, {2, 1, 3}, {1, 2, 3}, {1, 1, 5}};
    int tr = 1, tt = 1;
    double best = -1.0;
    for (int c = 0; c < 4; c++) {
        const double wgs = (double)((rows + 32u * cand[c][0] - 1) / (32u * cand[c][0])) *
                           (double)((tokens + 32u * cand[c][1] - 1) / (32u * cand[c][1]));
        const double rounds = wgs / ((double)d->cus * cand[c][2]);
        const double fill = rounds / ceil(rounds);
        if (fill >= 0.9) {
            tr = cand[c][0];
            tt = cand[c][1];
            break;
        }
        if (fill > best) {
            best = fill;
            tr = cand[c][0];
            tt = cand[c][1];
        }
    }
    const char *env = getenv("MYNAH_INT8_TILE");
    if (env != NULL && env[0] >= '1' && env[0] <= '2' && env[1] >= '1' && env[1] <= '2') {
        tr = env[0] - '0';
        tt = env[1] - '0';
    }
    if (type == MYNAH_Q5_K) tr = tt = 2;      /* the one Q5_K tile */
    const int k = type == MYNAH_Q5_K ? MYNAH_K_Q5K_GEMM_INT8_22
                  : tr == 1 ? (tt == 1 ? MYNAH_K_Q4K_GEMM_INT8_11 : MYNAH_K_Q4K_GEMM_INT8_12)
                            : (tt == 1 ? MYNAH_K_Q4K_GEMM_INT8_21 : MYNAH_K_Q4K_GEMM_INT8_22);
    const size_t wr = (size_t)32 * tr, wt = (size_t)32 * tt;
    return mynah_launch(d, k, (unsigned)((rows + wr - 1) / wr), (unsigned)((tokens + wt - 1) / wt),
                        256, 0, stream, args);
}

/* Workspace of one call: xq, xs, xsum, each 256-byte aligned. */
static size_t ws_bytes(size_t tokens, size_t cols, size_t *o_xs, size_t *o_sum) {
    const size_t nb = cols / 256;
    size_t off = (tokens * cols + 255) & ~(size_t)255;
    *o_xs = off;
    off += (tokens * nb * sizeof(float) + 255) & ~(size_t)255;
    *o_sum = off;
    off += tokens * nb * 8 * sizeof(int32_t);
    return off;
}

int mynah_int8_product(mynah_device *d, int type, const void *w, size_t rows, size_t cols,
                       const float *x, float *y, size_t tokens, hipStream_t stream) {
    if (check_kq(type, w, rows, cols, tokens) != 0) return -1;
    if (tokens > (SIZE_MAX / 2) / cols) {
        mynah_set_error("size overflow");
        return -1;
    }
    size_t o_xs, o_sum;
    const size_t bytes = ws_bytes(tokens, cols, &o_xs, &o_sum);
    /* The reference allocates its quantised activations per call
     * (kernels.c:1616-1622, 749-755); here the allocation is stream-ordered,
     * so concurrent calls on different streams each get their own. */
    unsigned char *ws = NULL;
    hipError_t e = hipMallocAsync((void **)&ws, bytes, stream);
    if (e != hipSuccess) {
        mynah_set_error("hipMallocAsync(int8 workspace): %s", hipGetErrorString(e));
        return -1;
    }
    int rc = mynah_q8_quantize_launch(d, x, tokens, cols, (int8_t *)ws, (float *)(ws + o_xs),
                                      (int32_t *)(ws + o_sum), stream);
    if (rc == 0)
        rc = mynah_q4k_int8_launch(d, type, w, rows, cols, (const int8_t *)ws,
                                   (const float *)(ws + o_xs), (const int32_t *)(ws + o_sum), y,
                                   tokens, stream);
    e = hipFreeAsync(ws, stream);
    if (rc == 0 && e != hipSuccess) {
        mynah_set_error("hipFreeAsync(int8 workspace): %s", hipGetErrorString(e));
        return -1;
    }
    return rc;
}

/* ── public entry points ─────────────────────────────────────────────────── */

/* The int8 product with its workspace in the device's fixed array (the
 * address the runtime resolved when it loaded the code object): no
 * allocation of any kind, so it may run under stream capture or in a loop
 * that must not allocate. Calls that overlap on one device share the array
 * and race. */
int mynah_hip_int8_product_noalloc_dev(int type, const void *w, size_t rows, size_t cols,
                                       const float *x, float *y, size_t tokens, void *stream) {
    mynah_device *d = mynah_dev();
    if (d == NULL) return -1;
    if (w == NULL || x == NULL || y == NULL) {
        mynah_set_error("null argument");
        return -1;
    }
    if (check_kq(type, w, rows, cols, tokens) != 0) return -1;
    if (tokens > (SIZE_MAX / 2) / cols) {
        mynah_set_error("size overflow");
        return -1;
    }
    size_t o_xs, o_sum;
    const size_t bytes = ws_bytes(tokens, cols, &o_xs, &o_sum);
    if (d->scratch == NULL || bytes > d->scratch_bytes) {
        mynah_set_error("int8 workspace of %zu bytes (%zu tokens x %zu columns) exceeds the "
                        "fixed %zu-byte scratch", bytes, tokens, cols, d->scratch_bytes);
        return -1;
    }
    hipStream_t s = mynah_stream_or_default(d, stream);
    unsigned char *ws = d->scratch;
    int rc = mynah_q8_quantize_launch(d, x, tokens, cols, (int8_t *)ws, (float *)(ws + o_xs),
                                      (int32_t *)(ws + o_sum), s);
    if (rc == 0)
        rc = mynah_q4k_int8_launch(d, type, w, rows, cols, (const int8_t *)ws,
                                   (const float *)(ws + o_xs), (const int32_t *)(ws + o_sum), y,
                                   tokens, s);
    return rc;
}

int mynah_hip_q8_quantize_dev(const float *x, size_t tokens, size_t cols, int8_t *xq, float *xs,
                              int32_t *xsum, void *stream) {
    mynah_device *d = mynah_dev();
    if (d == NULL) return -1;
    return mynah_q8_quantize_launch(d, x, tokens, cols, xq, xs, xsum,
                                    mynah_stream_or_default(d, stream));
}

int mynah_hip_q4k_int8_dev(const void *w, size_t rows, size_t cols, const int8_t *xq,
                           const float *xs, const int32_t *xsum, float *y, size_t tokens,
                           void *stream) {
    mynah_device *d = mynah_dev();
    if (d == NULL) return -1;
    return mynah_q4k_int8_launch(d, MYNAH_Q4_K, w, rows, cols, xq, xs, xsum, y, tokens,
                                 mynah_stream_or_default(d, stream));
}
