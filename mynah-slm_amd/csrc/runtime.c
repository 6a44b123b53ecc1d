/* runtime.c — C11 host side of the gfx950 kernels: module loading, launch
 * geometry, the ingot-compatible entry points and the device-resident API
 * declared in include/kernels_hip.h.
 *
 * The kernels are one code object (hipcc --genco, gfx950) embedded in this
 * library; each device loads it with hipModuleLoadData on first use and the
 * kernels run through hipModuleLaunchKernel. No C++ host code, no PyTorch.
 *
 * SPDX-License-Identifier: MIT */
#define _GNU_SOURCE
#include "kernels_hip.h"
#include "runtime_internal.h"
#include "scratch.h"

#include <pthread.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

extern const unsigned char mynah_codeobj[];

static _Thread_local char last_error[512];

void mynah_set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(last_error, sizeof last_error, fmt, ap);
    va_end(ap);
}

const char *mynah_hip_last_error(void) { return last_error; }

#define HIP_OK(call, what)                                                            \
    do {                                                                              \
        hipError_t e_ = (call);                                                       \
        if (e_ != hipSuccess) {                                                       \
            mynah_set_error("%s: %s", what, hipGetErrorString(e_));                   \
            return -1;                                                                \
        }                                                                             \
    } while (0)

/* ── per-device state ────────────────────────────────────────────────────── */

static const char *const kernel_names[MYNAH_K_COUNT] = {
#define X(id, name) [id] = name,
    MYNAH_KERNEL_LIST(X)
#undef X
};

static mynah_device devices[MYNAH_MAX_DEVICES];
static int index_order_sums;
static int current_device = -1;
static pthread_mutex_t init_mu = PTHREAD_MUTEX_INITIALIZER;
static pthread_mutex_t host_mu = PTHREAD_MUTEX_INITIALIZER;

static int load_device(int dev) {
    mynah_device *d = &devices[dev];
    if (d->loaded) return 0;
    HIP_OK(hipSetDevice(dev), "hipSetDevice");
    HIP_OK(hipModuleLoadData(&d->module, mynah_codeobj), "hipModuleLoadData");
    for (int k = 0; k < MYNAH_K_COUNT; k++) {
        if (kernel_names[k] == NULL) continue;
        hipError_t e = hipModuleGetFunction(&d->fn[k], d->module, kernel_names[k]);
        if (e != hipSuccess) {
            mynah_set_error("kernel %s missing from the code object: %s", kernel_names[k],
                            hipGetErrorString(e));
            return -1;
        }
    }
    /* The allocation-free entry point's workspace is a device array of the
     * code object; its address on this device (each device has its own
     * copy) is looked up here, once, with the device current. Host code uses
     * only this address, never the symbol. */
    {
        hipDeviceptr_t p = 0;
        size_t bytes = 0;
        HIP_OK(hipModuleGetGlobal(&p, &bytes, d->module, "mynah_scratch"),
               "hipModuleGetGlobal(mynah_scratch)");
        if (p == 0 || bytes != MYNAH_SCRATCH_BYTES) {
            mynah_set_error("mynah_scratch: %zu bytes, expected %u", bytes,
                            (unsigned)MYNAH_SCRATCH_BYTES);
            return -1;
        }
        d->scratch = (unsigned char *)p;
        d->scratch_bytes = bytes;
        HIP_OK(hipModuleGetGlobal(&p, &bytes, d->module, "mynah_index_sums"),
               "hipModuleGetGlobal(mynah_index_sums)");
        d->index_sums = (uint32_t *)p;
    }
    HIP_OK(hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking), "hipStreamCreate");
    /* The switch starts at 0 with the code object; it is written only when
     * on, through the library's stream: a copy on the null stream here
     * measurably slowed every later decode step (about 1 %). */
    if (index_order_sums) {
        const uint32_t on = 1u;
        HIP_OK(hipMemcpyHtoDAsync((hipDeviceptr_t)d->index_sums, (void *)&on, sizeof on, d->stream),
               "hipMemcpyHtoDAsync(mynah_index_sums)");
        HIP_OK(hipStreamSynchronize(d->stream), "hipStreamSynchronize");
    }
    if (hipDeviceGetAttribute(&d->cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        d->cus <= 0)
        d->cus = 256;
    d->loaded = 1;
    return 0;
}

int mynah_hip_init(int device) {
    pthread_mutex_lock(&init_mu);
    int rc = 0;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        mynah_set_error("no HIP device visible");
        rc = -1;
    } else if (device < 0 || device >= count || device >= MYNAH_MAX_DEVICES) {
        mynah_set_error("device %d out of range (have %d)", device, count);
        rc = -1;
    } else {
        rc = load_device(device);
        if (rc == 0) current_device = device;
    }
    pthread_mutex_unlock(&init_mu);
    return rc;
}

mynah_device *mynah_dev(void) {
    if (current_device < 0) {
        const char *env = getenv("MYNAH_HIP_DEVICE");
        if (mynah_hip_init(env ? atoi(env) : 0) != 0) return NULL;
    }
    mynah_device *d = &devices[current_device];
    if (hipSetDevice(current_device) != hipSuccess) {
        mynah_set_error("hipSetDevice(%d) failed", current_device);
        return NULL;
    }
    return d;
}

hipStream_t mynah_stream_or_default(mynah_device *d, void *stream) {
    return stream ? (hipStream_t)stream : d->stream;
}

int mynah_launch(mynah_device *d, int kernel, unsigned gx, unsigned gy, unsigned block,
                 size_t shmem, hipStream_t stream, void **args) {
    hipError_t e = hipModuleLaunchKernel(d->fn[kernel], gx, gy, 1, block, 1, 1,
                                         (unsigned)shmem, stream, args, NULL);
    if (e != hipSuccess) {
        mynah_set_error("launch of %s: %s", kernel_names[kernel], hipGetErrorString(e));
        return -1;
    }
    return 0;
}

int mynah_launch3(mynah_device *d, int kernel, unsigned gx, unsigned gy, unsigned gz,
                  unsigned block, size_t shmem, hipStream_t stream, void **args) {
    hipError_t e = hipModuleLaunchKernel(d->fn[kernel], gx, gy, gz, block, 1, 1,
                                         (unsigned)shmem, stream, args, NULL);
    if (e != hipSuccess) {
        mynah_set_error("launch of %s: %s", kernel_names[kernel], hipGetErrorString(e));
        return -1;
    }
    return 0;
}

/* ── geometry ────────────────────────────────────────────────────────────── */

int mynah_geometry(int type, size_t rows, size_t cols, size_t *row_bytes) {
    size_t elems, bytes;
    switch (type) {
    case MYNAH_Q4_K: elems = 256; bytes = 144; break;
    case MYNAH_Q5_K: elems = 256; bytes = 176; break;
    case MYNAH_Q6_K: elems = 256; bytes = 210; break;
    case MYNAH_Q8_0: elems = 32;  bytes = 34;  break;
    case MYNAH_Q4_0: elems = 32;  bytes = 18;  break;
    default:
        mynah_set_error("type %d has no kernel", type);
        return -1;
    }
    if (rows == 0 || cols == 0 || cols % elems != 0) {
        mynah_set_error("bad geometry rows=%zu cols=%zu for type %d", rows, cols, type);
        return -1;
    }
    const size_t blocks = cols / elems;
    if (blocks > SIZE_MAX / bytes || rows > SIZE_MAX / (blocks * bytes) ||
        rows > SIZE_MAX / cols || rows > 0xffffffffu || cols > 0xffffffffu) {
        mynah_set_error("size overflow");
        return -1;
    }
    *row_bytes = blocks * bytes;
    return 0;
}

/* ── GEMV launch ─────────────────────────────────────────────────────────── */

#define GEMV_WG 256

static int gemv_order = MYNAH_GEMV_EXACT;

int mynah_hip_set_gemv_order(int order) {
    if (order != MYNAH_GEMV_EXACT && order != MYNAH_GEMV_REORDERED) {
        mynah_set_error("unknown GEMV order %d", order);
        return -1;
    }
    gemv_order = order;
    return 0;
}

int mynah_hip_gemv_order(void) { return gemv_order; }

int mynah_hip_set_index_order_sums(int on) {
    if (on != 0 && on != 1) {
        mynah_set_error("index-order sums: %d is neither 0 nor 1", on);
        return -1;
    }
    pthread_mutex_lock(&init_mu);
    index_order_sums = on;
    int rc = 0, cur = -1;
    (void)hipGetDevice(&cur);
    for (int dev = 0; dev < MYNAH_MAX_DEVICES && rc == 0; dev++) {
        mynah_device *d = &devices[dev];
        if (!d->loaded) continue;
        const uint32_t v = (uint32_t)on;
        if (hipSetDevice(dev) != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
            hipMemcpyHtoDAsync((hipDeviceptr_t)d->index_sums, (void *)&v, sizeof v, d->stream) !=
                hipSuccess ||
            hipStreamSynchronize(d->stream) != hipSuccess) {
            mynah_set_error("index-order sums: setting the switch on device %d failed", dev);
            rc = -1;
        }
    }
    if (cur >= 0) (void)hipSetDevice(cur);
    pthread_mutex_unlock(&init_mu);
    return rc;
}

/* allow_int8 == 0 keeps the exact order whatever the int8 lane's mode (the
 * reference's ingot_q4_k_matvec_scalar). */
static int gemv_launch(mynah_device *d, int type, const void *w, size_t rows, size_t cols,
                       const float *x, float *y, hipStream_t stream, int allow_int8) {
    size_t rb;
    if (mynah_geometry(type, rows, cols, &rb) != 0) return -1;
    /* INGOT_SDOT=1 semantics: the Q4_K matvec quantises its input
     * (third_party/ingot/src/kernels.c:819-834). */
    if (allow_int8 && type == MYNAH_Q4_K && mynah_int8_mode() == MYNAH_INT8_ALL)
        return mynah_int8_product(d, MYNAH_Q4_K, w, rows, cols, x, y, 1, stream);
    if (type == MYNAH_Q4_0) return mynah_q40_launch(d, w, rows, cols, x, y, 1, NULL, stream);
    if (type != MYNAH_Q8_0 && cols % 256 != 0) {
        mynah_set_error("cols must be a multiple of 256");
        return -1;
    }
    if (((uintptr_t)x & 15u) != 0) {
        mynah_set_error("x must be 16-byte aligned");
        return -1;
    }
    if (mynah_w_misaligned(type, w)) {
        mynah_set_error("weights misaligned for type %d", type);
        return -1;
    }
    if (rb > 0xffffffffu) {
        mynah_set_error("row too long");
        return -1;
    }
    mynah_gemv_group g;
    memset(&g, 0, sizeof g);
    g.n = 1;
    if (mynah_gemv_desc_init(&g.d[0], type, w, rows, cols, x, y) != 0) return -1;
    return mynah_gemv_group_launch(d, &g, stream, NULL, -1);
}

int mynah_gemv_launch(mynah_device *d, int type, const void *w, size_t rows, size_t cols,
                      const float *x, float *y, hipStream_t stream) {
    return gemv_launch(d, type, w, rows, cols, x, y, stream, 1);
}

static long env_long(const char *name, long dflt);

int mynah_q40_launch(mynah_device *d, const void *w, size_t rows, size_t cols, const float *x,
                     float *y, size_t tokens, const float *res, hipStream_t stream) {
    size_t rb;
    if (mynah_geometry(MYNAH_Q4_0, rows, cols, &rb) != 0) return -1;
    /* Batched: T token chains per lane, the largest of 8, 4, 2 that still
     * gives >= 2048 one-wave workgroups (two per SIMD), since each chain is
     * serial and a lane's T chains are its only overlap. */
    const size_t row_groups = (rows + 63) / 64;
    size_t per = tokens == 1 ? 1 : 8;
    while (per > 2 && row_groups * ((tokens + per - 1) / per) < 2048) per /= 2;
    const size_t groups = (tokens + per - 1) / per;
    if (tokens == 0 || groups > 65535u || rb > 0xffffffffu) {
        mynah_set_error("bad token count for the Q4_0 product");
        return -1;
    }
    if (((uintptr_t)w & 1u) != 0 || ((uintptr_t)x & 15u) != 0) {
        mynah_set_error("misaligned operand for the Q4_0 product");
        return -1;
    }
    uint32_t r32 = (uint32_t)rows, c32 = (uint32_t)cols, t32 = (uint32_t)tokens, rb32 = (uint32_t)rb;
    const unsigned grid = (unsigned)((rows + 63) / 64);
    /* The matvec below 32,768 rows: one adding wave and three product waves
     * per 64 rows, the chain then runs ~1.5x faster (9.5 against 14 ns per
     * weight). With more rows the one-wave kernel already fills the chip and
     * does less work in all (151936 x 1024: 35 against 53 us).
     * MYNAH_Q40_PC=0 always takes the one-wave kernel. */
    if (tokens == 1 && res == NULL && rows < 32768u && env_long("MYNAH_Q40_PC", 1) != 0) {
        void *args[] = {&w, &x, &y, &r32, &c32, &rb32};
        return mynah_launch(d, MYNAH_K_Q40_CHAIN_PC, grid, 1, 256, 0, stream, args);
    }
    void *args[] = {&w, &x, &y, &r32, &c32, &t32, &rb32, &res};
    const int k = per == 1 ? MYNAH_K_Q40_CHAIN1 : per == 2 ? MYNAH_K_Q40_CHAIN2
                : per == 4 ? MYNAH_K_Q40_CHAIN4 : MYNAH_K_Q40_CHAIN8;
    return mynah_launch(d, k, grid, (unsigned)groups, 64, 0, stream, args);
}

int mynah_gemv_desc_init(mynah_gemv_desc *g, int type, const void *w, size_t rows, size_t cols,
                         const float *x, float *y) {
    size_t rb;
    memset(g, 0, sizeof *g);
    if (mynah_geometry(type, rows, cols, &rb) != 0) return -1;
    if ((type != MYNAH_Q8_0 && type != MYNAH_Q4_0 && cols % 256 != 0) || rb > 0xffffffffu) {
        mynah_set_error("cols must be a multiple of 256");
        return -1;
    }
    if (mynah_w_misaligned(type, w) || ((uintptr_t)x & 3u) != 0) {
        mynah_set_error("misaligned operand for type %d", type);
        return -1;
    }
    g->w = w;
    g->x = x;
    g->y = y;
    g->rows = (uint32_t)rows;
    g->cols = (uint32_t)cols;
    g->units = (uint32_t)(type == MYNAH_Q8_0 || type == MYNAH_Q4_0 ? cols / 32 : cols / 256);
    g->row_bytes = (uint32_t)rb;
    g->type = (uint32_t)type;
    return 0;
}

static uint32_t fast_ks(uint32_t all_rows) {
    return all_rows >= 32768u ? 1u : all_rows >= 8192u ? 2u : 4u;
}

/* Exact-order layout of a grouped launch: K unit slots per row in a wave
 * (64 / K rows per wave), WS waves sharing rows, WR row groups per
 * workgroup. Small launches spread one unit per lane over as many
 * workgroups as possible (they are latency-bound); large ones keep every
 * lane busy (K divides the units) and group rows to share the staged x. */
static void exact_shape(uint32_t all_rows, uint32_t units, uint32_t *lk, uint32_t *ws,
                        uint32_t *wr) {
    uint32_t k = 1;
    if (all_rows >= 16384u) {
        while (k < 16u && units % (2u * k) == 0) k *= 2u;
    } else {
        while (k < 16u && k < units) k *= 2u;
    }
    uint32_t w = (units + k - 1u) / k;
    if (w > 16u) w = 16u;
    /* Large launches: at most two waves share rows, so each lane sums a few
     * units (measured on the 151936 x 2560 head: 76 us against 117 us with
     * one unit per lane over five waves). */
    if (all_rows >= 16384u && w > 2u) w = 2u;
    const uint32_t rpw = 64u / k;
    uint32_t r = 1, tiles = (all_rows + rpw - 1u) / rpw;
    while (w * r * 2u <= 4u && rpw * r * 2u <= 64u && tiles / (r * 2u) >= 1024u) r *= 2u;
    uint32_t l = 0;
    while ((1u << l) < k) l++;
    *lk = l;
    *ws = w;
    *wr = r;
}

static long env_long(const char *name, long dflt) {
    const char *e = getenv(name);
    return (e != NULL && e[0] != '\0') ? strtol(e, NULL, 10) : dflt;
}

/* How a grouped GEMV runs: which kernel, its grid, block, LDS and shape
 * word (and, for the streaming kernel, its descriptor). */
typedef struct {
    int kernel;
    uint32_t grid, threads, shape;
    uint32_t tile_rows;      /* rows per workgroup; 0: each descriptor's pad */
    size_t lds;
    mynah_stream_desc sd;
} gemv_plan;

/* The streaming exact GEMV (gemv_stream.hip) for one large Q4_K / Q6_K
 * matrix with long rows and no epilogue beyond the input RMSNorm and argmax
 * keys: a persistent launch of four 4-wave workgroups per CU, each owning a
 * balanced range of rows. Returns 1 when the launch does not qualify (the
 * grouped kernel runs instead), 0 planned. Tuning switches:
 * MYNAH_GEMV_STREAM=0 off, MYNAH_GEMV_MIX=1 the v_fma_mix_f32 form,
 * MYNAH_STREAM_WGS, MYNAH_STREAM_MIN_UNITS, MYNAH_STREAM_MIN_ROW_UNITS. */
static int gemv_stream_plan(const mynah_device *d, const mynah_gemv_group *grp, gemv_plan *p) {
    if (grp->n != 1 || env_long("MYNAH_GEMV_STREAM", 1) == 0) return 1;
    const mynah_gemv_desc *g = &grp->d[0];
    if (g->w2 != NULL || g->res != NULL || g->ypos != NULL ||
        (g->type != MYNAH_Q4_K && g->type != MYNAH_Q6_K))
        return 1;
    const uint64_t units = (uint64_t)g->rows * g->units;
    /* Long rows only: with four super-blocks per row (the 0.6B head) the
     * grouped kernel is faster. */
    if (units < (uint64_t)env_long("MYNAH_STREAM_MIN_UNITS", 131072) ||
        g->units < (uint32_t)env_long("MYNAH_STREAM_MIN_ROW_UNITS", 8))
        return 1;
    long wgs = env_long("MYNAH_STREAM_WGS", 4L * d->cus);
    if (wgs < 1) wgs = 1;
    if ((uint64_t)wgs > g->rows) wgs = (long)g->rows;
    const uint64_t max_rows = ((uint64_t)g->rows + (uint64_t)wgs - 1u) / (uint64_t)wgs;
    const uint64_t nf = (max_rows * g->units + 4u) & ~(uint64_t)3u;   /* + spare slot */
    const size_t lds = ((size_t)g->cols + 4u * ((g->cols + 255u) / 256u) + nf +
                        (g->norm_w ? (size_t)g->cols : 0u)) * 4u;
    if (lds > 64u * 1024u) return 1;
    mynah_stream_desc sd = {g->w, g->x, g->y, g->norm_w, g->keys, g->rows, g->units,
                            g->row_bytes, g->type, g->cols, g->eps};
    p->sd = sd;
    p->kernel = env_long("MYNAH_GEMV_MIX", 0) ? MYNAH_K_GEMV_STREAM : MYNAH_K_GEMV_STREAM_CVT;
    p->grid = (uint32_t)wgs;
    p->tile_rows = 0;
    p->threads = 256;
    p->lds = lds;
    p->shape = 0;
    return 0;
}

/* Flat layout: every thread of a T-thread workgroup owns one (row, unit)
 * pair of R = min(64, T / units) whole rows (units of a gate/up pair
 * counted twice). T is the multiple of 64 up to 1024 that scores best on
 * lane use times CU coverage (min(1, workgroups / CUs)); among scores within
 * 0.02 of the best the largest T wins, since each workgroup stages (and
 * normalises) the whole input once. MYNAH_FLAT_T forces T. */
static int gemv_flat_plan(const mynah_device *d, mynah_gemv_group *grp, gemv_plan *p) {
    const long forced = env_long("MYNAH_FLAT_T", 0);
    uint32_t max_ut = 1;
    for (uint32_t i = 0; i < grp->n; i++) {
        const mynah_gemv_desc *g = &grp->d[i];
        const uint32_t ut = g->w2 ? 2u * g->units : g->units;
        if (ut > max_ut) max_ut = ut;
    }
    double score[17] = {0};
    double best = -1.0;
    for (uint32_t t = 64; t <= 1024; t += 64) {
        if (t < max_ut || (forced > 0 && (long)t != forced)) continue;
        uint64_t used = 0, wgs = 0;
        for (uint32_t i = 0; i < grp->n; i++) {
            const mynah_gemv_desc *g = &grp->d[i];
            const uint32_t ut = g->w2 ? 2u * g->units : g->units;
            uint32_t r = t / ut;
            if (r > 64u) r = 64u;
            const uint64_t tiles = (g->rows + r - 1u) / r;
            wgs += tiles;
            used += (uint64_t)r * ut * tiles;
        }
        const double cover = wgs >= (uint64_t)d->cus ? 1.0 : (double)wgs / (double)d->cus;
        score[t / 64] = (double)used / ((double)t * (double)wgs) * cover;
        if (score[t / 64] > best) best = score[t / 64];
    }
    if (best < 0.0) {
        mynah_set_error("no flat layout for %u units per row", max_ut);
        return -1;
    }
    uint32_t T = 64;
    for (uint32_t t = 64; t <= 1024; t += 64)
        if (score[t / 64] > 0.0 && score[t / 64] >= best - 0.02) T = t;
    uint32_t tiles = 0;
    size_t lds = 0;
    int all_q4k = T <= 512u, all_q6k = T <= 512u;
    for (uint32_t i = 0; i < grp->n; i++) {
        mynah_gemv_desc *g = &grp->d[i];
        const uint32_t ut = g->w2 ? 2u * g->units : g->units;
        uint32_t r = T / ut;
        if (r > 64u) r = 64u;
        g->pad = r;
        g->tile0 = tiles;
        tiles += (g->rows + r - 1u) / r;
        const size_t need = ((size_t)g->cols + 4u * ((g->cols + 255u) / 256u) +
                             (size_t)r * (ut | 1u) +
                             (g->norm_w ? (size_t)g->cols : 0u)) * 4u;
        if (need > lds) lds = need;
        all_q4k = all_q4k && g->type == MYNAH_Q4_K;
        all_q6k = all_q6k && g->type == MYNAH_Q6_K;
    }
    if (lds > 60u * 1024u) {
        mynah_set_error("input of this GEMV exceeds the LDS budget (%zu B)", lds);
        return -1;
    }
    p->grid = tiles;
    p->tile_rows = 0;
    p->lds = lds;
    p->threads = T;
    p->shape = 1u << 25;
    p->kernel = MYNAH_K_GEMV_GROUP;
    if (env_long("MYNAH_GEMV_TYPED", 1) != 0) {
        if (all_q4k) p->kernel = MYNAH_K_GEMV_FLAT_Q4K;
        else if (all_q6k) p->kernel = MYNAH_K_GEMV_FLAT_Q6K;
    }
    return 0;
}

/* Producer/consumer layout (gemv_pc.hip) for all-Q4_K launches: a
 * workgroup of one adding wave and four producing waves owns R = min(64,
 * 64 / Ut) whole rows, one super-block per adding lane. Returns 1 when the
 * launch does not qualify (rows longer than 64 super-blocks, or LDS over
 * 64 KiB). */
static int gemv_pc_plan(mynah_gemv_group *grp, gemv_plan *p) {
    uint32_t tiles = 0;
    size_t lds = 0;
    for (uint32_t i = 0; i < grp->n; i++) {
        mynah_gemv_desc *g = &grp->d[i];
        const uint32_t ut = g->w2 ? 2u * g->units : g->units;
        if (g->type != MYNAH_Q4_K || ut > 64u) return 1;
        const uint32_t r = 64u / ut;
        const size_t slots = 2u * (size_t)r * ut * 68u;
        const size_t tail = g->norm_w && g->cols > slots ? g->cols : slots;
        const size_t need = ((size_t)g->cols + 4u * ((g->cols + 255u) / 256u) +
                             (((size_t)r * (ut | 1u) + 3u) & ~(size_t)3u) + tail) * 4u;
        if (need > lds) lds = need;
    }
    if (lds > 64u * 1024u) return 1;
    for (uint32_t i = 0; i < grp->n; i++) {
        mynah_gemv_desc *g = &grp->d[i];
        const uint32_t r = 64u / (g->w2 ? 2u * g->units : g->units);
        g->pad = r;
        g->tile0 = tiles;
        tiles += (g->rows + r - 1u) / r;
    }
    p->grid = tiles;
    p->tile_rows = 0;
    p->lds = lds;
    p->threads = 320u;
    p->shape = 0;
    p->kernel = MYNAH_K_GEMV_PC_Q4K;
    return 0;
}

/* Plan a grouped GEMV in the given order (-1: the library's current one):
 * exact (lane = row x unit slot, unit sums folded in order; a single large
 * matrix with long rows takes the streaming kernel) or reordered (8-lane row
 * blocks, KS waves splitting the super-blocks of a tile). Sets each
 * descriptor's tile0. */
static int gemv_group_plan(const mynah_device *d, mynah_gemv_group *grp, int order, gemv_plan *p) {
    if (grp->n == 0 || grp->n > MYNAH_GROUP_MAX) {
        mynah_set_error("group of %u matrices", grp->n);
        return -1;
    }
    int exact = (order < 0 ? gemv_order : order) == MYNAH_GEMV_EXACT;
    uint32_t all_rows = 0, max_units = 1;
    uint64_t all_units = 0;
    int split = 1, chain = 0;
    for (uint32_t i = 0; i < grp->n; i++) {
        mynah_gemv_desc *g = &grp->d[i];
        if (g->type != MYNAH_Q4_K && g->type != MYNAH_Q5_K && g->type != MYNAH_Q6_K &&
            g->type != MYNAH_Q8_0 && g->type != MYNAH_Q4_0) {
            mynah_set_error("type %u has no grouped GEMV", g->type);
            return -1;
        }
        /* Q5_K and Q4_0 have only the exact kernel; their order is the
         * reference's anyway. */
        if (g->type == MYNAH_Q5_K) exact = 1;
        if (g->type == MYNAH_Q4_0) exact = 1, chain = 1;
        all_rows += g->rows;
        const uint32_t u = g->w2 ? 2u * g->units : g->units;
        if (u > max_units) max_units = u;
        all_units += (uint64_t)g->rows * u;
        if (g->type == MYNAH_Q8_0) split = 0;
        if (g->cols % 8 != 0 || ((uintptr_t)g->x & 15u) != 0 ||
            ((uintptr_t)g->norm_w & 15u) != 0) {
            mynah_set_error("grouped GEMV needs 16-byte aligned x and norm weights, cols %% 8 == 0");
            return -1;
        }
    }
    if (exact && !chain && gemv_stream_plan(d, grp, p) == 0) return 0;
    /* The producer/consumer layout for small all-Q4_K launches, whose
     * one-lane chains leave most SIMDs idle: MYNAH_GEMV_PC=1 wherever it
     * fits, 0 never; by default between MYNAH_PC_MIN_UNITS and
     * MYNAH_PC_MAX_UNITS super-blocks per launch. */
    if (exact && !chain) {
        const long pc = env_long("MYNAH_GEMV_PC", -1);
        const int want = pc == 1 || (pc < 0 &&
                         all_units >= (uint64_t)env_long("MYNAH_PC_MIN_UNITS", 1L << 62) &&
                         all_units <= (uint64_t)env_long("MYNAH_PC_MAX_UNITS", 0));
        if (want && gemv_pc_plan(grp, p) == 0) return 0;
    }
    /* A Q4_0 row is one running sum: with a Q4_0 matrix in the launch every
     * lane owns a whole row (K = 1, one wave of 64 rows per workgroup). */
    if (chain) split = 0;
    /* Split super-blocks across quads when the launch is small enough that
     * four times the waves still fit the 1,024 SIMDs about twice. */
    if (all_units > (uint64_t)env_long("MYNAH_SPLIT_UNITS", 32768)) split = 0;
    const char *env = getenv("MYNAH_GEMV_SPLIT");
    if (env != NULL) split = split && env[0] != '0';
    /* The flat layout (gemv_exact.hip group_flat) for the one-lane exact
     * kernels: MYNAH_GEMV_FLAT=0 keeps the slot layout below. */
    if (exact && !split && !chain && env_long("MYNAH_GEMV_FLAT", 1) != 0)
        return gemv_flat_plan(d, grp, p);
    uint32_t lk = 0, ws = 1, wr = 1, ks = 1, tile_rows;
    if (exact && split) {
        uint32_t k = 1;
        while (k < 16u && k < max_units) k *= 2u;
        ws = (max_units + k - 1u) / k;
        if (ws > 16u) ws = 16u;
        while ((1u << lk) < k) lk++;
        /* Four (eight for a gate/up pair) row groups per workgroup: fewer
         * workgroups each staging x (and its RMSNorm) with more threads. */
        wr = 4u;
        for (uint32_t i = 0; i < grp->n; i++)
            if (grp->d[i].w2 != NULL) wr = 8u;
        while (wr > 1u && ws * wr > 16u) wr /= 2u;
        tile_rows = (16u >> lk) * wr;
    } else if (exact && chain) {
        tile_rows = 64u;
    } else if (exact) {
        exact_shape(all_rows, max_units, &lk, &ws, &wr);
        tile_rows = (64u >> lk) * wr;
    } else {
        /* Reordered: small launches use KS = 4 for more waves in flight,
         * large ones KS = 1. */
        ks = fast_ks(all_rows);
        tile_rows = 32u / ks;
    }
    uint32_t tiles = 0;
    size_t lds = 0;
    for (uint32_t i = 0; i < grp->n; i++) {
        mynah_gemv_desc *g = &grp->d[i];
        const uint32_t ut = g->w2 ? 2u * g->units : g->units;
        /* Q4_0 keeps no unit partials in LDS. */
        const size_t parts = g->type == MYNAH_Q4_0 ? 0u : (size_t)tile_rows * (ut | 1u);
        const size_t need = exact ? ((size_t)g->cols + 4u * ((g->cols + 255u) / 256u) + parts +
                                     (g->norm_w ? (size_t)g->cols : 0u)) * 4u
                                  : ((size_t)g->cols + g->cols / 16 + g->cols / 8 +
                                     (g->norm_w ? (size_t)g->cols : 0u)) * 4u;
        if (need > lds) lds = need;
        g->tile0 = tiles;
        tiles += (g->rows + tile_rows - 1u) / tile_rows;
    }
    if (lds > 60u * 1024u) {
        mynah_set_error("input of this GEMV exceeds the LDS budget (%zu B)", lds);
        return -1;
    }
    p->grid = tiles;
    p->tile_rows = tile_rows;
    p->lds = lds;
    if (!exact) {
        p->kernel = MYNAH_K_GEMV_FAST_GROUP;
        p->threads = 256;
        p->shape = ks;
    } else {
        p->kernel = MYNAH_K_GEMV_GROUP;
        p->threads = 64u * ws * wr;
        p->shape = lk | (ws << 8) | (wr << 16) | ((uint32_t)(exact && split) << 24);
        /* Single-type launches in the one-lane layout, at most 256 threads:
         * entries compiled for that type alone hold more waves per SIMD
         * (Q6_K five, Q4_K six, against four). MYNAH_GEMV_TYPED=0 keeps the
         * general entry. */
        int all_q6k = !split && p->threads <= 256u, all_q4k = all_q6k;
        for (uint32_t i = 0; i < grp->n; i++) {
            all_q6k = all_q6k && grp->d[i].type == MYNAH_Q6_K;
            all_q4k = all_q4k && grp->d[i].type == MYNAH_Q4_K;
        }
        if (env_long("MYNAH_GEMV_TYPED", 1) != 0) {
            if (all_q6k) p->kernel = MYNAH_K_GEMV_GROUP_Q6K;
            else if (all_q4k) p->kernel = MYNAH_K_GEMV_GROUP_Q4K;
        }
    }
    return 0;
}

int mynah_gemv_group_threads(mynah_gemv_group *grp, int order, uint32_t *threads) {
    return mynah_gemv_group_geometry(grp, order, threads, NULL);
}

int mynah_gemv_group_geometry(mynah_gemv_group *grp, int order, uint32_t *threads,
                              uint32_t *grid) {
    mynah_device *d = mynah_dev();
    gemv_plan p;
    if (d == NULL || gemv_group_plan(d, grp, order, &p) != 0) return -1;
    if (threads) *threads = p.threads;
    if (grid) *grid = p.grid;
    return 0;
}

const char *mynah_hip_gemv_kernel(int type, size_t rows, size_t cols, int order) {
    mynah_device *d = mynah_dev();
    if (d == NULL) return NULL;
    if (type == MYNAH_Q4_0)
        return kernel_names[rows < 32768u && env_long("MYNAH_Q40_PC", 1) != 0
                                ? MYNAH_K_Q40_CHAIN_PC : MYNAH_K_Q40_CHAIN1];
    if (type == MYNAH_Q4_K && mynah_int8_mode() == MYNAH_INT8_ALL)
        return kernel_names[MYNAH_K_Q4K_GEMV_INT8];
    /* The plan reads shapes and pointer alignment only: stand-in addresses
     * aligned like a device allocation. */
    const uintptr_t fake = 4096;
    mynah_gemv_group g;
    memset(&g, 0, sizeof g);
    g.n = 1;
    if (mynah_gemv_desc_init(&g.d[0], type, (const void *)fake, rows, cols,
                             (const float *)fake, (float *)fake) != 0)
        return NULL;
    gemv_plan p;
    if (gemv_group_plan(d, &g, order, &p) != 0) return NULL;
    return kernel_names[p.kernel];
}

int mynah_gemv_group_launch(mynah_device *d, mynah_gemv_group *grp, hipStream_t stream,
                            uint32_t *tiles_out, int order) {
    gemv_plan p;
    if (gemv_group_plan(d, grp, order, &p) != 0) return -1;
    if (tiles_out) *tiles_out = p.grid;
    if (p.kernel == MYNAH_K_GEMV_STREAM || p.kernel == MYNAH_K_GEMV_STREAM_CVT) {
        void *args[] = {&p.sd};
        return mynah_launch(d, p.kernel, p.grid, 1, p.threads, p.lds, stream, args);
    }
    grp->shape = p.shape;
    grp->pf.host_tiles = p.grid;
    if (grp->pf.wgs % 8u != 0 || grp->pf.n > MYNAH_PF_SEGS) {
        mynah_set_error("prefetch of %u workgroups, %u segments", grp->pf.wgs, grp->pf.n);
        return -1;
    }
    void *args[] = {grp};
    return mynah_launch(d, p.kernel, p.grid + grp->pf.wgs, 1, p.threads, p.lds, stream, args);
}

int mynah_gemv_prefetch_plan(const mynah_gemv_group *next, int order, uint32_t wgs,
                             uint32_t bytes_per_wg, uint64_t max_bytes, uint32_t step_log2,
                             mynah_gemv_prefetch *pf) {
    memset(pf, 0, sizeof *pf);
    if (wgs == 0 && bytes_per_wg == 0) return 0;
    if (wgs % 8u != 0 || step_log2 < 2u || step_log2 > 12u) {
        mynah_set_error("prefetch of %u workgroups, step 2^%u", wgs, step_log2);
        return -1;
    }
    mynah_device *d = mynah_dev();
    if (d == NULL) return -1;
    mynah_gemv_group g = *next;
    gemv_plan p;
    if (gemv_group_plan(d, &g, order, &p) != 0) return -1;
    if (p.kernel == MYNAH_K_GEMV_STREAM || p.kernel == MYNAH_K_GEMV_STREAM_CVT) return 0;
    uint32_t n = 0;
    for (uint32_t i = 0; i < g.n; i++) {
        const mynah_gemv_desc *e = &g.d[i];
        const uint32_t r = p.tile_rows ? p.tile_rows : e->pad;
        const uint32_t end = i + 1 < g.n ? g.d[i + 1].tile0 : p.grid;
        const uint64_t bytes = (uint64_t)e->rows * e->row_bytes;
        if (r == 0 || bytes > 0xffffffffull || (uint64_t)r * e->row_bytes > 0xffffffffull) {
            memset(pf, 0, sizeof *pf);
            return 0;
        }
        const void *w[2] = {e->w, e->w2};
        for (int k = 0; k < 2 && n < MYNAH_PF_SEGS; k++) {
            if (w[k] == NULL) continue;
            pf->base[n] = w[k];
            pf->t0[n] = e->tile0;
            pf->nt[n] = end - e->tile0;
            pf->bpt[n] = r * e->row_bytes;
            pf->bytes[n] = (uint32_t)bytes;
            n++;
        }
    }
    uint64_t total = 0;
    for (uint32_t k = 0; k < n; k++) total += pf->bytes[k];
    if (total > max_bytes) n = 0;
    if (bytes_per_wg != 0) {
        const uint64_t w = (total + bytes_per_wg - 1u) / bytes_per_wg;
        wgs = w >= 1024u ? 1024u : (uint32_t)((w + 7u) & ~7ull);
    }
    pf->n = n;
    pf->wgs = n ? wgs : 0u;
    pf->step_log2 = step_log2;
    return 0;
}

int mynah_dequant_launch(mynah_device *d, int type, const void *w, size_t rows, size_t cols,
                         float *y, hipStream_t stream) {
    size_t rb;
    if (mynah_geometry(type, rows, cols, &rb) != 0) return -1;
    /* Like the reference (kernels.c:2096-2101, 2563-2567): matrix dequant
     * works in 256-value units for every type, ragged Q8_0 rows included,
     * except Q4_0, whose dequant takes any multiple of 32 (kernels.c:2500-2514). */
    if (type != MYNAH_Q4_0 && cols % 256 != 0) {
        mynah_set_error("cols must be a multiple of 256");
        return -1;
    }
    const size_t units = rows * (cols / 32);
    if (units / GEMV_WG + 1 > 0x7fffffffu) {
        mynah_set_error("dequant too large");
        return -1;
    }
    uint32_t t = (uint32_t)type, r = (uint32_t)rows, c = (uint32_t)cols;
    void *args[] = {&w, &y, &t, &r, &c};
    return mynah_launch(d, MYNAH_K_DEQUANT, (unsigned)((units + GEMV_WG - 1) / GEMV_WG), 1,
                        GEMV_WG, 0, stream, args);
}

/* ── host-range registry ─────────────────────────────────────────────────── */

#define MAX_RANGES 64
typedef struct {
    const unsigned char *host;
    size_t bytes;
    unsigned char *alloc;    /* hipMalloc result */
    unsigned char *dev;      /* device address of host[0] */
    int device;
} range;
static range ranges[MAX_RANGES];
static pthread_mutex_t reg_mu = PTHREAD_MUTEX_INITIALIZER;

int mynah_hip_register(const void *host, size_t bytes) {
    mynah_device *d = mynah_dev();
    if (d == NULL) return -1;
    if (host == NULL || bytes == 0) {
        mynah_set_error("register: empty range");
        return -1;
    }
    const size_t skew = (uintptr_t)host & 255u;
    unsigned char *alloc = NULL;
    HIP_OK(hipMalloc((void **)&alloc, bytes + skew), "hipMalloc(register)");
    if (hipMemcpy(alloc + skew, host, bytes, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(alloc);
        mynah_set_error("register: upload failed");
        return -1;
    }
    pthread_mutex_lock(&reg_mu);
    int slot = -1;
    for (int i = 0; i < MAX_RANGES; i++)
        if (ranges[i].host == NULL) { slot = i; break; }
    if (slot >= 0) {
        ranges[slot].host = (const unsigned char *)host;
        ranges[slot].bytes = bytes;
        ranges[slot].alloc = alloc;
        ranges[slot].dev = alloc + skew;
        ranges[slot].device = current_device;
    }
    pthread_mutex_unlock(&reg_mu);
    if (slot < 0) {
        (void)hipFree(alloc);
        mynah_set_error("register: too many ranges (max %d)", MAX_RANGES);
        return -1;
    }
    return 0;
}

int mynah_hip_unregister(const void *host) {
    pthread_mutex_lock(&reg_mu);
    int found = -1;
    for (int i = 0; i < MAX_RANGES; i++)
        if (ranges[i].host == (const unsigned char *)host) { found = i; break; }
    range r = found >= 0 ? ranges[found] : (range){0};
    if (found >= 0) memset(&ranges[found], 0, sizeof ranges[found]);
    pthread_mutex_unlock(&reg_mu);
    if (found < 0) {
        mynah_set_error("unregister: unknown range");
        return -1;
    }
    (void)hipSetDevice(r.device);
    HIP_OK(hipDeviceSynchronize(), "hipDeviceSynchronize");
    HIP_OK(hipFree(r.alloc), "hipFree(register)");
    return 0;
}

/* Device address for [host, host + bytes) if it lies inside one range. */
static const void *lookup(const void *host, size_t bytes) {
    const unsigned char *p = (const unsigned char *)host;
    const void *out = NULL;
    pthread_mutex_lock(&reg_mu);
    for (int i = 0; i < MAX_RANGES; i++) {
        const range *r = &ranges[i];
        if (r->host != NULL && r->device == current_device && p >= r->host &&
            (size_t)(p - r->host) <= r->bytes && bytes <= r->bytes - (size_t)(p - r->host)) {
            out = r->dev + (p - r->host);
            break;
        }
    }
    pthread_mutex_unlock(&reg_mu);
    return out;
}

void *mynah_hip_device_ptr(const void *host) { return (void *)lookup(host, 1); }

/* ── host-pointer entry points (the ingot ABI) ───────────────────────────── */

/* Staging buffers reused across calls (grown, never shrunk). */
static unsigned char *stage_w, *stage_x, *stage_y;
static size_t cap_w, cap_x, cap_y;

static int grow(unsigned char **buf, size_t *cap, size_t need) {
    if (need <= *cap) return 0;
    if (*buf) (void)hipFree(*buf);
    *buf = NULL;
    *cap = 0;
    size_t n = need < 4096 ? 4096 : need + need / 4;
    HIP_OK(hipMalloc((void **)buf, n), "hipMalloc(staging)");
    *cap = n;
    return 0;
}

typedef enum {
    OP_MATVEC, OP_MATVEC_EXACT, OP_MATVEC_INT8, OP_MATMAT, OP_MATMAT_EXACT, OP_DEQUANT
} host_op;

static int host_call(host_op op, int type, const void *w, size_t rows, size_t cols,
                     const float *x, float *y, size_t tokens) {
    if (w == NULL || y == NULL || (op != OP_DEQUANT && x == NULL) || tokens == 0) {
        mynah_set_error("null argument");
        return -1;
    }
    size_t rb;
    if (mynah_geometry(type, rows, cols, &rb) != 0) return -1;
    if (op == OP_MATMAT && tokens > SIZE_MAX / (rows > cols ? rows : cols) / sizeof(float)) {
        mynah_set_error("size overflow");
        return -1;
    }
    mynah_device *d = mynah_dev();
    if (d == NULL) return -1;
    pthread_mutex_lock(&host_mu);
    int rc = -1;
    const size_t wbytes = rows * rb;
    const size_t xbytes = op == OP_DEQUANT ? 0 : tokens * cols * sizeof(float);
    const size_t ybytes = (op == OP_DEQUANT ? rows * cols : tokens * rows) * sizeof(float);
    const void *wd = lookup(w, wbytes);
    hipStream_t s = d->stream;
    /* The reference reads blocks at any address (test_quant.c:208-295); a
     * registered copy keeps the host address's skew, so a tensor that sits
     * off the kernels' word alignment is staged into an aligned buffer. */
    if (wd != NULL && mynah_w_misaligned(type, wd)) wd = NULL;
    if (wd == NULL) {
        if (grow(&stage_w, &cap_w, wbytes) != 0) goto out;
        if (hipMemcpyAsync(stage_w, w, wbytes, hipMemcpyHostToDevice, s) != hipSuccess) {
            mynah_set_error("weight upload failed");
            goto out;
        }
        wd = stage_w;
    }
    if (grow(&stage_y, &cap_y, ybytes) != 0) goto out;
    if (xbytes) {
        if (grow(&stage_x, &cap_x, xbytes) != 0) goto out;
        if (hipMemcpyAsync(stage_x, x, xbytes, hipMemcpyHostToDevice, s) != hipSuccess) {
            mynah_set_error("input upload failed");
            goto out;
        }
    }
    if (op == OP_MATVEC || op == OP_MATVEC_EXACT)
        rc = gemv_launch(d, type, wd, rows, cols, (const float *)stage_x, (float *)stage_y, s,
                         op == OP_MATVEC);
    else if (op == OP_MATVEC_INT8) rc = mynah_int8_product(d, MYNAH_Q4_K, wd, rows, cols,
                                                           (const float *)stage_x,
                                                           (float *)stage_y, 1, s);
    else if (op == OP_MATMAT || op == OP_MATMAT_EXACT)
        rc = mynah_matmat_launch(d, type, wd, rows, cols, (const float *)stage_x,
                                 (float *)stage_y, tokens, op == OP_MATMAT_EXACT, s);
    else rc = mynah_dequant_launch(d, type, wd, rows, cols, (float *)stage_y, s);
    if (rc != 0) goto out;
    rc = -1;
    if (hipMemcpyAsync(y, stage_y, ybytes, hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess) {
        mynah_set_error("result download failed");
        goto out;
    }
    rc = 0;
out:
    pthread_mutex_unlock(&host_mu);
    return rc;
}

int ingot_matvec(int type, const void *weights, size_t rows, size_t cols,
                 const float *input, float *output) {
    return host_call(OP_MATVEC, type, weights, rows, cols, input, output, 1);
}

int ingot_matmat(int type, const void *weights, size_t rows, size_t cols,
                 const float *input, float *output, size_t tokens) {
    return host_call(tokens == 1 ? OP_MATVEC : OP_MATMAT, type, weights, rows, cols, input,
                     output, tokens);
}

int ingot_dequant_matrix(int type, const void *weights, size_t rows, size_t cols,
                         float *output) {
    return host_call(OP_DEQUANT, type, weights, rows, cols, NULL, output, 1);
}

int ingot_has_kernel(int type) {
    return type == MYNAH_Q4_K || type == MYNAH_Q5_K || type == MYNAH_Q6_K ||
           type == MYNAH_Q8_0 || type == MYNAH_Q4_0;
}

int ingot_matmat_is_exact(size_t tokens) {
    if (tokens <= 1) return 1;
    return mynah_int8_mode() == MYNAH_INT8_OFF;
}

#define PER_TYPE(prefix, id)                                                              \
    int ingot_##prefix##_matvec(const void *w, size_t rows, size_t cols, const float *x,   \
                                float *y) {                                                \
        return ingot_matvec(id, w, rows, cols, x, y);                                      \
    }                                                                                      \
    int ingot_##prefix##_dequant(const void *w, size_t rows, size_t cols, float *y) {      \
        return ingot_dequant_matrix(id, w, rows, cols, y);                                 \
    }                                                                                      \
    int ingot_##prefix##_matmat(const void *w, size_t rows, size_t cols, const float *x,   \
                                float *y, size_t tokens) {                                 \
        return ingot_matmat(id, w, rows, cols, x, y, tokens);                              \
    }
PER_TYPE(q4_k, MYNAH_Q4_K)
PER_TYPE(q5_k, MYNAH_Q5_K)
PER_TYPE(q6_k, MYNAH_Q6_K)
PER_TYPE(q8_0, MYNAH_Q8_0)
#undef PER_TYPE

/* The as-built Q5_K matvec is its scalar lane (kernels.c:1924-1939 without
 * -march), so the scalar entry point gives the same bits. */
int ingot_q5_k_matvec_scalar(const void *w, size_t rows, size_t cols, const float *x, float *y) {
    return ingot_matvec(MYNAH_Q5_K, w, rows, cols, x, y);
}

int ingot_q5_k_matmat_exact(const void *w, size_t rows, size_t cols, const float *x, float *y,
                            size_t tokens) {
    return host_call(tokens == 1 ? OP_MATVEC : OP_MATMAT_EXACT, MYNAH_Q5_K, w, rows, cols, x, y,
                     tokens);
}

int ingot_q4_0_matvec(const void *w, size_t rows, size_t cols, const float *x, float *y) {
    return ingot_matvec(MYNAH_Q4_0, w, rows, cols, x, y);
}

int ingot_q4_0_dequant(const void *w, size_t rows, size_t cols, float *y) {
    return ingot_dequant_matrix(MYNAH_Q4_0, w, rows, cols, y);
}

int ingot_q4_k_matmat_exact(const void *w, size_t rows, size_t cols, const float *x, float *y,
                            size_t tokens) {
    return host_call(tokens == 1 ? OP_MATVEC : OP_MATMAT_EXACT, MYNAH_Q4_K, w, rows, cols, x, y,
                     tokens);
}

int ingot_q4_k_matvec_int8(const void *w, size_t rows, size_t cols, const float *x, float *y) {
    return host_call(OP_MATVEC_INT8, MYNAH_Q4_K, w, rows, cols, x, y, 1);
}

/* kernels.c:319-337: the scalar lane whatever the build or INGOT_SDOT; the
 * exact order is that lane's, so this is the exact matvec with the int8
 * lane bypassed. */
int ingot_q4_k_matvec_scalar(const void *w, size_t rows, size_t cols, const float *x, float *y) {
    return host_call(OP_MATVEC_EXACT, MYNAH_Q4_K, w, rows, cols, x, y, 1);
}

/* The reference's tensor descriptor (third_party/ingot/include/ingot/gguf.h:41-50)
 * and data accessor (gguf.h:74-76), resolved from the host process. */
typedef struct {
    const char *name;
    int type;
    uint32_t rank;
    uint64_t ne[8];
    uint64_t nelem, nbytes, offset;
    uint32_t shard;
} ingot_tensor_view;
extern const void *ingot_gguf_data(const void *g, const void *t) __attribute__((weak));

/* generic.c:148-155: ggml's ne[0] is the input width, so rows = ne[1] and
 * cols = ne[0]; rank 1 is one row; rank 0, rank > 2 and zero dimensions are
 * refused. The data pointer is looked up first, as there (generic.c:161). */
static const void *gguf_tensor(const void *g, const void *t, size_t *rows, size_t *cols) {
    if (ingot_gguf_data == NULL) {
        mynah_set_error("ingot_gguf_data is not linked into this process");
        return NULL;
    }
    const void *w = ingot_gguf_data(g, t);
    if (w == NULL) {
        mynah_set_error("tensor data not found");
        return NULL;
    }
    const ingot_tensor_view *tv = (const ingot_tensor_view *)t;
    if (tv->rank == 0 || tv->rank > 2) {
        mynah_set_error("tensor rank %u is not 1 or 2", tv->rank);
        return NULL;
    }
    *cols = (size_t)tv->ne[0];
    *rows = tv->rank == 2 ? (size_t)tv->ne[1] : 1;
    if (*rows == 0 || *cols == 0) {
        mynah_set_error("tensor has a zero dimension");
        return NULL;
    }
    return w;
}

/* quant.h:179-183 (generic.c:157-173) */
int ingot_gguf_matmat(const void *g, const void *t, const float *input, float *output,
                      size_t tokens) {
    size_t rows, cols;
    const void *w = gguf_tensor(g, t, &rows, &cols);
    if (w == NULL) return -1;
    return ingot_matmat(((const ingot_tensor_view *)t)->type, w, rows, cols, input, output,
                        tokens);
}

int ingot_gguf_matvec(const void *g, const void *t, const float *input, float *output) {
    return ingot_gguf_matmat(g, t, input, output, 1);
}

int ingot_gguf_dequant_matrix(const void *g, const void *t, float *output) {
    size_t rows, cols;
    const void *w = gguf_tensor(g, t, &rows, &cols);
    if (w == NULL) return -1;
    return ingot_dequant_matrix(((const ingot_tensor_view *)t)->type, w, rows, cols, output);
}

/* ── device-resident API ─────────────────────────────────────────────────── */

int mynah_hip_matvec_dev(int type, const void *w, size_t rows, size_t cols, const float *x,
                         float *y, void *stream) {
    mynah_device *d = mynah_dev();
    if (d == NULL) return -1;
    if (w == NULL || x == NULL || y == NULL) {
        mynah_set_error("null argument");
        return -1;
    }
    return mynah_gemv_launch(d, type, w, rows, cols, x, y, mynah_stream_or_default(d, stream));
}

int mynah_hip_matmat_mv_dev(int type, const void *w, size_t rows, size_t cols, const float *x,
                            float *y, size_t tokens, const float *res, void *stream) {
    mynah_device *d = mynah_dev();
    if (d == NULL) return -1;
    if (w == NULL || x == NULL || y == NULL || tokens == 0) {
        mynah_set_error("null argument");
        return -1;
    }
    return mynah_matmat_mv_launch(d, type, w, rows, cols, x, y, tokens, res,
                                  mynah_stream_or_default(d, stream));
}

int mynah_hip_matmat_dev(int type, const void *w, size_t rows, size_t cols, const float *x,
                         float *y, size_t tokens, void *stream) {
    mynah_device *d = mynah_dev();
    if (d == NULL) return -1;
    if (w == NULL || x == NULL || y == NULL || tokens == 0) {
        mynah_set_error("null argument");
        return -1;
    }
    hipStream_t s = mynah_stream_or_default(d, stream);
    if (tokens == 1) return mynah_gemv_launch(d, type, w, rows, cols, x, y, s);
    return mynah_matmat_launch(d, type, w, rows, cols, x, y, tokens, 0, s);
}

int mynah_hip_dequant_dev(int type, const void *w, size_t rows, size_t cols, float *y,
                          void *stream) {
    mynah_device *d = mynah_dev();
    if (d == NULL) return -1;
    if (w == NULL || y == NULL) {
        mynah_set_error("null argument");
        return -1;
    }
    return mynah_dequant_launch(d, type, w, rows, cols, y, mynah_stream_or_default(d, stream));
}

void *mynah_hip_alloc(size_t bytes) {
    if (mynah_dev() == NULL) return NULL;
    void *p = NULL;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) {
        mynah_set_error("hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
        return NULL;
    }
    return p;
}

int mynah_hip_free(void *p) {
    if (p == NULL) return 0;
    if (mynah_dev() == NULL) return -1;
    HIP_OK(hipFree(p), "hipFree");
    return 0;
}

int mynah_hip_h2d(void *dst, const void *src, size_t bytes) {
    if (mynah_dev() == NULL) return -1;
    HIP_OK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
    return 0;
}

int mynah_hip_d2h(void *dst, const void *src, size_t bytes) {
    if (mynah_dev() == NULL) return -1;
    HIP_OK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    return 0;
}

int mynah_hip_memset(void *dst, int value, size_t bytes) {
    if (mynah_dev() == NULL) return -1;
    HIP_OK(hipMemset(dst, value, bytes), "hipMemset");
    return 0;
}

int mynah_hip_copy_dev(void *dst, const void *src, size_t bytes, void *stream) {
    mynah_device *d = mynah_dev();
    if (d == NULL) return -1;
    if (dst == NULL || src == NULL || bytes == 0 || bytes % 16 != 0 ||
        ((uintptr_t)dst & 15u) != 0 || ((uintptr_t)src & 15u) != 0) {
        mynah_set_error("copy needs 16-byte aligned buffers and a multiple of 16 bytes");
        return -1;
    }
    uint64_t n16 = bytes / 16;
    uint64_t want = (n16 + 255) / 256;
    unsigned grid = (unsigned)(want < 8192 ? want : 8192);
    void *args[] = {&src, &dst, &n16};
    return mynah_launch(d, MYNAH_K_COPY16, grid, 1, 256, 0, mynah_stream_or_default(d, stream),
                        args);
}

int mynah_hip_read_dev(const void *src, size_t bytes, void *sink, void *stream) {
    mynah_device *d = mynah_dev();
    if (d == NULL) return -1;
    if (src == NULL || sink == NULL || bytes == 0 || bytes % 16 != 0 ||
        ((uintptr_t)src & 15u) != 0 || ((uintptr_t)sink & 3u) != 0) {
        mynah_set_error("read needs a 16-byte aligned source, a multiple of 16 bytes and a sink");
        return -1;
    }
    uint64_t n16 = bytes / 16;
    /* At least four workgroups per CU where the size allows, up to eight
     * chunks per thread. */
    uint64_t per = n16 / (256u * 4u * (uint64_t)d->cus);
    if (per < 1) per = 1;
    if (per > 8) per = 8;
    uint64_t want = (n16 + 256u * per - 1) / (256u * per);
    unsigned grid = (unsigned)(want < 65535 ? want : 65535);
    void *args[] = {&src, &n16, &sink};
    return mynah_launch(d, MYNAH_K_READ16, grid, 1, 256, 0, mynah_stream_or_default(d, stream),
                        args);
}

int mynah_hip_mfma_probe(const float *a, const float *b, const float *c, float *prod,
                         float *acc, float *mul, float *fused, uint32_t waves, void *stream) {
    mynah_device *d = mynah_dev();
    if (d == NULL) return -1;
    if (a == NULL || b == NULL || c == NULL || prod == NULL || acc == NULL || mul == NULL ||
        fused == NULL || waves == 0 || waves > 65535u) {
        mynah_set_error("mfma probe: null buffer or waves outside 1..65535");
        return -1;
    }
    void *args[] = {&a, &b, &c, &prod, &acc, &mul, &fused};
    return mynah_launch(d, MYNAH_K_MFMA_PROBE, waves, 1, 64, 0,
                        mynah_stream_or_default(d, stream), args);
}

int mynah_hip_valu_add_rate(uint32_t iters, float *ns_per_instr, uint32_t *simds) {
    mynah_device *d = mynah_dev();
    if (d == NULL) return -1;
    if (ns_per_instr == NULL || iters == 0) {
        mynah_set_error("valu rate: null output or zero iterations");
        return -1;
    }
    /* Eight waves per SIMD: 4-wave workgroups, two per SIMD's worth. */
    const unsigned grid = 8u * (unsigned)d->cus;
    float *sink = NULL;
    HIP_OK(hipMalloc((void **)&sink, 4), "hipMalloc(valu rate sink)");
    float c = 1.0001f, never = -1.0f;
    hipEvent_t e0 = NULL, e1 = NULL;
    int rc = -1;
    if (hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess) {
        void *args[] = {&iters, &c, &never, &sink};
        float ms = 0.0f;
        rc = mynah_launch(d, MYNAH_K_VALU_ADD_RATE, grid, 1, 256, 0, d->stream, args);
        rc = rc ? rc : (hipEventRecord(e0, d->stream) == hipSuccess ? 0 : -1);
        rc = rc ? rc : mynah_launch(d, MYNAH_K_VALU_ADD_RATE, grid, 1, 256, 0, d->stream, args);
        rc = rc ? rc : (hipEventRecord(e1, d->stream) == hipSuccess ? 0 : -1);
        rc = rc ? rc : (hipEventSynchronize(e1) == hipSuccess ? 0 : -1);
        rc = rc ? rc : (hipEventElapsedTime(&ms, e0, e1) == hipSuccess ? 0 : -1);
        /* wave64 adds per SIMD: 8 waves x iters x 8 chains */
        if (rc == 0) {
            *ns_per_instr = ms * 1e6f / (8.0f * (float)iters * 8.0f);
            if (simds) *simds = 4u * (uint32_t)d->cus;
        }
        else mynah_set_error("valu rate: launch or event failed");
    } else {
        mynah_set_error("valu rate: hipEventCreate failed");
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipFree(sink);
    return rc;
}

int mynah_hip_expf_dev(const float *x, float *y, size_t n, void *stream) {
    mynah_device *d = mynah_dev();
    if (d == NULL) return -1;
    if (x == NULL || y == NULL) {
        mynah_set_error("null argument");
        return -1;
    }
    if (n == 0) return 0;
    uint64_t n64 = n;
    const uint64_t want = (n64 + 255) / 256;
    const unsigned grid = (unsigned)(want < 8192 ? want : 8192);
    void *args[] = {&x, &y, &n64};
    return mynah_launch(d, MYNAH_K_EXPF, grid, 1, 256, 0, mynah_stream_or_default(d, stream),
                        args);
}

int mynah_hip_sync(void *stream) {
    mynah_device *d = mynah_dev();
    if (d == NULL) return -1;
    HIP_OK(hipStreamSynchronize(mynah_stream_or_default(d, stream)), "hipStreamSynchronize");
    return 0;
}

void *mynah_hip_stream(void) {
    mynah_device *d = mynah_dev();
    return d ? (void *)d->stream : NULL;
}

int mynah_hip_time_matvec(int type, const void *const *w_copies, int n_copies, size_t rows,
                          size_t cols, const float *x, float *y, int iters, float *ms) {
    mynah_device *d = mynah_dev();
    if (d == NULL) return -1;
    if (w_copies == NULL || n_copies <= 0 || iters <= 0 || ms == NULL) {
        mynah_set_error("bad timing arguments");
        return -1;
    }
    hipEvent_t a, b;
    HIP_OK(hipEventCreate(&a), "hipEventCreate");
    if (hipEventCreate(&b) != hipSuccess) {
        (void)hipEventDestroy(a);
        mynah_set_error("hipEventCreate");
        return -1;
    }
    int rc = 0;
    if (hipEventRecord(a, d->stream) != hipSuccess) rc = -1;
    for (int i = 0; i < iters && rc == 0; i++)
        rc = mynah_gemv_launch(d, type, w_copies[i % n_copies], rows, cols, x, y, d->stream);
    if (rc == 0 && (hipEventRecord(b, d->stream) != hipSuccess ||
                    hipEventSynchronize(b) != hipSuccess ||
                    hipEventElapsedTime(ms, a, b) != hipSuccess)) {
        mynah_set_error("event timing failed");
        rc = -1;
    }
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    return rc;
}

void *mynah_hip_event_create(void) {
    if (mynah_dev() == NULL) return NULL;
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) {
        mynah_set_error("hipEventCreate failed");
        return NULL;
    }
    return (void *)e;
}

int mynah_hip_event_record(void *event, void *stream) {
    mynah_device *d = mynah_dev();
    if (d == NULL) return -1;
    HIP_OK(hipEventRecord((hipEvent_t)event, mynah_stream_or_default(d, stream)), "hipEventRecord");
    return 0;
}

int mynah_hip_event_elapsed(void *start, void *end, float *ms) {
    HIP_OK(hipEventSynchronize((hipEvent_t)end), "hipEventSynchronize");
    HIP_OK(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end), "hipEventElapsedTime");
    return 0;
}

int mynah_hip_event_destroy(void *event) {
    HIP_OK(hipEventDestroy((hipEvent_t)event), "hipEventDestroy");
    return 0;
}

int mynah_hip_time_sweep(int n, const int *types, const void *const *w, int copies,
                         const size_t *rows, const size_t *cols, const float *const *x,
                         float *const *y, int steps, int timed, int every, float *ms_total,
                         float *ms_timed) {
    mynah_device *d = mynah_dev();
    if (d == NULL) return -1;
    if (n <= 0 || copies <= 0 || steps <= 0 || types == NULL || w == NULL || rows == NULL ||
        cols == NULL || x == NULL || y == NULL || ms_total == NULL || ms_timed == NULL ||
        timed >= n || every <= 0) {
        mynah_set_error("bad sweep arguments");
        return -1;
    }
    hipEvent_t a = NULL, b = NULL;
    hipEvent_t *ev = (hipEvent_t *)calloc((size_t)2 * steps, sizeof *ev);
    int rc = ev ? 0 : -1;
    if (rc == 0 && (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess)) rc = -1;
    for (int i = 0; rc == 0 && timed >= 0 && i < 2 * steps; i++)
        if (hipEventCreate(&ev[i]) != hipSuccess) rc = -1;
    if (rc == 0 && hipEventRecord(a, d->stream) != hipSuccess) rc = -1;
    for (int i = 0; rc == 0 && i < steps; i++) {
        const int mark = i % every == 0;
        for (int m = 0; rc == 0 && m < n; m++) {
            if (m == timed && mark) (void)hipEventRecord(ev[2 * i], d->stream);
            rc = mynah_gemv_launch(d, types[m], w[(size_t)m * copies + (size_t)(i % copies)],
                                   rows[m], cols[m], x[m], y[m], d->stream);
            if (m == timed && mark) (void)hipEventRecord(ev[2 * i + 1], d->stream);
        }
    }
    if (rc == 0 && (hipEventRecord(b, d->stream) != hipSuccess ||
                    hipEventSynchronize(b) != hipSuccess ||
                    hipEventElapsedTime(ms_total, a, b) != hipSuccess))
        rc = -1;
    *ms_timed = 0.0f;
    int marked = 0;
    for (int i = 0; rc == 0 && timed >= 0 && i < steps; i += every) {
        float t = 0.0f;
        if (hipEventElapsedTime(&t, ev[2 * i], ev[2 * i + 1]) != hipSuccess) rc = -1;
        *ms_timed += t;
        marked++;
    }
    if (marked > 0) *ms_timed /= (float)marked;
    if (rc != 0 && mynah_hip_last_error()[0] == 0) mynah_set_error("sweep timing failed");
    for (int i = 0; ev && timed >= 0 && i < 2 * steps; i++)
        if (ev[i]) (void)hipEventDestroy(ev[i]);
    free(ev);
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    return rc;
}
