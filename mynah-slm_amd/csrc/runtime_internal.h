/* runtime_internal.h — shared by the C11 host files of the library.
 *
 * SPDX-License-Identifier: MIT */
#ifndef MYNAH_RUNTIME_INTERNAL_H
#define MYNAH_RUNTIME_INTERNAL_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

enum { MYNAH_Q4_0 = 2, MYNAH_Q8_0 = 8, MYNAH_Q4_K = 12, MYNAH_Q5_K = 13, MYNAH_Q6_K = 14 };

/* Every kernel of the embedded code object: id and symbol name. */
#define MYNAH_KERNEL_LIST(X)                          \
    X(MYNAH_K_DEQUANT, "mynah_dequant")                 \
    X(MYNAH_K_Q4K_GEMM, "mynah_q4k_gemm_exact")        \
    X(MYNAH_K_Q5K_GEMM, "mynah_q5k_gemm_exact")        \
    X(MYNAH_K_Q5K_GEMM_MV, "mynah_q5k_gemm_mv")        \
    X(MYNAH_K_Q40_CHAIN1, "mynah_q40_chain1")          \
    X(MYNAH_K_Q40_CHAIN2, "mynah_q40_chain2")          \
    X(MYNAH_K_Q40_CHAIN4, "mynah_q40_chain4")          \
    X(MYNAH_K_Q40_CHAIN8, "mynah_q40_chain8")          \
    X(MYNAH_K_Q40_CHAIN_PC, "mynah_q40_chain_pc")      \
    X(MYNAH_K_Q6K_GEMM, "mynah_q6k_gemm_exact")        \
    X(MYNAH_K_Q80_GEMM, "mynah_q80_gemm_exact")        \
    X(MYNAH_K_Q4K_GEMM_MV, "mynah_q4k_gemm_mv")        \
    X(MYNAH_K_Q6K_GEMM_MV, "mynah_q6k_gemm_mv")        \
    X(MYNAH_K_Q80_GEMM_MV, "mynah_q80_gemm_mv")        \
    X(MYNAH_K_Q4K_GEMM_MFMA, "mynah_q4k_gemm_exact_mfma") \
    X(MYNAH_K_Q5K_GEMM_MFMA, "mynah_q5k_gemm_exact_mfma") \
    X(MYNAH_K_Q6K_GEMM_MFMA, "mynah_q6k_gemm_exact_mfma") \
    X(MYNAH_K_Q80_GEMM_MFMA, "mynah_q80_gemm_exact_mfma") \
    X(MYNAH_K_Q4K_GEMM_MV_MFMA, "mynah_q4k_gemm_mv_mfma") \
    X(MYNAH_K_Q5K_GEMM_MV_MFMA, "mynah_q5k_gemm_mv_mfma") \
    X(MYNAH_K_Q6K_GEMM_MV_MFMA, "mynah_q6k_gemm_mv_mfma") \
    X(MYNAH_K_Q80_GEMM_MV_MFMA, "mynah_q80_gemm_mv_mfma") \
    X(MYNAH_K_GEMM_FOLD, "mynah_gemm_fold")            \
    X(MYNAH_K_GEMV_GROUP, "mynah_gemv_group")          \
    X(MYNAH_K_GEMV_GROUP_Q6K, "mynah_gemv_group_q6k")  \
    X(MYNAH_K_GEMV_GROUP_Q4K, "mynah_gemv_group_q4k")  \
    X(MYNAH_K_GEMV_FLAT_Q4K, "mynah_gemv_flat_q4k")    \
    X(MYNAH_K_GEMV_FLAT_Q6K, "mynah_gemv_flat_q6k")    \
    X(MYNAH_K_GEMV_PC_Q4K, "mynah_gemv_pc_q4k")        \
    X(MYNAH_K_GEMV_STREAM, "mynah_gemv_stream")        \
    X(MYNAH_K_GEMV_STREAM_CVT, "mynah_gemv_stream_cvt") \
    X(MYNAH_K_GEMV_FAST_GROUP, "mynah_gemv_fast_group") \
    X(MYNAH_K_ATTN_SCORES, "mynah_attn_scores")        \
    X(MYNAH_K_ATTN_OUT, "mynah_attn_out")              \
    X(MYNAH_K_ATTN_SOFTMAX, "mynah_attn_softmax")      \
    X(MYNAH_K_ATTN_OUT_LONG, "mynah_attn_out_long")    \
    X(MYNAH_K_ATTN_PV_1, "mynah_attn_pv_1")            \
    X(MYNAH_K_ATTN_PV_2, "mynah_attn_pv_2")            \
    X(MYNAH_K_ATTN_PV_3, "mynah_attn_pv_3")            \
    X(MYNAH_K_ATTN_PV_4, "mynah_attn_pv_4")            \
    X(MYNAH_K_ATTN_PV_M, "mynah_attn_pv_m")            \
    X(MYNAH_K_ATTN_SPLIT, "mynah_attn_split")          \
    X(MYNAH_K_ATTN_SPLIT_G2_32, "mynah_attn_split_g2_32") \
    X(MYNAH_K_ATTN_SPLIT_G2_64, "mynah_attn_split_g2_64") \
    X(MYNAH_K_ATTN_SPLIT_G2_128, "mynah_attn_split_g2_128") \
    X(MYNAH_K_ATTN_SPLIT_G4_32, "mynah_attn_split_g4_32") \
    X(MYNAH_K_ATTN_SPLIT_G4_64, "mynah_attn_split_g4_64") \
    X(MYNAH_K_ATTN_SPLIT_G4_128, "mynah_attn_split_g4_128") \
    X(MYNAH_K_ATTN_COMBINE, "mynah_attn_combine")      \
    X(MYNAH_K_ATTN_COMBINE1, "mynah_attn_combine1")    \
    X(MYNAH_K_ARGMAX, "mynah_argmax_advance")          \
    X(MYNAH_K_SAMP_PENALIZE, "mynah_samp_penalize")    \
    X(MYNAH_K_SAMP_EXP, "mynah_samp_exp")              \
    X(MYNAH_K_SAMP_TOPK, "mynah_samp_topk")            \
    X(MYNAH_K_SAMP_PICK, "mynah_samp_pick")            \
    X(MYNAH_K_RMSNORM, "mynah_rmsnorm")                \
    X(MYNAH_K_EMBED, "mynah_embed_row")                \
    X(MYNAH_K_RMSNORM_ROWS, "mynah_rmsnorm_rows")      \
    X(MYNAH_K_SWIGLU_ROWS, "mynah_swiglu_rows")        \
    X(MYNAH_K_EMBED_ROWS, "mynah_embed_rows")          \
    X(MYNAH_K_PREFILL_ROPE, "mynah_prefill_rope")      \
    X(MYNAH_K_PREFILL_SCORES, "mynah_prefill_scores")  \
    X(MYNAH_K_PREFILL_SOFTMAX, "mynah_prefill_softmax") \
    X(MYNAH_K_PREFILL_PV, "mynah_prefill_pv")          \
    X(MYNAH_K_COPY16, "mynah_copy16")                  \
    X(MYNAH_K_READ16, "mynah_read16")                  \
    X(MYNAH_K_VALU_ADD_RATE, "mynah_valu_add_rate")  \
    X(MYNAH_K_MFMA_PROBE, "mynah_mfma_probe")          \
    X(MYNAH_K_EXPF, "mynah_expf_map")                  \
    X(MYNAH_K_Q8_QUANTIZE, "mynah_q8_quantize")        \
    X(MYNAH_K_Q4K_GEMV_INT8, "mynah_q4k_gemv_int8")    \
    X(MYNAH_K_Q4K_GEMM_INT8_11, "mynah_q4k_gemm_int8_11") \
    X(MYNAH_K_Q4K_GEMM_INT8_12, "mynah_q4k_gemm_int8_12") \
    X(MYNAH_K_Q4K_GEMM_INT8_21, "mynah_q4k_gemm_int8_21") \
    X(MYNAH_K_Q4K_GEMM_INT8_22, "mynah_q4k_gemm_int8_22") \
    X(MYNAH_K_Q5K_GEMM_INT8_22, "mynah_q5k_gemm_int8_22")

enum {
#define X(id, name) id,
    MYNAH_KERNEL_LIST(X)
#undef X
    MYNAH_K_COUNT
};

#define MYNAH_MAX_DEVICES 16

/* Positions per workgroup of the generic split attention kernel (decode.hip
 * AS_CH); the kernels for 2 and 4 query heads per key head take 32, 64 or
 * 128, chosen by the context length. */
/* Dimensions per workgroup of the exact attention's PV kernel (= PV_SW in
 * decode.hip). */
#define MYNAH_PV_SW 16
/* Loader waves of the exact attention's PV kernel (= DPV_LW in decode.hip). */
#ifndef MYNAH_PV_LW
#define MYNAH_PV_LW 4
#endif
#define MYNAH_AS_CH 32
/* Most chunks mynah_attn_combine1 (one wave per query head) takes. */
#define MYNAH_AC1_MAX 32

typedef struct {
    int loaded;
    hipModule_t module;
    hipFunction_t fn[MYNAH_K_COUNT];
    hipStream_t stream;
    int cus;                  /* compute units (sizes the persistent launches) */
    /* Device address and size of the code object's fixed workspace
     * (mynah_scratch, int8.hip), resolved once when the module loads. */
    unsigned char *scratch;
    size_t scratch_bytes;
    /* Device address of mynah_index_sums (common.hip.h), the switch that
     * sends every norm and softmax sum through the index-order path. */
    uint32_t *index_sums;
} mynah_device;

void mynah_set_error(const char *fmt, ...);
mynah_device *mynah_dev(void);
hipStream_t mynah_stream_or_default(mynah_device *d, void *stream);
int mynah_launch(mynah_device *d, int kernel, unsigned gx, unsigned gy, unsigned block,
                 size_t shmem, hipStream_t stream, void **args);
int mynah_launch3(mynah_device *d, int kernel, unsigned gx, unsigned gy, unsigned gz,
                  unsigned block, size_t shmem, hipStream_t stream, void **args);
int mynah_geometry(int type, size_t rows, size_t cols, size_t *row_bytes);
/* Alignment the kernels need of a weight pointer of `type`: 16 bytes for the
 * super-blocks read as uint4 (Q4_K, Q5_K), 2 bytes otherwise. */
static inline int mynah_w_misaligned(int type, const void *w) {
    const uintptr_t m = (type == MYNAH_Q4_K || type == MYNAH_Q5_K) ? 15u : 1u;
    return ((uintptr_t)w & m) != 0;
}
/* Q4_0 products (gemv_q40.hip): y[t][r] for tokens >= 1, the reference's
 * single running sum per (row, token) — the matvec's order and the batched
 * product's alike. res (NULL, or may equal y): y = res + that sum. */
int mynah_q40_launch(mynah_device *d, const void *w, size_t rows, size_t cols, const float *x,
                     float *y, size_t tokens, const float *res, hipStream_t stream);

int mynah_gemv_launch(mynah_device *d, int type, const void *w, size_t rows, size_t cols,
                      const float *x, float *y, hipStream_t stream);
int mynah_dequant_launch(mynah_device *d, int type, const void *w, size_t rows, size_t cols,
                         float *y, hipStream_t stream);
/* exact != 0 keeps the exact batched order whatever the int8 lane's mode
 * (ingot_q4_k_matmat_exact). */
int mynah_matmat_launch(mynah_device *d, int type, const void *w, size_t rows, size_t cols,
                        const float *x, float *y, size_t tokens, int exact, hipStream_t stream);

/* int8 activation lane (int8.c): the current mode (MYNAH_INT8_*), the
 * quantiser, the product on quantised activations (tokens == 1: the matvec
 * epilogue, else the batched one), and both behind one call with a
 * stream-ordered workspace. */
int mynah_int8_mode(void);
int mynah_q8_quantize_launch(mynah_device *d, const float *x, size_t tokens, size_t cols,
                             int8_t *xq, float *xs, int32_t *xsum, hipStream_t stream);
int mynah_q4k_int8_launch(mynah_device *d, int type, const void *w, size_t rows, size_t cols,
                          const int8_t *xq, const float *xs, const int32_t *xsum, float *y,
                          size_t tokens, hipStream_t stream);
/* type: Q4_K (any token count) or Q5_K (tokens >= 2, the batched lane only). */
int mynah_int8_product(mynah_device *d, int type, const void *w, size_t rows, size_t cols,
                       const float *x, float *y, size_t tokens, hipStream_t stream);

/* Host mirror of the grouped exact GEMV launch (gemv_exact.hip GemvGroup). */
#define MYNAH_GROUP_MAX 8
typedef struct {
    const void *w, *w2;
    const float *x;
    float *y;
    const float *res;
    const uint32_t *ypos;
    const float *norm_w;     /* input = RMSNorm(x) * norm_w when set */
    unsigned long long *keys; /* one argmax key per workgroup tile when set */
    uint32_t ystride, rows, units, row_bytes, type, tile0, cols;
    float eps;
    uint32_t pad;            /* flat layout: rows per workgroup (set by the launch) */
} mynah_gemv_desc;

/* Host mirror of the streaming GEMV's descriptor (gemv_stream.hip
 * StreamDesc). */
typedef struct {
    const void *w;
    const float *x;
    float *y;
    const float *norm_w;
    unsigned long long *keys;
    uint32_t rows, units, row_bytes, type, cols;
    float eps;
} mynah_stream_desc;

/* Host mirror of gemv_exact.hip GemvPrefetch: wgs extra workgroups of a
 * grouped launch that pull the next launch's weight tiles into the L2 of
 * the XCD that will read them (mynah_gemv_prefetch_plan fills it; the
 * launch sets host_tiles). All zero: no prefetch. */
#define MYNAH_PF_SEGS 4
typedef struct {
    const void *base[MYNAH_PF_SEGS];
    uint32_t t0[MYNAH_PF_SEGS], nt[MYNAH_PF_SEGS], bpt[MYNAH_PF_SEGS], bytes[MYNAH_PF_SEGS];
    uint32_t n, wgs, host_tiles, step_log2;
} mynah_gemv_prefetch;

typedef struct {
    uint32_t n, shape;        /* shape: set by the launch */
    mynah_gemv_desc d[MYNAH_GROUP_MAX];
    mynah_gemv_prefetch pf;
} mynah_gemv_group;

/* Fill tile0 and launch. Each desc needs w, x, y, rows, type and (from
 * cols) units / row_bytes, which mynah_gemv_desc_init sets. */
int mynah_gemv_desc_init(mynah_gemv_desc *g, int type, const void *w, size_t rows, size_t cols,
                         const float *x, float *y);
/* *tiles (optional) receives the number of workgroups, which is also the
 * length of a descriptor's argmax key array when the group has one member.
 * order: MYNAH_GEMV_EXACT / MYNAH_GEMV_REORDERED, or -1 for the library's
 * current order. */
int mynah_gemv_group_launch(mynah_device *d, mynah_gemv_group *grp, hipStream_t stream,
                            uint32_t *tiles, int order);
/* The block size the launch above would use (its input RMSNorm reduces in
 * an order that depends on it). */
int mynah_gemv_group_threads(mynah_gemv_group *grp, int order, uint32_t *threads);
/* Block size and workgroup count of that launch, without launching (either
 * pointer may be NULL). The workgroup count is the length of the argmax key
 * array a one-member group with `keys` writes. */
int mynah_gemv_group_geometry(mynah_gemv_group *grp, int order, uint32_t *threads,
                              uint32_t *grid);
/* Fill *pf so that a launch carrying it prefetches the weights of `next`
 * (planned in `order`) with wgs workgroups (a multiple of 8), or with one
 * workgroup per bytes_per_wg bytes (rounded up to a multiple of 8, at most
 * 1024) when bytes_per_wg is not 0; one byte touched per 2^step_log2
 * bytes. Both 0 clears *pf. A next launch of more than max_bytes, one that
 * the streaming kernel runs, or one larger than 4 GiB per matrix, gets no
 * prefetch. */
int mynah_gemv_prefetch_plan(const mynah_gemv_group *next, int order, uint32_t wgs,
                             uint32_t bytes_per_wg, uint64_t max_bytes, uint32_t step_log2,
                             mynah_gemv_prefetch *pf);

/* Y[tokens][rows] = (res +) X[tokens][cols] · W^T in the matvec summation
 * order (every output bit-identical to the matvec of its token);
 * cols % 256 == 0; res may be NULL or alias y. */
int mynah_matmat_mv_launch(mynah_device *d, int type, const void *w, size_t rows, size_t cols,
                           const float *x, float *y, size_t tokens, const float *res,
                           hipStream_t stream);

/* mynah_hip_qwen3_new over a blob of blob_bytes assembled from n_parts
 * host parts, part i (part_bytes[i] bytes) at offset part_at[i]: the data
 * sections of a split checkpoint's shards (gguf.c). */
#include "mynah_decode.h"
mynah_qwen3 *mynah_qwen3_new_parts(const mynah_qwen3_shape *c, const mynah_synth_tensor *table,
                                   size_t count, const void *const *parts,
                                   const uint64_t *part_bytes, const uint64_t *part_at,
                                   uint32_t n_parts, uint64_t blob_bytes, uint32_t n_ctx,
                                   char *err, size_t errsz);

#endif
