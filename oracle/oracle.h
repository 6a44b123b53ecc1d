/* oracle.h — CPU restatement of the reference's quantized hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: tests/, the smoke
 * check and bench.py's cpu_baseline leg call it. The product path (the HIP
 * library under mynah-slm_amd/) never links, loads or calls it.
 *
 * It restates, in C11 of this repository's own writing, the arithmetic of the
 * as-built x86-64 reference: ingot compiled with its own `CFLAGS ?= -O2` and no
 * -march, which selects the scalar lanes of third_party/ingot/src/kernels.c,
 * and mynah-slm's decoder compiled with `-O3 -march=native` (AVX2 + FMA lanes
 * of src/kernels.c). Every function cites the reference lines it follows.
 * Operation order is kept so the results are bit-identical; the committed
 * golden vectors (tests/golden/) made from the compiled reference prove it.
 *
 * SPDX-License-Identifier: MIT */
#ifndef MYNAH_ORACLE_H
#define MYNAH_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (third_party/ingot/include/ingot/dtype.h:24-59). */
enum { ORC_Q4_0 = 2, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14 };

/* ── formats (third_party/ingot/src/kernels.c:57-136, 2176-2199, 2518-2523) ─ */
float orc_f16_to_f32(uint16_t h);
void  orc_scale_min(const unsigned char *scales, int j,
                    unsigned char *sc, unsigned char *m);
int   orc_type_geometry(int type, uint64_t *block_elems, uint64_t *block_bytes);

/* ── kernels, same contract as ingot's quant.h:64-183 ───────────────────── */
int orc_dequant_matrix(int type, const void *w, size_t rows, size_t cols, float *y);
int orc_matvec(int type, const void *w, size_t rows, size_t cols,
               const float *x, float *y);
int orc_matmat(int type, const void *w, size_t rows, size_t cols,
               const float *x, float *y, size_t tokens);
int orc_has_kernel(int type);

/* ── threading of the CPU baseline (src/threads.c, src/arch_qwen3.c:52-83) ─ */
int  orc_threads_init(int n);          /* <= 0: all online cores; returns count */
void orc_threads_shutdown(void);
int  orc_threads_count(void);
/* project(): 4*nth contiguous row chunks, serial below 64 rows. */
int  orc_project(int type, const void *w, size_t rows, size_t cols,
                 const float *x, float *y);
/* The AVX2 + FMA lanes of an ingot build with -mavx2 -mfma (Q4_K, Q6_K,
 * Q8_0; the secondary CPU baseline), alone and as project(). */
int  orc_matvec_avx2(int type, const void *w, size_t rows, size_t cols,
                     const float *x, float *y);
int  orc_project_avx2(int type, const void *w, size_t rows, size_t cols,
                      const float *x, float *y);
/* The batched exact matmat with the pool injected over 8-row strips
 * (ingot_set_parallel_for, third_party/ingot/src/cpu.c:217-230). */
int  orc_matmat_mt(int type, const void *w, size_t rows, size_t cols,
                   const float *x, float *y, size_t tokens);

/* ── int8 activation lane of Q4_K (int8.c; kernels.c:636-788, 1120-1751) ── */
/* One 256-value block: int8 quants, the eight 32-value integer sums, returns
 * the activation scale amax / 127 (0 and zeros for an all-zero block). */
float   orc_q8_quantize_block(const float *x, int8_t *q, int32_t sums[8]);
/* Integer dot of sub-block j (0..7) of one Q4_K block with the quants. */
int32_t orc_q4k_int8_dot(const unsigned char *blk, const int8_t *xq, int j);
int32_t orc_q5k_int8_dot(const unsigned char *blk, const int8_t *xq, int j);
int     orc_q4k_matvec_int8(const void *w, size_t rows, size_t cols, const float *x, float *y);
int     orc_q4k_matmat_int8(const void *w, size_t rows, size_t cols, const float *x, float *y,
                            size_t tokens);
int     orc_q5k_matmat_int8(const void *w, size_t rows, size_t cols, const float *x, float *y,
                            size_t tokens);

/* ── Qwen3 decoder restatement (src/arch_qwen3.c:178-252) ───────────────── */
typedef struct {
    uint32_t n_layers, d_model, d_ff, n_heads, n_kv_heads, head_dim, vocab;
    float rms_eps, rope_theta;
} orc_qwen3_config;

/* One tensor of a model: type id (0 = F32), rows, cols, bytes. */
typedef struct {
    int type;
    uint64_t rows, cols;
    const void *data;
} orc_tensor;

typedef struct {
    orc_tensor attn_norm, wq, wk, wv, q_norm, k_norm, wo, ffn_norm, gate, up, down;
} orc_layer;

typedef struct orc_qwen3 orc_qwen3;

orc_qwen3 *orc_qwen3_new(const orc_qwen3_config *c, const orc_tensor *embed,
                         const orc_tensor *out_norm, const orc_layer *layers,
                         uint32_t n_ctx);
void  orc_qwen3_free(orc_qwen3 *s);
/* Raw KV cache access, [layer][n_ctx][kv_dim] f32 (arch_qwen3.h:27-29). */
float *orc_qwen3_k_cache(orc_qwen3 *s);
float *orc_qwen3_v_cache(orc_qwen3 *s);
void  orc_qwen3_set_n_past(orc_qwen3 *s, uint32_t n_past);
uint32_t orc_qwen3_n_past(const orc_qwen3 *s);
const float *orc_qwen3_last_q(const orc_qwen3 *s);
const float *orc_qwen3_last_attn(const orc_qwen3 *s);
/* mynah_slm_forward: 0, or -1 when the context is full. */
int   orc_qwen3_forward(orc_qwen3 *s, uint32_t token, float *logits);

/* The token sampler (src/sampler.h:16-43, src/sampler.c). */
typedef struct {
    float temp;
    uint32_t top_k;
    float top_p, min_p;
    float repeat_penalty, freq_penalty, presence_penalty;
    uint32_t penalty_window;
    uint64_t seed;
} orc_sampler_params;
typedef struct orc_sampler orc_sampler;
orc_sampler *orc_sampler_new(const orc_sampler_params *p, uint32_t vocab);
void     orc_sampler_free(orc_sampler *s);
void     orc_sampler_accept(orc_sampler *s, uint32_t token);
uint32_t orc_sampler_sample(orc_sampler *s, float *logits);
/* Greedy choice of src/sampler.c:122-129: first index of the maximum. */
uint32_t orc_argmax(const float *logits, size_t n);

#ifdef __cplusplus
}
#endif
#endif
