/* mynah_synth.h — the seeded synthetic-input generator shared by the GPU
 * library, the CPU oracle and the reference harness.
 *
 * No counterpart in the reference: the reference benchmarks real checkpoints.
 * The benchmark configurations describe random GGUF block bytes instead, and
 * every consumer (GPU kernels, CPU oracle, compiled reference) must see the
 * same bytes, so the generator is one C file compiled into each of them.
 *
 * Stream: splitmix64. A tensor with seed `ts` draws row r from its own stream
 * whose state starts at mynah_synth_substream(ts, r), so rows can be generated
 * in parallel and any row can be regenerated alone.
 *   - a uniform byte: the next byte of the current 64-bit output, low byte
 *     first (8 bytes per output);
 *   - N(0,1): Box-Muller in double from two fresh 53-bit uniforms, cosine leg;
 *   - int8 uniform in [lo, hi]: rejection on uniform bytes;
 *   - f16 fields: |N| * scale rounded to f16 (round to nearest even).
 *
 * Block fields are drawn in their byte order:
 *   Q4_K (144 B): d, dmin = f16(|N|*0.01); 12 scale bytes; 128 quant bytes.
 *   Q6_K (210 B): 128 ql bytes; 64 qh bytes; 16 scales int8 in [-64, 63];
 *                 d = f16(|N|*0.005) at byte 208.
 *   Q8_0 (34 B):  d = f16(|N|*0.01); 32 int8 in [-127, 127].
 *   Q5_K (176 B): d, dmin = f16(|N|*0.01); 12 scale bytes, 32 qh bytes and
 *                 128 quant bytes, all uniform.
 *   Q4_0 (18 B):  d = f16(|N|*0.01); 16 quant bytes uniform.
 *
 * SPDX-License-Identifier: MIT */
#ifndef MYNAH_SYNTH_H
#define MYNAH_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The k-th output of the splitmix64 stream seeded with `seed`: the state a
 * sub-stream (a row, a tensor) starts from. */
uint64_t mynah_synth_substream(uint64_t seed, uint64_t k);

/* f32 -> f16 bits, round to nearest even, subnormals and overflow handled. */
uint16_t mynah_synth_f32_to_f16(float value);

/* Fill `rows` rows of `cols` weights in block format `type` (12 = Q4_K,
 * 13 = Q5_K, 14 = Q6_K, 8 = Q8_0, 2 = Q4_0) into `out`, rows
 * [row0, row0 + rows) of a tensor whose seed is `seed`. Returns 0, or -1 for
 * an unsupported type or a partial block.
 * Uses up to `threads` threads (<= 0: all online cores). */
int mynah_synth_blocks(int type, uint64_t seed, size_t row0, size_t rows,
                       size_t cols, void *out, int threads);

/* n values of mean + std * N(0,1) as f32; value i comes from row i / 4096 of
 * the tensor stream, so long vectors generate in parallel too. */
int mynah_synth_normal(uint64_t seed, size_t n, float mean, float std,
                       float *out, int threads);

/* n uniform integers in [0, bound) (token ids). */
int mynah_synth_uniform_u32(uint64_t seed, size_t n, uint32_t bound,
                            uint32_t *out);

/* ── random-init Qwen3 in the Q4_K_M type mix ─────────────────────────────
 * Tensor names and shapes follow the GGUF the reference loads
 * (src/model.c:142-228): token_embd (tied head), per layer attn_norm,
 * attn_q/k/v, attn_q_norm, attn_k_norm, attn_output, ffn_norm, ffn_gate/up/
 * down, then output_norm. Types: Q6_K for token_embd, and for attn_v and
 * ffn_down on the layers llama.cpp's Q4_K_M recipe bumps
 * (i < n/8, i >= 7n/8, or (i - n/8) % 3 == 2); Q4_K for every other matrix;
 * F32 norm weights 1 + 0.02 N(0,1). Tensor i draws from
 * mynah_synth_substream(seed, i). */
typedef struct {
    uint32_t n_layers, d_model, d_ff, n_heads, n_kv_heads, head_dim, vocab;
    float rms_eps, rope_theta;
} mynah_qwen3_shape;

typedef struct {
    char name[48];
    int type;                /* 0 = F32, 8 = Q8_0, 12 = Q4_K, 14 = Q6_K */
    uint32_t rank;           /* 1 for norm vectors, 2 for matrices */
    uint64_t rows, cols;     /* rows = ne[1] (outputs), cols = ne[0] (inputs) */
    uint64_t offset, nbytes; /* within the blob; offsets 256-byte aligned */
} mynah_synth_tensor;

/* Writes up to `cap` descriptors; *count gets the number needed and *total
 * the blob size. Returns 0, or -1 on a bad shape. */
int mynah_synth_qwen3_layout(const mynah_qwen3_shape *shape, mynah_synth_tensor *table,
                             size_t cap, size_t *count, uint64_t *total);
/* Fills the blob laid out by mynah_synth_qwen3_layout. */
int mynah_synth_qwen3_fill(const mynah_qwen3_shape *shape, uint64_t seed,
                           const mynah_synth_tensor *table, size_t count,
                           void *blob, int threads);
/* 1 when layer `i` of `n` takes Q6_K for attn_v / ffn_down in Q4_K_M. */
int mynah_synth_q4_k_m_bumped(uint32_t i, uint32_t n);

#ifdef __cplusplus
}
#endif
#endif
