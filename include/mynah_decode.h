/* mynah_decode.h — the resident Qwen3 decode step on one MI355X.
 *
 * The GPU twin of the reference decoder's state and step
 * (src/arch_qwen3.h:21-62): init owns the KV cache and every scratch buffer,
 * forward() advances one position, reset() drops the history. The model is
 * described by a tensor table (names, ggml types and shapes of the GGUF the
 * reference loads, src/model.c:142-228) over one byte blob that is uploaded
 * unchanged; Q4_K, Q6_K and Q8_0 projections run through the bit-exact GEMVs
 * of kernels_hip.h, the f32 operators follow src/kernels.c.
 *
 * SPDX-License-Identifier: MIT */
#ifndef MYNAH_DECODE_H
#define MYNAH_DECODE_H

#include <stddef.h>
#include <stdint.h>

#include "mynah_synth.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mynah_qwen3 mynah_qwen3;

/* src/arch_qwen3.h:52-53 (mynah_slm_state_init): bind the tensors of
 * `table` (offsets into `blob`, blob_bytes long), upload the blob, allocate
 * the state for n_ctx positions. Tied head when "output.weight" is absent.
 * NULL on failure, with the reason in err. */
mynah_qwen3 *mynah_hip_qwen3_new(const mynah_qwen3_shape *shape, const mynah_synth_tensor *table,
                                 size_t count, const void *blob, uint64_t blob_bytes,
                                 uint32_t n_ctx, char *err, size_t errsz);
/* src/arch_qwen3.h:54 */
void mynah_hip_qwen3_free(mynah_qwen3 *s);
/* src/arch_qwen3.h:56-57 (mynah_slm_state_reset) */
void mynah_hip_qwen3_reset(mynah_qwen3 *s);

/* src/arch_qwen3.h:59-62 (mynah_slm_forward): one token at position n_past;
 * logits (host, vocab floats) may be NULL. 0, or -1 with the context full. */
int mynah_hip_qwen3_forward(mynah_qwen3 *s, uint32_t token, float *logits);

/* Greedy decoding (src/generate.c:47-77 with src/sampler.c:122-129) of
 * n_steps tokens from first_token, the whole loop resident on the GPU (one
 * captured step replayed per token). tokens_out gets the n_steps sampled
 * ids; *ms (optional) the GPU time of the loop. */
int mynah_hip_qwen3_generate(mynah_qwen3 *s, uint32_t first_token, uint32_t n_steps,
                             uint32_t *tokens_out, float *ms);

/* Teacher forcing (no reference counterpart: the reference's loop always
 * feeds back its own choice, src/generate.c:47-77): n steps whose inputs are
 * inputs[0 .. n) at positions n_past .. n_past + n - 1, replayed through the
 * same captured step graphs as generate(). greedy_out[i] receives the greedy
 * choice of step i's logits (src/sampler.c:122-129); last_logits (optional,
 * host, vocab floats) the logits of the last step. n_past advances by n. */
int mynah_hip_qwen3_forced(mynah_qwen3 *s, const uint32_t *inputs, uint32_t n,
                           uint32_t *greedy_out, float *last_logits);

/* Fill positions [0, n_pos) of the KV cache from host arrays laid out
 * [layer][n_pos][kv_dim] and set n_past = n_pos (the configs prefill the
 * cache with synthetic values instead of running a prompt). */
int mynah_hip_qwen3_set_kv(mynah_qwen3 *s, const float *k, const float *v, uint32_t n_pos);

/* The mirror of set_kv: positions [0, n_pos) of the cache into host arrays
 * [layer][n_pos][kv_dim] (the keys as the attention uses them: normalised
 * and rotated). */
int mynah_hip_qwen3_get_kv(const mynah_qwen3 *s, float *k, float *v, uint32_t n_pos);

uint32_t mynah_hip_qwen3_n_past(const mynah_qwen3 *s);
/* Test hook, no reference counterpart: the attention output of the last
 * layer of the most recent step (n_heads * head_dim floats, the `out` of
 * src/kernels.c:228-250 for that layer), into host memory. */
int mynah_hip_qwen3_read_attn(const mynah_qwen3 *s, float *out);
/* src/generate.c:13-86 with greedy sampling: the prompt's tokens fill the
 * cache (all but the last without logits, the head is skipped), then
 * n_steps greedy steps start from the last prompt token; tokens_out gets the
 * n_steps generated ids. *prefill_ms covers the n_prompt - 1 cache-filling
 * steps, *decode_ms the greedy steps (either may be NULL). The position
 * advances by n_prompt - 1 + n_steps. */
int mynah_hip_qwen3_prompt(mynah_qwen3 *s, const uint32_t *prompt, uint32_t n_prompt,
                           uint32_t n_steps, uint32_t *tokens_out, float *prefill_ms,
                           float *decode_ms);

/* Fill positions n_past .. n_past + n - 1 of the cache with n tokens and
 * advance n_past by n, without logits — the same bits n calls of
 * mynah_hip_qwen3_forward(s, token, NULL) leave in the exact GEMV order and
 * the exact attention (no reference counterpart: the reference prefills
 * token by token, src/arch_qwen3.c:3-7). Tokens run in chunks of up to 2048
 * (MYNAH_PREFILL_CHUNK) through matvec-order GEMMs, per-row RMSNorm and
 * SwiGLU, and per-query attention; the chunk buffers are allocated on first
 * use; Q4_0 projections take the Q4_0 chains, whose batched order is the
 * matvec's. 0, or -1 when the tokens do not fit the context. */
int mynah_hip_qwen3_prefill(mynah_qwen3 *s, const uint32_t *tokens, uint32_t n);

/* How mynah_hip_qwen3_prompt fills the cache with the prompt:
 *   MYNAH_PREFILL_BATCHED (default): mynah_hip_qwen3_prefill;
 *   MYNAH_PREFILL_STEPS: one decode step per token, in the current GEMV
 *     order and attention mode (the reference's loop). */
enum { MYNAH_PREFILL_BATCHED = 0, MYNAH_PREFILL_STEPS = 1 };
int mynah_hip_qwen3_set_prefill(mynah_qwen3 *s, int mode);

/* 1 when the step runs as a replayed hipGraph, 0 when launched directly. */
int mynah_hip_qwen3_uses_graph(const mynah_qwen3 *s);

/* Attention of the decode step (no reference counterpart; the reference's
 * attention is src/kernels.c:228-293):
 *   MYNAH_ATTN_EXACT (default): the reference's operations in its order — the
 *     full softmax over all positions, then o = fma(v_t, p_t, o) for t in
 *     order; two launches per layer;
 *   MYNAH_ATTN_SPLIT: positions split across workgroups (32-position chunks
 *     up to n_ctx 32,768, 64 up to 65,536, 128 beyond; MYNAH_AS_CH forces
 *     one when the decoder is made), per-chunk softmax partials combined by
 *     a second small launch; short FMA chains; differs from the reference by
 *     f32 rounding only; refused (-1) past 16,384 chunks (the combine's
 *     per-chunk weights fill 64 KiB of LDS there). */
enum { MYNAH_ATTN_EXACT = 0, MYNAH_ATTN_SPLIT = 1 };
int mynah_hip_qwen3_set_attention(mynah_qwen3 *s, int mode);

#ifdef __cplusplus
}
#endif
#endif
