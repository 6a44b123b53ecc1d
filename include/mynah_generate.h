/* mynah_generate.h — the generation loop over the resident decoder: the GPU
 * twin of the reference's mynah_slm_generate (src/generate.c:13-86), which
 * the CLI `run` command (cli/main.c:225-315) and the server's completion
 * handler (server/main.c:175-300) both drive.
 *
 * The loop is the reference's, step for step:
 *   - every prompt token but the last only fills the cache (the batched
 *     prefill, which leaves the same cache bits as one step per token), and
 *     each is shown to the sampler's accept hook;
 *   - then up to max_new steps: forward the current token, pick the next id,
 *     accept it, stop on any of the EOS ids (the EOS id counts as generated
 *     but is not passed to on_token), else pass it to on_token (non-zero
 *     stops), and feed it back;
 *   - a full context ends the loop (the ids so far stand).
 * The return value is the number of ids generated, or -1.
 *
 * Picking the next id:
 *   - sample == NULL: greedy on the device (src/sampler.c:122-129, first
 *     index of the largest logit), with the logits never leaving HBM; steps
 *     run as captured graphs, up to `chunk` per host round trip (0: 8), the
 *     first step alone so TTFT is one step. This is the reference's sampler
 *     at temp <= 0 with every penalty off; with penalties on, pass a
 *     device sampler or the reference's sampler as below.
 *   - sample != NULL: every step's logits are copied to a host buffer and
 *     sample(sampler, logits) picks (the reference's mynah_slm_sample, which
 *     may modify the logits in place, fits as is); accept(sampler, id), when
 *     set, is called where the reference calls mynah_slm_sampler_accept.
 *   - device_sampler != NULL (sample, accept and sampler are then unused):
 *     the reference's sampler on the device (below), inside the captured
 *     steps like greedy, so the logits never leave HBM; the prompt tokens
 *     and every generated id enter its window, and its rng advances once
 *     per sampled id, exactly as the reference's sampler object would.
 *
 * Detokenisation and the thinking channel (src/generate.c:38-77) stay with
 * the caller: on_token receives the id, and the reference's binding feeds
 * its own detokenizer and routes the think markers inside that callback.
 *
 * Timing follows src/timing.c:30-62 (CLOCK_MONOTONIC, host side): prefill_s
 * from the call to the end of the prompt, decode_s from there to the end,
 * ttft_s stamped at the first generated id (prefill plus that step).
 *
 * SPDX-License-Identifier: MIT */
#ifndef MYNAH_GENERATE_H
#define MYNAH_GENERATE_H

#include <stddef.h>
#include <stdint.h>

#include "mynah_decode.h"

#ifdef __cplusplus
extern "C" {
#endif

/* src/generate.h:13-15 (mynah_slm_token_cb), without the text: non-zero
 * stops generation after this id. */
typedef int (*mynah_hip_token_fn)(void *ctx, uint32_t id);
/* src/sampler.h:40-43 (mynah_slm_sample, mynah_slm_sampler_accept). */
typedef uint32_t (*mynah_hip_sample_fn)(void *sampler, float *logits);
typedef void (*mynah_hip_accept_fn)(void *sampler, uint32_t id);

/* src/generate.h:18-45 (mynah_slm_gen_params) */
typedef struct {
    const uint32_t *prompt;
    size_t n_prompt;
    uint32_t max_new;
    const uint32_t *eos;            /* stop on any of these */
    size_t n_eos;
    mynah_hip_token_fn on_token;
    void *token_ctx;
    mynah_hip_sample_fn sample;     /* NULL: greedy on the device */
    mynah_hip_accept_fn accept;     /* optional */
    void *sampler;
    uint32_t chunk;                 /* device steps per round trip, 0 = 8 */
    struct mynah_hip_sampler *device_sampler; /* NULL: as above */
} mynah_hip_gen_params;

/* src/timing.h:14-28 (mynah_slm_timing), the fields the loop fills. */
typedef struct {
    double prefill_s, decode_s, ttft_s;
    uint32_t n_prompt, n_gen;
    int ttft_done;
} mynah_hip_timing;

/* ── the reference's sampler on the device ─────────────────────────────────
 * src/sampler.h:16-30 (mynah_slm_sampler_params), field for field. */
typedef struct {
    float temp;                     /* <= 0: greedy */
    uint32_t top_k;                 /* 0 = off (host sampler only when temp > 0) */
    float top_p, min_p;
    float repeat_penalty, freq_penalty, presence_penalty;
    uint32_t penalty_window;
    uint64_t seed;
} mynah_hip_sampler_params;

/* A sampler object like the reference's (src/sampler.c:16-25): parameters,
 * splitmix64 state and penalty window, kept in device memory. Every id it
 * returns is the one mynah_slm_sample returns for the same logits and
 * history (the same penalties, f32 exponentials, double sum, f32
 * probabilities, candidate order, draw and walk). It takes what the
 * reference's defaults use: with temp > 0, 1 <= top_k <= 128 (and below the
 * vocabulary; the reference's top_k = 0 sorts the whole vocabulary, which
 * this sampler does not), a penalty window of at most 4096; otherwise
 * mynah_hip_sampler_new returns NULL (mynah_hip_last_error says why) and
 * the caller keeps the reference's sampler on the host. */
typedef struct mynah_hip_sampler mynah_hip_sampler;

/* src/sampler.c:48-64 (mynah_slm_sampler_new); seed 0 takes the same
 * fixed default state. */
mynah_hip_sampler *mynah_hip_sampler_new(const mynah_hip_sampler_params *p, uint32_t vocab);
/* src/sampler.c:66-71 (mynah_slm_sampler_free). */
void mynah_hip_sampler_free(mynah_hip_sampler *s);
/* src/sampler.c:73-78 (mynah_slm_sampler_accept). 0, or -1. */
int mynah_hip_sampler_accept(mynah_hip_sampler *s, uint32_t token);
/* src/sampler.c:116-187 (mynah_slm_sample) over host logits, modified in
 * place like the reference's (the penalties): *id is the picked token. The
 * generation loop samples on the device without this host copy. 0, or -1. */
int mynah_hip_sample(mynah_hip_sampler *s, float *logits, uint32_t *id);

/* src/generate.h:47-52 (mynah_slm_generate). t may be NULL. */
long mynah_hip_qwen3_generate_tokens(mynah_qwen3 *s, const mynah_hip_gen_params *p,
                                     mynah_hip_timing *t);

#ifdef __cplusplus
}
#endif
#endif
