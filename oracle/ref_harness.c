/* ref_harness.c — drives the compiled reference (oracle/_ref/) for golden
 * vectors and for validating the restatement.
 *
 * TEST INFRASTRUCTURE ONLY. Built by oracle/Makefile against the reference
 * sources where they lie under /root/reference (nothing is copied); the
 * result lands in oracle/_ref/, which is never committed. The only calls made
 * are the reference's own public entry points:
 *   third_party/ingot/include/ingot/quant.h:155-183 (ingot_matvec/matmat/
 *   dequant_matrix), :64-116 (per-type kernels), :30-35 (ingot_dequant, the
 *   independent decoder lineage of src/dequant.c);
 *   third_party/ingot/include/ingot/write.h:30-64 (GGUF writer);
 *   src/model.h + src/model.c:177 (mynah_slm_load), src/arch_qwen3.h:52-62
 *   (state, forward), src/sampler.h:21-43 (greedy sampling), src/threads.h.
 *
 * SPDX-License-Identifier: MIT */
#include "ingot/gguf.h"
#include "ingot/quant.h"
#include "ingot/write.h"

#include "arch_qwen3.h"
#include "generate.h"
#include "model.h"
#include "mynah_slm.h"
#include "sampler.h"
#include "threads.h"
#include "timing.h"
#include "tokenizer.h"

#include "mynah_synth.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

int ref_matvec(int type, const void *w, size_t rows, size_t cols, const float *x, float *y) {
    return ingot_matvec(type, w, rows, cols, x, y);
}

int ref_matmat(int type, const void *w, size_t rows, size_t cols, const float *x, float *y,
               size_t tokens) {
    return ingot_matmat(type, w, rows, cols, x, y, tokens);
}

int ref_q4_k_matmat_exact(const void *w, size_t rows, size_t cols, const float *x, float *y,
                          size_t tokens) {
    return ingot_q4_k_matmat_exact(w, rows, cols, x, y, tokens);
}

int ref_matmat_is_exact(size_t tokens) { return ingot_matmat_is_exact(tokens); }

int ref_dequant_matrix(int type, const void *w, size_t rows, size_t cols, float *y) {
    return ingot_dequant_matrix(type, w, rows, cols, y);
}

/* The second decoder lineage (third_party/ingot/src/dequant.c:483-535). */
int ref_dequant(int type, const void *src, size_t nelem, float *dst) {
    return ingot_dequant(type, src, nelem, dst);
}

int ref_type_geometry(int type, uint64_t *elems, uint64_t *bytes) {
    return ingot_type_geometry(type, elems, bytes);
}

int ref_has_kernel(int type) { return ingot_has_kernel(type); }

/* Write a random-init Qwen3 (tensor table + blob from mynah_synth_qwen3_*)
 * as a GGUF the reference loader accepts. */
static int write_qwen3(const char *path, const mynah_qwen3_shape *s,
                       const mynah_synth_tensor *table, size_t count, const void *blob,
                       uint32_t n_ctx, int with_vocab, char *err, size_t errsz) {
    ingot_gguf_writer *w = ingot_gguf_writer_new();
    if (w == NULL) { snprintf(err, errsz, "writer alloc"); return -1; }
    int rc = 0;
    if (with_vocab) {
        /* A vocabulary for src/tokenizer.c's loader and detokenizer: token i
         * is the text "t<i>", one merge. */
        char **tok = (char **)calloc(s->vocab, sizeof *tok);
        rc = tok ? 0 : -1;
        for (uint32_t i = 0; i < s->vocab && rc == 0; i++) {
            tok[i] = (char *)malloc(16);
            if (tok[i] == NULL) rc = -1;
            else snprintf(tok[i], 16, "t%u", i);
        }
        const char *merges[1] = {"t 0"};
        if (rc == 0)
            rc |= ingot_gguf_kv_array_string(w, "tokenizer.ggml.tokens",
                                             (const char *const *)tok, s->vocab);
        rc |= ingot_gguf_kv_array_string(w, "tokenizer.ggml.merges", merges, 1);
        for (uint32_t i = 0; tok && i < s->vocab; i++) free(tok[i]);
        free(tok);
    }
    rc |= ingot_gguf_kv_string(w, "general.architecture", "qwen3");
    rc |= ingot_gguf_kv_u32(w, "qwen3.block_count", s->n_layers);
    rc |= ingot_gguf_kv_u32(w, "qwen3.embedding_length", s->d_model);
    rc |= ingot_gguf_kv_u32(w, "qwen3.feed_forward_length", s->d_ff);
    rc |= ingot_gguf_kv_u32(w, "qwen3.attention.head_count", s->n_heads);
    rc |= ingot_gguf_kv_u32(w, "qwen3.attention.head_count_kv", s->n_kv_heads);
    rc |= ingot_gguf_kv_u32(w, "qwen3.attention.key_length", s->head_dim);
    rc |= ingot_gguf_kv_u32(w, "qwen3.attention.value_length", s->head_dim);
    rc |= ingot_gguf_kv_u32(w, "qwen3.context_length", n_ctx);
    rc |= ingot_gguf_kv_f32(w, "qwen3.attention.layer_norm_rms_epsilon", s->rms_eps);
    rc |= ingot_gguf_kv_f32(w, "qwen3.rope.freq_base", s->rope_theta);
    for (size_t i = 0; i < count && rc == 0; i++) {
        const mynah_synth_tensor *t = &table[i];
        uint64_t ne[2] = { t->cols, t->rows };
        rc |= ingot_gguf_add_tensor(w, t->name, t->type, t->rank, ne,
                                    (const unsigned char *)blob + t->offset);
    }
    if (rc != 0) {
        snprintf(err, errsz, "writer rejected a key or tensor");
        ingot_gguf_writer_free(w);
        return -1;
    }
    rc = ingot_gguf_writer_save(w, path, err, errsz);
    ingot_gguf_writer_free(w);
    return rc;
}

int ref_write_qwen3_gguf(const char *path, const mynah_qwen3_shape *s,
                         const mynah_synth_tensor *table, size_t count, const void *blob,
                         uint32_t n_ctx, char *err, size_t errsz) {
    return write_qwen3(path, s, table, count, blob, n_ctx, 0, err, errsz);
}

/* The same checkpoint with a vocabulary, for the generation loop. */
int ref_write_qwen3_gguf_vocab(const char *path, const mynah_qwen3_shape *s,
                               const mynah_synth_tensor *table, size_t count, const void *blob,
                               uint32_t n_ctx, char *err, size_t errsz) {
    return write_qwen3(path, s, table, count, blob, n_ctx, 1, err, errsz);
}

/* A token callback that records the ids it sees and asks to stop once it
 * has seen stop_after of them (0: never). */
typedef struct {
    uint32_t *ids;
    size_t cap, n, stop_after;
} ref_rec;

static int ref_rec_cb(void *ctx, uint32_t id, const char *text, size_t len) {
    (void)text;
    (void)len;
    ref_rec *r = (ref_rec *)ctx;
    if (r->n < r->cap) r->ids[r->n] = id;
    r->n++;
    return r->stop_after != 0 && r->n >= r->stop_after;
}

/* src/generate.c:13-86 itself, on the checkpoint at `path` (written with a
 * vocabulary) with a fresh state of n_ctx positions and the reference's
 * sampler (`sp`; NULL: greedy). The answer channel's callback records into
 * answer (stopping after stop_after ids when non-zero), the thinking
 * channel's into think; think_open / think_close -1 disables the split.
 * Reports the loop's return value, the timing's generated count and the
 * state's position afterwards. */
int ref_generate_record(const char *path, uint32_t n_ctx, const uint32_t *prompt,
                        size_t n_prompt, uint32_t max_new, const uint32_t *eos, size_t n_eos,
                        long think_open, long think_close, size_t stop_after,
                        const mynah_slm_sampler_params *sp, uint32_t *answer, size_t answer_cap,
                        size_t *n_answer, uint32_t *think, size_t think_cap, size_t *n_think,
                        long *produced, uint32_t *n_gen, uint32_t *n_past, char *err,
                        size_t errsz) {
    mynah_slm_threads_init(0);
    mynah_slm_model_t *m = mynah_slm_load(path, err, errsz);
    if (m == NULL) return -1;
    mynah_slm_tokenizer *tok = mynah_slm_tokenizer_load(m->gguf, err, errsz);
    if (tok == NULL) {
        mynah_slm_free(m);
        return -1;
    }
    mynah_slm_state st;
    if (mynah_slm_state_init(&st, m, n_ctx, err, errsz) != 0) {
        mynah_slm_tokenizer_free(tok);
        mynah_slm_free(m);
        return -1;
    }
    const mynah_slm_config *c = mynah_slm_model_config(m);
    mynah_slm_sampler_params greedy;
    memset(&greedy, 0, sizeof greedy);
    greedy.temp = 0.0f;
    greedy.top_p = 1.0f;
    greedy.repeat_penalty = 1.0f;
    mynah_slm_sampler *sam = mynah_slm_sampler_new(sp ? sp : &greedy, c->vocab_size);
    ref_rec ra = {answer, answer_cap, 0, stop_after}, rt = {think, think_cap, 0, 0};
    mynah_slm_gen_params gp;
    memset(&gp, 0, sizeof gp);
    gp.prompt = prompt;
    gp.n_prompt = n_prompt;
    gp.max_new = max_new;
    gp.eos = eos;
    gp.n_eos = n_eos;
    gp.cb = ref_rec_cb;
    gp.cb_ctx = &ra;
    gp.cb_think = ref_rec_cb;
    gp.cb_think_ctx = &rt;
    gp.think_open = think_open;
    gp.think_close = think_close;
    mynah_slm_timing tm;
    mynah_slm_timing_reset(&tm);
    mynah_slm_timing_start(&tm);
    int rc = 0;
    if (sam == NULL) {
        snprintf(err, errsz, "sampler alloc");
        rc = -1;
    } else {
        *produced = mynah_slm_generate(&st, tok, sam, &gp, &tm);
        *n_answer = ra.n;
        *n_think = rt.n;
        *n_gen = tm.n_gen;
        *n_past = st.n_past;
    }
    if (sam) mynah_slm_sampler_free(sam);
    mynah_slm_state_free(&st);
    mynah_slm_tokenizer_free(tok);
    mynah_slm_free(m);
    return rc;
}

/* Load `path` with the reference loader, prefill the KV cache with
 * n_prefill positions (k/v: [layer][n_prefill][kv_dim]), then run n_steps
 * greedy decode steps starting from `first_token`: token[i+1] is the greedy
 * sample of forward(token[i]). Writes the n_steps sampled ids, and when
 * `logits0` is non-NULL the logits of the first step. */
int ref_qwen3_greedy(const char *path, const float *k_prefill, const float *v_prefill,
                     uint32_t n_prefill, uint32_t first_token, uint32_t n_steps,
                     uint32_t n_ctx, int threads, uint32_t *tokens_out, float *logits0,
                     char *err, size_t errsz) {
    mynah_slm_threads_init(threads);
    mynah_slm_model_t *m = mynah_slm_load(path, err, errsz);
    if (m == NULL) return -1;
    mynah_slm_state st;
    if (mynah_slm_state_init(&st, m, n_ctx, err, errsz) != 0) {
        mynah_slm_free(m);
        return -1;
    }
    const mynah_slm_config *c = mynah_slm_model_config(m);
    if (n_prefill > 0) {
        const size_t per_layer = (size_t)st.n_ctx * c->kv_dim;
        const size_t row = (size_t)n_prefill * c->kv_dim;
        for (uint32_t l = 0; l < c->n_layers; l++) {
            memcpy(st.k_cache + l * per_layer, k_prefill + l * row, row * sizeof(float));
            memcpy(st.v_cache + l * per_layer, v_prefill + l * row, row * sizeof(float));
        }
        st.n_past = n_prefill;
    }
    mynah_slm_sampler_params p;
    memset(&p, 0, sizeof p);
    p.temp = 0.0f;
    p.top_p = 1.0f;
    p.repeat_penalty = 1.0f;
    mynah_slm_sampler *sam = mynah_slm_sampler_new(&p, c->vocab_size);
    int rc = sam ? 0 : -1;
    uint32_t tok = first_token;
    for (uint32_t i = 0; i < n_steps && rc == 0; i++) {
        if (mynah_slm_forward(&st, tok, st.logits) != 0) { rc = -1; break; }
        if (i == 0 && logits0) memcpy(logits0, st.logits, c->vocab_size * sizeof(float));
        tok = mynah_slm_sample(sam, st.logits);
        tokens_out[i] = tok;
    }
    if (rc != 0) snprintf(err, errsz, "forward failed at a step");
    mynah_slm_sampler_free(sam);
    mynah_slm_state_free(&st);
    mynah_slm_free(m);
    return rc;
}

/* src/generate.c:13-86 with greedy sampling: the prompt's tokens but the
 * last fill the cache without logits, then n_steps greedy steps start from
 * the last prompt token. logits_first receives the logits of that first step
 * (the last prompt token). */
int ref_qwen3_prompt_greedy(const char *path, const uint32_t *prompt, uint32_t n_prompt,
                            uint32_t n_steps, uint32_t n_ctx, int threads, uint32_t *tokens_out,
                            float *logits_first, char *err, size_t errsz) {
    mynah_slm_threads_init(threads);
    mynah_slm_model_t *m = mynah_slm_load(path, err, errsz);
    if (m == NULL) return -1;
    mynah_slm_state st;
    if (mynah_slm_state_init(&st, m, n_ctx, err, errsz) != 0) {
        mynah_slm_free(m);
        return -1;
    }
    const mynah_slm_config *c = mynah_slm_model_config(m);
    mynah_slm_sampler_params p;
    memset(&p, 0, sizeof p);
    p.temp = 0.0f;
    p.top_p = 1.0f;
    p.repeat_penalty = 1.0f;
    mynah_slm_sampler *sam = mynah_slm_sampler_new(&p, c->vocab_size);
    int rc = sam ? 0 : -1;
    for (uint32_t i = 0; i + 1 < n_prompt && rc == 0; i++)
        if (mynah_slm_forward(&st, prompt[i], NULL) != 0) rc = -1;
    uint32_t tok = prompt[n_prompt - 1];
    for (uint32_t i = 0; i < n_steps && rc == 0; i++) {
        if (mynah_slm_forward(&st, tok, st.logits) != 0) { rc = -1; break; }
        if (i == 0 && logits_first) memcpy(logits_first, st.logits, c->vocab_size * sizeof(float));
        tok = mynah_slm_sample(sam, st.logits);
        tokens_out[i] = tok;
    }
    if (rc != 0) snprintf(err, errsz, "forward failed");
    if (sam) mynah_slm_sampler_free(sam);
    mynah_slm_state_free(&st);
    mynah_slm_free(m);
    return rc;
}

/* One run of the reference decoder on the model at `path`, for golden
 * vectors: optional KV prefill (k/v [layer][n_prefill][kv_dim]), optional
 * prompt (all but its last token fill the cache without logits, as
 * src/generate.c:33-36 does; the last is step 0's input), then n_steps
 * steps. Step i's input is inputs[i] when `inputs` is given (teacher
 * forcing), else step 0's input is `first` (or the prompt's last token) and
 * step i + 1's the greedy sample of step i (src/sampler.c:122-129).
 * greedy_out[i] is the greedy sample of step i's logits either way;
 * logits_out (n_steps x vocab, optional) gets every step's logits. */
int ref_qwen3_run(const char *path, const float *k_prefill, const float *v_prefill,
                  uint32_t n_prefill, const uint32_t *prompt, uint32_t n_prompt, uint32_t first,
                  const uint32_t *inputs, uint32_t n_steps, uint32_t n_ctx, int threads,
                  uint32_t *greedy_out, float *logits_out, char *err, size_t errsz) {
    mynah_slm_threads_init(threads);
    mynah_slm_model_t *m = mynah_slm_load(path, err, errsz);
    if (m == NULL) return -1;
    mynah_slm_state st;
    if (mynah_slm_state_init(&st, m, n_ctx, err, errsz) != 0) {
        mynah_slm_free(m);
        return -1;
    }
    const mynah_slm_config *c = mynah_slm_model_config(m);
    if (n_prefill > 0) {
        const size_t per_layer = (size_t)st.n_ctx * c->kv_dim;
        const size_t row = (size_t)n_prefill * c->kv_dim;
        for (uint32_t l = 0; l < c->n_layers; l++) {
            memcpy(st.k_cache + l * per_layer, k_prefill + l * row, row * sizeof(float));
            memcpy(st.v_cache + l * per_layer, v_prefill + l * row, row * sizeof(float));
        }
        st.n_past = n_prefill;
    }
    mynah_slm_sampler_params p;
    memset(&p, 0, sizeof p);
    p.temp = 0.0f;
    p.top_p = 1.0f;
    p.repeat_penalty = 1.0f;
    mynah_slm_sampler *sam = mynah_slm_sampler_new(&p, c->vocab_size);
    int rc = sam ? 0 : -1;
    for (uint32_t i = 0; i + 1 < n_prompt && rc == 0; i++)
        if (mynah_slm_forward(&st, prompt[i], NULL) != 0) rc = -1;
    uint32_t tok = n_prompt > 0 ? prompt[n_prompt - 1] : first;
    for (uint32_t i = 0; i < n_steps && rc == 0; i++) {
        if (inputs) tok = inputs[i];
        if (mynah_slm_forward(&st, tok, st.logits) != 0) { rc = -1; break; }
        if (logits_out)
            memcpy(logits_out + (size_t)i * c->vocab_size, st.logits, c->vocab_size * sizeof(float));
        tok = mynah_slm_sample(sam, st.logits);
        greedy_out[i] = tok;
    }
    if (rc != 0) snprintf(err, errsz, "forward failed");
    if (sam) mynah_slm_sampler_free(sam);
    mynah_slm_state_free(&st);
    mynah_slm_free(m);
    return rc;
}
