/* generate_hip.c — the front-end binding of the generation loop: what a
 * maintainer adds beside the reference's src/generate.c so that its CLI and
 * server (cli/main.c:272-296, server/main.c:284-296) generate on the GPU.
 *
 * TEST INFRASTRUCTURE HERE: oracle/Makefile's `linkcheck` compiles it
 * against the reference's headers under /root/reference and links it, with
 * the reference's decoder and CLI, against libmynah_hip.so with
 * --no-undefined (tests/test_integration_link.py); the integration notes
 * show the same code. Nothing of it is part of the library or runs on the
 * GPU box.
 *
 * mynah_slm_generate_hip has mynah_slm_generate's contract
 * (src/generate.h:47-52) over the resident decoder: the loop itself is
 * mynah_hip_qwen3_generate_tokens (include/mynah_generate.h); per generated
 * id this callback does what src/generate.c:60-77 does — the think markers
 * switch the channel and reach neither callback, each channel has its own
 * detokenizer and callback — and afterwards the answer detokenizer is
 * flushed (src/generate.c:80-83) and the timing copied.
 * mynah_slm_generate_hip_dev is the same with the sampler on the device: a
 * front end makes it from its mynah_slm_sampler_params (same fields, same
 * order) with mynah_hip_sampler_new and keeps the reference's sampler for
 * the settings that returns NULL for.
 *
 * SPDX-License-Identifier: MIT */
#include "generate.h"
#include "sampler.h"
#include "timing.h"
#include "tokenizer.h"

#include "mynah_generate.h"

static uint32_t sample_cb(void *sam, float *logits) { return mynah_slm_sample(sam, logits); }
static void accept_cb(void *sam, uint32_t id) { mynah_slm_sampler_accept(sam, id); }

struct chan {
    const mynah_slm_gen_params *p;
    mynah_slm_detok d_answer, d_think;
    int in_think;
};

static int token_cb(void *c_, uint32_t id) {
    struct chan *c = c_;
    const mynah_slm_gen_params *p = c->p;
    const int split = p->think_open >= 0 && p->think_close >= 0;
    if (split && id == (uint32_t)p->think_open) { c->in_think = 1; return 0; }
    if (split && id == (uint32_t)p->think_close) { c->in_think = 0; return 0; }
    char piece[512];
    const long w = mynah_slm_detok_feed(c->in_think ? &c->d_think : &c->d_answer, id, piece,
                                        sizeof piece - 1);
    if (w < 0) return 1;
    piece[w] = '\0';
    mynah_slm_token_cb cb = c->in_think ? p->cb_think : p->cb;
    return cb ? cb(c->in_think ? p->cb_think_ctx : p->cb_ctx, id, piece, (size_t)w) : 0;
}

static long generate(mynah_qwen3 *gpu, const mynah_slm_tokenizer *tok, mynah_slm_sampler *sam,
                     mynah_hip_sampler *dev, const mynah_slm_gen_params *p, mynah_slm_timing *t) {
    struct chan c = {.p = p};
    mynah_slm_detok_init(&c.d_answer, tok);
    mynah_slm_detok_init(&c.d_think, tok);
    mynah_hip_gen_params g = {p->prompt, p->n_prompt, p->max_new, p->eos, p->n_eos,
                              token_cb, &c, sample_cb, accept_cb, sam, 0, dev};
    mynah_hip_timing ht;
    const long n = mynah_hip_qwen3_generate_tokens(gpu, &g, &ht);
    char piece[512];
    const long w = mynah_slm_detok_finish(&c.d_answer, piece, sizeof piece - 1);
    if (w > 0 && p->cb) { piece[w] = '\0'; p->cb(p->cb_ctx, 0, piece, (size_t)w); }
    mynah_slm_detok_finish(&c.d_think, piece, sizeof piece - 1);
    if (t != NULL && n >= 0) {
        t->prefill_s = ht.prefill_s;
        t->decode_s = ht.decode_s;
        t->ttft_s = ht.ttft_s;
        t->n_prompt = ht.n_prompt;
        t->n_gen = ht.n_gen;
    }
    return n;
}

long mynah_slm_generate_hip(mynah_qwen3 *gpu, const mynah_slm_tokenizer *tok,
                            mynah_slm_sampler *sam, const mynah_slm_gen_params *p,
                            mynah_slm_timing *t) {
    return generate(gpu, tok, sam, NULL, p, t);
}

long mynah_slm_generate_hip_dev(mynah_qwen3 *gpu, const mynah_slm_tokenizer *tok,
                                mynah_hip_sampler *dev, const mynah_slm_gen_params *p,
                                mynah_slm_timing *t) {
    return generate(gpu, tok, NULL, dev, p, t);
}
