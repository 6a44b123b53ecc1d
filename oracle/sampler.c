/* sampler.c — TEST INFRASTRUCTURE ONLY: a C11 restatement of the reference's
 * token sampler (src/sampler.c), used by the tests as the host-side sampler
 * of the generation loop's host-sampling mode. Pinned against the compiled
 * reference's sampler on the same logits (tests/test_sampler_oracle.py).
 *
 * Order of operations (src/sampler.c:116-187): penalties over the recent
 * window (divide a positive logit by repeat_penalty, multiply a negative
 * one; subtract freq_penalty * count and presence_penalty, :63-94); greedy
 * = first index of the largest value (:122-129); else softmax at
 * temperature (f32 exponentials of (l - max) / temp, double sum, f32
 * reciprocal, :131-143), a full sort by probability then id (:97-103),
 * top-k, min-p relative to the best, top-p keeping the crossing candidate,
 * and one splitmix64 draw over the kept mass (:40-46, :173-186).
 *
 * SPDX-License-Identifier: MIT */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    float p;
    uint32_t id;
} orc_cand;

struct orc_sampler {
    orc_sampler_params par;
    uint32_t vocab;
    orc_cand *work;
    uint32_t *window;
    uint32_t n_window, head;
    uint64_t state;
};

static double draw(uint64_t *state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (double)(z >> 11) * (1.0 / 9007199254740992.0);
}

orc_sampler *orc_sampler_new(const orc_sampler_params *p, uint32_t vocab) {
    orc_sampler *s = (orc_sampler *)calloc(1, sizeof *s);
    if (s == NULL) return NULL;
    s->par = *p;
    s->vocab = vocab;
    s->state = p->seed ? p->seed : 0x853C49E6748FEA9Bull;
    s->work = (orc_cand *)malloc((size_t)vocab * sizeof *s->work);
    s->window = p->penalty_window ? (uint32_t *)calloc(p->penalty_window, 4) : NULL;
    if (s->work == NULL || (p->penalty_window && s->window == NULL)) {
        orc_sampler_free(s);
        return NULL;
    }
    return s;
}

void orc_sampler_free(orc_sampler *s) {
    if (s == NULL) return;
    free(s->work);
    free(s->window);
    free(s);
}

void orc_sampler_accept(orc_sampler *s, uint32_t token) {
    if (s->window == NULL || s->par.penalty_window == 0) return;
    s->window[s->head] = token;
    s->head = (s->head + 1) % s->par.penalty_window;
    if (s->n_window < s->par.penalty_window) s->n_window++;
}

static void penalise(orc_sampler *s, float *logits) {
    const orc_sampler_params *p = &s->par;
    if (s->window == NULL || s->n_window == 0) return;
    if (p->repeat_penalty == 1.0f && p->freq_penalty == 0.0f && p->presence_penalty == 0.0f)
        return;
    for (uint32_t i = 0; i < s->n_window; i++) {
        const uint32_t tok = s->window[i];
        if (tok >= s->vocab) continue;
        uint32_t count = 0;
        for (uint32_t k = 0; k < s->n_window; k++) count += s->window[k] == tok;
        float l = logits[tok];
        if (p->repeat_penalty != 1.0f) l = l > 0.0f ? l / p->repeat_penalty : l * p->repeat_penalty;
        l -= p->freq_penalty * (float)count;
        l -= p->presence_penalty;
        logits[tok] = l;
    }
}

static int by_prob(const void *a, const void *b) {
    const orc_cand *x = (const orc_cand *)a, *y = (const orc_cand *)b;
    if (x->p != y->p) return x->p > y->p ? -1 : 1;
    return x->id < y->id ? -1 : (x->id > y->id);
}

uint32_t orc_sampler_sample(orc_sampler *s, float *logits) {
    const orc_sampler_params *p = &s->par;
    const uint32_t n_all = s->vocab;
    penalise(s, logits);
    if (p->temp <= 0.0f) {
        uint32_t best = 0;
        for (uint32_t i = 1; i < n_all; i++)
            if (logits[i] > logits[best]) best = i;
        return best;
    }
    float mx = logits[0];
    for (uint32_t i = 1; i < n_all; i++) mx = logits[i] > mx ? logits[i] : mx;
    double total = 0.0;
    for (uint32_t i = 0; i < n_all; i++) {
        const float e = expf((logits[i] - mx) / p->temp);
        s->work[i].p = e;
        s->work[i].id = i;
        total += (double)e;
    }
    const float inv = (float)(1.0 / total);
    for (uint32_t i = 0; i < n_all; i++) s->work[i].p *= inv;
    qsort(s->work, n_all, sizeof *s->work, by_prob);
    uint32_t n = n_all;
    if (p->top_k > 0 && p->top_k < n) n = p->top_k;
    if (p->min_p > 0.0f && n > 0) {
        const float floor_p = p->min_p * s->work[0].p;
        uint32_t keep = 1;
        while (keep < n && s->work[keep].p >= floor_p) keep++;
        n = keep;
    }
    if (p->top_p < 1.0f && n > 0) {
        double mass = 0.0;
        uint32_t keep = 0;
        while (keep < n) {
            mass += (double)s->work[keep].p;
            keep++;
            if (mass >= (double)p->top_p) break;
        }
        n = keep;
    }
    if (n == 0) n = 1;
    double kept = 0.0;
    for (uint32_t i = 0; i < n; i++) kept += (double)s->work[i].p;
    double r = draw(&s->state) * kept;
    for (uint32_t i = 0; i < n; i++) {
        r -= (double)s->work[i].p;
        if (r <= 0.0) return s->work[i].id;
    }
    return s->work[n - 1].id;
}
