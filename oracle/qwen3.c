/* qwen3.c — restatement of the reference Qwen3 decode step.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Follows src/arch_qwen3.c:178-252 (mynah_slm_forward) and the f32 operators
 * of src/kernels.c, in the lanes an x86-64 `-O3 -march=native` build takes:
 * the AVX2+FMA dot_f32 / axpy_f32 (src/kernels.c:39-100, restated here with
 * fmaf in the same lane order) and plain f32 elsewhere (no contraction under
 * -std=c11). Projections go through orc_project (src/arch_qwen3.c:52-83).
 *
 * SPDX-License-Identifier: MIT */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

void orc_pool_run(int n, void (*fn)(void *, int), void *ctx);

struct orc_qwen3 {
    orc_qwen3_config c;
    orc_tensor embed, out_norm;
    orc_layer *layers;
    uint32_t n_ctx, n_past;
    uint32_t q_dim, kv_dim;
    float *rope_cos, *rope_sin;      /* [n_ctx][head_dim/2] */
    float *k_cache, *v_cache;        /* [layer][n_ctx][kv_dim] */
    float *x, *h, *q, *attn, *proj, *gate, *up, *scores, *logits;
};

/* src/kernels.c:39-72, AVX2 branch: two 8-lane FMA accumulators over steps of
 * 16, lanes added s0+s1, then high and low 128-bit halves added, then two
 * horizontal pair-adds; a scalar tail for n % 16 (none at head_dim 128). */
static float dot_lanes(const float *a, const float *b, uint32_t n) {
    float s0[8] = {0}, s1[8] = {0};
    uint32_t i = 0;
    for (; i + 16 <= n; i += 16)
        for (int l = 0; l < 8; l++) {
            s0[l] = fmaf(a[i + l], b[i + l], s0[l]);
            s1[l] = fmaf(a[i + 8 + l], b[i + 8 + l], s1[l]);
        }
    float t[8], v[4];
    for (int l = 0; l < 8; l++) t[l] = s0[l] + s1[l];
    for (int l = 0; l < 4; l++) v[l] = t[l] + t[l + 4];
    /* hadd(v, v) = [v0+v1, v2+v3, ...]; hadd again: (v0+v1) + (v2+v3) */
    float sum = (v[0] + v[1]) + (v[2] + v[3]);
    for (; i < n; i++) sum = sum + a[i] * b[i];
    return sum;
}

/* src/kernels.c:82-91, AVX2 branch: y = fma(x, w, y) per element, 8 wide;
 * the scalar tail (none at head_dim 128) is an unfused multiply-add. */
static void axpy_lanes(float *y, const float *x, float w, uint32_t n) {
    uint32_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) y[i + l] = fmaf(x[i + l], w, y[i + l]);
    for (; i < n; i++) y[i] = y[i] + w * x[i];
}

/* src/kernels.c:118-122: the mean square accumulated in double. */
static float rms_factor(const float *x, uint32_t n, float eps) {
    double acc = 0.0;
    for (uint32_t i = 0; i < n; i++) acc += (double)x[i] * (double)x[i];
    return (float)(1.0 / sqrt(acc / (double)n + (double)eps));
}

/* src/kernels.c:124-128: out = (x * s) * w. */
static void rms_norm(float *out, const float *x, const float *w, uint32_t n, float eps) {
    const float s = rms_factor(x, n, eps);
    for (uint32_t i = 0; i < n; i++) out[i] = x[i] * s * w[i];
}

/* src/kernels.c:130-137: in place, x = x * (s * w), per head. */
static void rms_norm_heads(float *x, const float *w, uint32_t heads, uint32_t hd, float eps) {
    for (uint32_t h = 0; h < heads; h++) {
        float *xh = x + (size_t)h * hd;
        const float s = rms_factor(xh, hd, eps);
        for (uint32_t i = 0; i < hd; i++) xh[i] = xh[i] * (s * w[i]);
    }
}

/* src/kernels.c:141-164: angles in double, rounded to f32 once. */
static void rope_tables(float *cs, float *sn, uint32_t hd, uint32_t n_pos, float theta) {
    const uint32_t half = hd / 2;
    for (uint32_t i = 0; i < half; i++) {
        const double inv = 1.0 / pow((double)theta, (2.0 * (double)i) / (double)hd);
        for (uint32_t p = 0; p < n_pos; p++) {
            const double a = (double)p * inv;
            cs[(size_t)p * half + i] = (float)cos(a);
            sn[(size_t)p * half + i] = (float)sin(a);
        }
    }
}

/* src/kernels.c:173-189: split-half rotation, element i pairs with i+half. */
static void rope(const orc_qwen3 *s, float *x, uint32_t heads, uint32_t pos) {
    const uint32_t hd = s->c.head_dim, half = hd / 2;
    const float *cs = s->rope_cos + (size_t)pos * half, *sn = s->rope_sin + (size_t)pos * half;
    for (uint32_t h = 0; h < heads; h++) {
        float *xh = x + (size_t)h * hd;
        for (uint32_t i = 0; i < half; i++) {
            const float a = xh[i], b = xh[i + half];
            xh[i] = a * cs[i] - b * sn[i];
            xh[i + half] = b * cs[i] + a * sn[i];
        }
    }
}

/* src/kernels.c:193-205. */
static float sigmoid_stable(float v) {
    if (v >= 0.0f) return 1.0f / (1.0f + expf(-v));
    const float e = expf(v);
    return e / (1.0f + e);
}

/* src/kernels.c:207-220: f32 max, expf of the shifted value, double sum,
 * multiply by the f32 reciprocal. */
static void softmax(float *x, uint32_t n) {
    float m = x[0];
    for (uint32_t i = 1; i < n; i++) if (x[i] > m) m = x[i];
    double sum = 0.0;
    for (uint32_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - m);
        sum += (double)x[i];
    }
    const float inv = (float)(1.0 / sum);
    for (uint32_t i = 0; i < n; i++) x[i] = x[i] * inv;
}

typedef struct {
    orc_qwen3 *s;
    const float *k, *v;
    uint32_t n_kv;
} attn_job;

/* src/kernels.c:253-293 (attention_head under attention_mt). */
static void attn_head(void *ctx, int hh) {
    attn_job *j = (attn_job *)ctx;
    orc_qwen3 *s = j->s;
    const uint32_t hd = s->c.head_dim, h = (uint32_t)hh;
    const uint32_t kvh = h / (s->c.n_heads / s->c.n_kv_heads);
    const float scale = 1.0f / sqrtf((float)hd);
    float *sc = s->scores + (size_t)h * s->n_ctx;
    const float *qh = s->q + (size_t)h * hd;
    for (uint32_t t = 0; t < j->n_kv; t++)
        sc[t] = dot_lanes(qh, j->k + (size_t)t * s->kv_dim + (size_t)kvh * hd, hd) * scale;
    softmax(sc, j->n_kv);
    float *oh = s->attn + (size_t)h * hd;
    memset(oh, 0, hd * sizeof *oh);
    for (uint32_t t = 0; t < j->n_kv; t++)
        axpy_lanes(oh, j->v + (size_t)t * s->kv_dim + (size_t)kvh * hd, sc[t], hd);
}

static int proj(const orc_tensor *w, const float *in, float *out) {
    return orc_project(w->type, w->data, (size_t)w->rows, (size_t)w->cols, in, out);
}

orc_qwen3 *orc_qwen3_new(const orc_qwen3_config *c, const orc_tensor *embed,
                         const orc_tensor *out_norm, const orc_layer *layers,
                         uint32_t n_ctx) {
    if (c == NULL || embed == NULL || out_norm == NULL || layers == NULL || n_ctx == 0 ||
        c->head_dim % 2 != 0 || c->n_kv_heads == 0 || c->n_heads % c->n_kv_heads != 0)
        return NULL;
    orc_qwen3 *s = (orc_qwen3 *)calloc(1, sizeof *s);
    if (s == NULL) return NULL;
    s->c = *c;
    s->embed = *embed;
    s->out_norm = *out_norm;
    s->n_ctx = n_ctx;
    s->q_dim = c->n_heads * c->head_dim;
    s->kv_dim = c->n_kv_heads * c->head_dim;
    s->layers = (orc_layer *)malloc(c->n_layers * sizeof *s->layers);
    const size_t half = c->head_dim / 2, kv = (size_t)n_ctx * s->kv_dim * c->n_layers;
    s->rope_cos = (float *)malloc((size_t)n_ctx * half * sizeof(float));
    s->rope_sin = (float *)malloc((size_t)n_ctx * half * sizeof(float));
    s->k_cache = (float *)calloc(kv, sizeof(float));
    s->v_cache = (float *)calloc(kv, sizeof(float));
    s->x = (float *)malloc(c->d_model * sizeof(float));
    s->h = (float *)malloc(c->d_model * sizeof(float));
    s->q = (float *)malloc(s->q_dim * sizeof(float));
    s->attn = (float *)malloc(s->q_dim * sizeof(float));
    s->proj = (float *)malloc(c->d_model * sizeof(float));
    s->gate = (float *)malloc(c->d_ff * sizeof(float));
    s->up = (float *)malloc(c->d_ff * sizeof(float));
    s->scores = (float *)malloc((size_t)n_ctx * c->n_heads * sizeof(float));
    s->logits = (float *)malloc((size_t)c->vocab * sizeof(float));
    if (!s->layers || !s->rope_cos || !s->rope_sin || !s->k_cache || !s->v_cache || !s->x ||
        !s->h || !s->q || !s->attn || !s->proj || !s->gate || !s->up || !s->scores ||
        !s->logits) {
        orc_qwen3_free(s);
        return NULL;
    }
    memcpy(s->layers, layers, c->n_layers * sizeof *s->layers);
    rope_tables(s->rope_cos, s->rope_sin, c->head_dim, n_ctx, c->rope_theta);
    return s;
}

void orc_qwen3_free(orc_qwen3 *s) {
    if (s == NULL) return;
    free(s->layers); free(s->rope_cos); free(s->rope_sin);
    free(s->k_cache); free(s->v_cache); free(s->x); free(s->h); free(s->q);
    free(s->attn); free(s->proj); free(s->gate); free(s->up); free(s->scores);
    free(s->logits);
    free(s);
}

float *orc_qwen3_k_cache(orc_qwen3 *s) { return s->k_cache; }
float *orc_qwen3_v_cache(orc_qwen3 *s) { return s->v_cache; }
void orc_qwen3_set_n_past(orc_qwen3 *s, uint32_t n) { s->n_past = n; }
uint32_t orc_qwen3_n_past(const orc_qwen3 *s) { return s->n_past; }
/* The last layer's normalised, rotated query heads and attention output of
 * the most recent step (n_heads * head_dim floats each). */
const float *orc_qwen3_last_q(const orc_qwen3 *s) { return s->q; }
const float *orc_qwen3_last_attn(const orc_qwen3 *s) { return s->attn; }

int orc_qwen3_forward(orc_qwen3 *s, uint32_t token, float *logits) {
    const orc_qwen3_config *c = &s->c;
    if (s->n_past >= s->n_ctx || token >= s->embed.rows) return -1;
    const uint32_t pos = s->n_past, n_kv = pos + 1;
    const size_t per_layer = (size_t)s->n_ctx * s->kv_dim;

    /* src/arch_qwen3.c:160-176, 186: the embedding row, decoded, unscaled. */
    {
        uint64_t be, bb;
        if (orc_type_geometry(s->embed.type, &be, &bb) != 0) return -1;
        const size_t rb = (size_t)(s->embed.cols / be * bb);
        if (orc_dequant_matrix(s->embed.type,
                               (const unsigned char *)s->embed.data + (size_t)token * rb,
                               1, c->d_model, s->x) != 0)
            return -1;
    }

    for (uint32_t l = 0; l < c->n_layers; l++) {
        const orc_layer *w = &s->layers[l];
        float *k_layer = s->k_cache + (size_t)l * per_layer;
        float *v_layer = s->v_cache + (size_t)l * per_layer;
        float *k_slot = k_layer + (size_t)pos * s->kv_dim;
        float *v_slot = v_layer + (size_t)pos * s->kv_dim;

        rms_norm(s->h, s->x, (const float *)w->attn_norm.data, c->d_model, c->rms_eps);
        if (proj(&w->wq, s->h, s->q) || proj(&w->wk, s->h, k_slot) ||
            proj(&w->wv, s->h, v_slot))
            return -1;
        rms_norm_heads(s->q, (const float *)w->q_norm.data, c->n_heads, c->head_dim, c->rms_eps);
        rms_norm_heads(k_slot, (const float *)w->k_norm.data, c->n_kv_heads, c->head_dim,
                       c->rms_eps);
        rope(s, s->q, c->n_heads, pos);
        rope(s, k_slot, c->n_kv_heads, pos);

        attn_job aj = { s, k_layer, v_layer, n_kv };
        orc_pool_run((int)c->n_heads, attn_head, &aj);

        if (proj(&w->wo, s->attn, s->proj)) return -1;
        for (uint32_t i = 0; i < c->d_model; i++) s->x[i] = s->x[i] + s->proj[i];

        rms_norm(s->h, s->x, (const float *)w->ffn_norm.data, c->d_model, c->rms_eps);
        if (proj(&w->gate, s->h, s->gate) || proj(&w->up, s->h, s->up)) return -1;
        for (uint32_t i = 0; i < c->d_ff; i++)
            s->gate[i] = s->gate[i] * sigmoid_stable(s->gate[i]) * s->up[i];
        if (proj(&w->down, s->gate, s->proj)) return -1;
        for (uint32_t i = 0; i < c->d_model; i++) s->x[i] = s->x[i] + s->proj[i];
    }

    rms_norm(s->h, s->x, (const float *)s->out_norm.data, c->d_model, c->rms_eps);
    if (proj(&s->embed, s->h, s->logits)) return -1;   /* tied head */
    s->n_past++;
    if (logits) memcpy(logits, s->logits, (size_t)c->vocab * sizeof(float));
    return 0;
}

/* src/sampler.c:122-129: strict '>' keeps the first maximum. */
uint32_t orc_argmax(const float *logits, size_t n) {
    uint32_t best = 0;
    float bv = logits[0];
    for (size_t i = 1; i < n; i++)
        if (logits[i] > bv) { bv = logits[i]; best = (uint32_t)i; }
    return best;
}
