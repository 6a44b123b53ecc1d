/* decode.c — the resident Qwen3 decode step on one GPU (C11 host side).
 *
 * Mirrors the reference decoder's interface and state
 * (src/arch_qwen3.h:21-62, src/arch_qwen3.c:89-252):
 *   - the model's bytes are uploaded once, unchanged, and every tensor is
 *     used in place (the GGUF block layout is never repacked);
 *   - the state owns the f32 KV cache [layer][n_ctx][kv_dim] (a position is
 *     contiguous), the RoPE tables built exactly like the reference's (angles
 *     in double, rounded to f32 once), and every scratch buffer, all
 *     allocated at init; nothing allocates in the token loop;
 *   - forward(token, logits) advances one position and returns -1 when the
 *     context is full, like mynah_slm_forward.
 *
 * One step is a fixed sequence of launches on the library stream: embedding
 * row, then per layer the q/k/v GEMVs as one grouped launch that also
 * computes the RMSNorm of their input (K and V written straight into the
 * cache slot), attention scores (QK-norm and RoPE folded in), softmax and
 * weighted V sum, the o GEMV with the residual add, gate/up as one paired
 * launch (RMSNorm in front, SwiGLU behind), the down GEMV with the residual
 * add; then the final RMSNorm, the tied head (each workgroup leaving the key
 * of its largest logit) and the greedy argmax over those keys, which also
 * advances the device-side position. The token and the position live in device memory, so the step is
 * captured once as a hipGraph and replayed for every generated token.
 *
 * SPDX-License-Identifier: MIT */
#define _GNU_SOURCE
#include "kernels_hip.h"
#include "mynah_decode.h"
#include "mynah_generate.h"
#include "runtime_internal.h"
#include "sample.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

typedef struct {
    int type;
    uint64_t rows, cols, row_bytes;
    const unsigned char *dev;
} dtensor;

/* STEP_MULTI + v: STEP_BATCH consecutive steps of variant v in one graph
 * (the counters live on the device, so the steps are identical launches);
 * it saves the per-launch gap between graphs. STEP_SAMPLE is STEP_FULL with
 * the device sampler between the head and the advance. */
enum { STEP_FULL = 0, STEP_PREFILL = 1, STEP_SAMPLE = 2, STEP_MULTI = 3, STEP_VARIANTS = 6 };
#define STEP_BATCH 8u

/* Scratch of the device sampler (sample.hip) for one vocabulary: the
 * exponentials, each workgroup's first-maximum key, double-double sum and
 * top_k keys, the picked id's key, and (standalone sampling) the logits. */
typedef struct {
    float *e, *logits;
    unsigned long long *wkey, *cand, *key;
    double *wsum;
    uint32_t nwg;
} samp_scratch;

/* Context buckets: a launch whose last step attends n_kv positions runs the
 * graph of the first bucket holding n_kv (its capacity clamped to n_ctx),
 * whose attention grids (16- or 32-position chunks) and exact PV kernel
 * (probabilities in LDS up to 4096 positions) are sized for that capacity,
 * not for the whole context. Capacities 256, 512, 1024, 2048, 3072, 4096,
 * then doubling to 2^20. */
#define N_BUCKETS 14u

typedef struct {
    dtensor attn_norm, wq, wk, wv, q_norm, k_norm, wo, ffn_norm, gate, up, down;
} dlayer;

struct mynah_qwen3 {
    mynah_qwen3_shape c;
    uint32_t n_ctx, n_past, q_dim, kv_dim;
    float scale;
    unsigned char *blob;            /* the model bytes, unchanged */
    dtensor embed, out_norm, head;
    dlayer *layers;
    float *k_cache, *v_cache, *rope_cos, *rope_sin;
    float *rope_now;          /* cos | sin of the position the next step writes (2 x hd / 2) */
    float *x, *q, *attn, *act, *logits, *scores;
    uint32_t *counters;             /* token, pos, step, forced-token count */
    uint32_t *forced;               /* prompt tokens replayed before greedy steps */
    unsigned long long *keys;       /* head workgroups' argmax keys */
    uint32_t n_keys;
    uint32_t sstride;               /* floats between the score rows of two heads */
    uint32_t *tokens;               /* [n_ctx] generated ids */
    /* Captured steps: [STEP_FULL] with the head and argmax, [STEP_PREFILL]
     * without the head (a prompt token whose logits nobody reads); one per
     * context bucket (the attention launches sized for the positions the
     * step reaches). */
    hipGraph_t graph[STEP_VARIANTS][N_BUCKETS];
    hipGraphExec_t exec[STEP_VARIANTS][N_BUCKETS];
    int graph_state[STEP_VARIANTS][N_BUCKETS];  /* 0 not tried, 1 ready, -1 unavailable */
    int graph_order[STEP_VARIANTS][N_BUCKETS];  /* GEMV order the graph was captured with */
    int graph_attn[STEP_VARIANTS][N_BUCKETS];   /* attention mode the graph was captured with */
    int buckets;                    /* 0: every step sized for the whole context */
    int attn_mode;                  /* MYNAH_ATTN_EXACT or MYNAH_ATTN_SPLIT */
    uint32_t nch_max;               /* split-attention partial slots per key head and group */
    uint32_t as_ch;                 /* positions per chunk at the whole context */
    float *pm, *po;                 /* split-attention partials: chunk max, weighted V */
    double *pl;                     /* split-attention partials: chunk exp sums */
    /* Batched prompt prefill (allocated on first use for pf_cap tokens):
     * rows of X, normalised X, Q (rotated in place), attention output,
     * gate (then SwiGLU) and up activations, scores, and the tokens. */
    int prefill_mode;               /* MYNAH_PREFILL_BATCHED or MYNAH_PREFILL_STEPS */
    uint32_t pf_cap;
    float *pf_x, *pf_xn, *pf_q, *pf_att, *pf_g, *pf_u, *pf_s;
    uint32_t *pf_tok;
    float *host_logits;             /* pinned: logits for a host-side sampler */
    /* The device sampler's state for sampled steps (a copy of the caller's
     * sampler for the length of a generation) and its scratch. */
    SampState *samp_st;
    samp_scratch samp_sc;
};

#define TOKEN(s) ((s)->counters + 0)
#define POS(s) ((s)->counters + 1)
#define STEP(s) ((s)->counters + 2)
#define NFORCED(s) ((s)->counters + 3)


/* The largest context (positions) a state takes: 2^20, far beyond any Qwen3
 * (40960), small enough that every offset fits 32 bits. */
#define MYNAH_MAX_CTX (1u << 20)
/* Exact attention keeps a key head's score rows (group * sstride floats) in
 * LDS up to this size; longer contexts take the two-launch form. */
#define EXACT_LDS_SCORES (48u * 1024u)

static int fail(char *err, size_t errsz, const char *msg, const char *detail) {
    if (err && errsz) snprintf(err, errsz, "%s%s%s", msg, detail ? ": " : "", detail ? detail : "");
    mynah_set_error("%s%s%s", msg, detail ? ": " : "", detail ? detail : "");
    return -1;
}

static const mynah_synth_tensor *find(const mynah_synth_tensor *t, size_t n, const char *name) {
    for (size_t i = 0; i < n; i++)
        if (strncmp(t[i].name, name, sizeof t[i].name) == 0) return &t[i];
    return NULL;
}

static int bind(dtensor *out, const mynah_synth_tensor *table, size_t count,
                const unsigned char *blob, uint64_t blob_bytes, const char *name, int want_type,
                uint64_t rows, uint64_t cols, char *err, size_t errsz) {
    const mynah_synth_tensor *t = find(table, count, name);
    if (t == NULL) return fail(err, errsz, "missing tensor", name);
    if (t->rows != rows || t->cols != cols || (want_type >= 0 && t->type != want_type))
        return fail(err, errsz, "tensor has the wrong shape or type", name);
    if (t->offset > blob_bytes || t->nbytes > blob_bytes - t->offset)
        return fail(err, errsz, "tensor outside the blob", name);
    /* The kernels read weights and norm vectors in 16-byte pieces. */
    if ((t->offset & 15u) != 0) return fail(err, errsz, "tensor offset not 16-byte aligned", name);
    size_t rb = cols * 4;
    /* The step's kernels take F32, Q4_0, Q4_K, Q5_K, Q6_K and Q8_0 tensors. */
    if (t->type != 0 && mynah_geometry(t->type, rows, cols, &rb) != 0)
        return fail(err, errsz, "tensor type has no kernel in the decode step", name);
    /* The kernels read rows * row_bytes from the tensor's offset: the table's
     * byte count must cover them (it lies inside the blob, checked above). */
    if (rows > UINT64_MAX / rb || t->nbytes < rows * rb)
        return fail(err, errsz, "tensor byte count shorter than its rows", name);
    out->type = t->type;
    out->rows = rows;
    out->cols = cols;
    out->row_bytes = rb;
    out->dev = blob + t->offset;
    return 0;
}

static void *dalloc(size_t bytes, int *ok) {
    void *p = NULL;
    if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) {
        *ok = 0;
        return NULL;
    }
    return p;
}

/* The head launch of a full step: final RMSNorm fused in front
 * (src/arch_qwen3.c:239), one argmax key per workgroup behind it
 * (src/sampler.c:124-129). */
static int head_group(const mynah_qwen3 *s, mynah_gemv_group *g) {
    memset(g, 0, sizeof *g);
    g->n = 1;
    if (mynah_gemv_desc_init(&g->d[0], s->head.type, s->head.dev, s->head.rows, s->head.cols,
                             s->x, s->logits) != 0)
        return -1;
    g->d[0].norm_w = (const float *)s->out_norm.dev;
    g->d[0].eps = s->c.rms_eps;
    g->d[0].keys = s->keys;
    return 0;
}

static void samp_scratch_free(samp_scratch *sc);
static int samp_enqueue(mynah_device *d, hipStream_t st, SampState *state, const samp_scratch *sc,
                        float *logits, uint32_t vocab, uint32_t accept);

void mynah_hip_qwen3_free(mynah_qwen3 *s) {
    if (s == NULL) return;
    for (int v = 0; v < STEP_VARIANTS; v++)
        for (uint32_t b = 0; b < N_BUCKETS; b++) {
            if (s->exec[v][b]) (void)hipGraphExecDestroy(s->exec[v][b]);
            if (s->graph[v][b]) (void)hipGraphDestroy(s->graph[v][b]);
        }
    void *bufs[] = {s->keys, s->blob, s->k_cache, s->v_cache, s->rope_cos, s->rope_sin, s->rope_now,
                    s->x, s->q,
                    s->attn, s->act, s->logits, s->scores, s->counters, s->tokens, s->forced, s->pm, s->pl,
                    s->po, s->pf_x, s->pf_xn, s->pf_q, s->pf_att, s->pf_g, s->pf_u, s->pf_s,
                    s->pf_tok};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++)
        if (bufs[i]) (void)hipFree(bufs[i]);
    if (s->host_logits) (void)hipHostFree(s->host_logits);
    samp_scratch_free(&s->samp_sc);
    if (s->samp_st) (void)hipFree(s->samp_st);
    free(s->layers);
    free(s);
}

static uint32_t split_chunk(const mynah_qwen3 *s, uint32_t cap, int *kernel);
static uint32_t bucket_cap(uint32_t b);

mynah_qwen3 *mynah_hip_qwen3_new(const mynah_qwen3_shape *c, const mynah_synth_tensor *table,
                                 size_t count, const void *blob, uint64_t blob_bytes,
                                 uint32_t n_ctx, char *err, size_t errsz) {
    const uint64_t at = 0;
    return mynah_qwen3_new_parts(c, table, count, &blob, &blob_bytes, &at, 1, blob_bytes, n_ctx,
                                 err, errsz);
}

mynah_qwen3 *mynah_qwen3_new_parts(const mynah_qwen3_shape *c, const mynah_synth_tensor *table,
                                   size_t count, const void *const *parts,
                                   const uint64_t *part_bytes, const uint64_t *part_at,
                                   uint32_t n_parts, uint64_t blob_bytes, uint32_t n_ctx,
                                   char *err, size_t errsz) {
    if (c == NULL || table == NULL || parts == NULL || n_parts == 0 || n_ctx == 0) {
        fail(err, errsz, "null argument", NULL);
        return NULL;
    }
    /* Any context the model and HBM allow (src/arch_qwen3.c:89-131 takes any
     * n_ctx): exact attention whose score rows fit the LDS keeps them there,
     * longer ones run its two-launch form. */
    if (c->n_kv_heads == 0 || c->n_heads % c->n_kv_heads != 0 ||
        c->n_heads / c->n_kv_heads > 8 || c->n_heads / c->n_kv_heads < 2 || c->head_dim != 128 ||
        c->d_model % 256 != 0 || c->d_ff % 256 != 0 || c->vocab % 4 != 0 ||
        n_ctx > MYNAH_MAX_CTX) {
        fail(err, errsz, "unsupported shape", NULL);
        return NULL;
    }
    mynah_device *d = mynah_dev();
    if (d == NULL) {
        fail(err, errsz, "no device", mynah_hip_last_error());
        return NULL;
    }
    mynah_qwen3 *s = (mynah_qwen3 *)calloc(1, sizeof *s);
    if (s == NULL) return NULL;
    s->c = *c;
    s->n_ctx = n_ctx;
    s->q_dim = c->n_heads * c->head_dim;
    s->kv_dim = c->n_kv_heads * c->head_dim;
    s->scale = 1.0f / sqrtf((float)c->head_dim);      /* src/kernels.c:233 */
    s->layers = (dlayer *)calloc(c->n_layers, sizeof *s->layers);
    int ok = s->layers != NULL;

    /* The parts (the shards' data sections of a split checkpoint; one part
     * otherwise) go to their places in one device blob, unchanged; the gaps
     * between them are never read. */
    s->blob = (unsigned char *)dalloc(blob_bytes, &ok);
    for (uint32_t i = 0; ok && i < n_parts; i++) {
        if (parts[i] == NULL || part_at[i] > blob_bytes || part_bytes[i] > blob_bytes - part_at[i])
            ok = 0;
        else if (part_bytes[i] != 0 && hipMemcpy(s->blob + part_at[i], parts[i], part_bytes[i],
                                                 hipMemcpyHostToDevice) != hipSuccess)
            ok = 0;
    }
    if (!ok) {
        fail(err, errsz, "cannot upload the model", NULL);
        mynah_hip_qwen3_free(s);
        return NULL;
    }

    const uint64_t dm = c->d_model, ff = c->d_ff, hd = c->head_dim;
    int rc = bind(&s->embed, table, count, s->blob, blob_bytes, "token_embd.weight", -1, c->vocab,
                  dm, err, errsz);
    rc = rc ? rc : bind(&s->out_norm, table, count, s->blob, blob_bytes, "output_norm.weight", 0,
                        1, dm, err, errsz);
    if (rc == 0 && find(table, count, "output.weight"))
        rc = bind(&s->head, table, count, s->blob, blob_bytes, "output.weight", -1, c->vocab, dm,
                  err, errsz);
    else
        s->head = s->embed;                              /* tied (src/model.c:200-203) */
    for (uint32_t l = 0; l < c->n_layers && rc == 0; l++) {
        dlayer *L = &s->layers[l];
        char n[64];
#define B(field, suffix, ty, r, cc)                                                     \
        if (rc == 0) {                                                                  \
            snprintf(n, sizeof n, "blk.%u." suffix, l);                                 \
            rc = bind(&L->field, table, count, s->blob, blob_bytes, n, ty, r, cc, err,  \
                      errsz);                                                           \
        }
        B(attn_norm, "attn_norm.weight", 0, 1, dm)
        B(wq, "attn_q.weight", -1, s->q_dim, dm)
        B(wk, "attn_k.weight", -1, s->kv_dim, dm)
        B(wv, "attn_v.weight", -1, s->kv_dim, dm)
        B(q_norm, "attn_q_norm.weight", 0, 1, hd)
        B(k_norm, "attn_k_norm.weight", 0, 1, hd)
        B(wo, "attn_output.weight", -1, dm, s->q_dim)
        B(ffn_norm, "ffn_norm.weight", 0, 1, dm)
        B(gate, "ffn_gate.weight", -1, ff, dm)
        B(up, "ffn_up.weight", -1, ff, dm)
        B(down, "ffn_down.weight", -1, dm, ff)
#undef B
        if (rc == 0 && (L->gate.type != L->up.type || L->gate.type == 0 || L->wq.type == 0 ||
                        L->wk.type == 0 || L->wv.type == 0 || L->wo.type == 0 ||
                        L->down.type == 0))
            rc = fail(err, errsz, "projection types must be quantized, gate/up alike", n);
    }
    if (rc == 0 && s->head.type == 0)
        rc = fail(err, errsz, "the output head must be quantized", NULL);
    if (rc != 0) {
        mynah_hip_qwen3_free(s);
        return NULL;
    }

    const size_t kv = (size_t)c->n_layers * n_ctx * s->kv_dim;
    const size_t half = hd / 2;
    s->k_cache = (float *)dalloc(kv * 4, &ok);
    s->v_cache = (float *)dalloc(kv * 4, &ok);
    s->rope_cos = (float *)dalloc((size_t)n_ctx * half * 4, &ok);
    s->rope_sin = (float *)dalloc((size_t)n_ctx * half * 4, &ok);
    s->rope_now = (float *)dalloc(2 * half * 4, &ok);
    s->x = (float *)dalloc(dm * 4, &ok);
    s->q = (float *)dalloc((size_t)s->q_dim * 4, &ok);
    s->attn = (float *)dalloc((size_t)s->q_dim * 4, &ok);
    s->act = (float *)dalloc(ff * 4, &ok);
    s->logits = (float *)dalloc((size_t)c->vocab * 4, &ok);
    s->sstride = (n_ctx + 63) & ~63u;
    s->scores = (float *)dalloc((size_t)c->n_heads * s->sstride * 4, &ok);
    s->counters = (uint32_t *)dalloc(16, &ok);
    s->forced = (uint32_t *)dalloc((size_t)n_ctx * 4, &ok);
    s->buckets = getenv("MYNAH_CTX_BUCKETS") == NULL || atoi(getenv("MYNAH_CTX_BUCKETS")) != 0;
    {
        /* Partial slots for the bucket with the most chunks. */
        s->as_ch = split_chunk(s, n_ctx, NULL);
        s->nch_max = (n_ctx + s->as_ch - 1) / s->as_ch;
        for (uint32_t b = 0; s->buckets && b < N_BUCKETS && bucket_cap(b) < n_ctx; b++) {
            const uint32_t ch = split_chunk(s, bucket_cap(b), NULL);
            const uint32_t n = (bucket_cap(b) + ch - 1) / ch;
            if (n > s->nch_max) s->nch_max = n;
        }
        const size_t parts = (size_t)c->n_kv_heads * s->nch_max * (c->n_heads / c->n_kv_heads);
        s->pm = (float *)dalloc(parts * 4, &ok);
        s->pl = (double *)dalloc(parts * 8, &ok);
        s->po = (float *)dalloc(parts * 128 * 4, &ok);
    }
    /* One argmax key per head workgroup: sized from the head launch as it
     * is planned now (x and logits exist, so the plan sees its real
     * operands); enqueue_step re-plans and refuses a launch that would
     * outgrow the buffer before anything is enqueued. */
    s->n_keys = c->vocab / 8 + 64;
    if (ok) {
        mynah_gemv_group hg;
        uint32_t grid = 0;
        if (head_group(s, &hg) != 0 ||
            mynah_gemv_group_geometry(&hg, MYNAH_GEMV_EXACT, NULL, &grid) != 0) {
            fail(err, errsz, "the output head has no GEMV launch", mynah_hip_last_error());
            mynah_hip_qwen3_free(s);
            return NULL;
        }
        if (grid > s->n_keys) s->n_keys = grid;
    }
    s->keys = (unsigned long long *)dalloc((size_t)s->n_keys * 8, &ok);
    s->tokens = (uint32_t *)dalloc((size_t)n_ctx * 4, &ok);
    if (!ok) {
        fail(err, errsz, "out of device memory for the state", NULL);
        mynah_hip_qwen3_free(s);
        return NULL;
    }
    /* src/kernels.c:141-164: angle p * theta^(-2i/hd) in double, cos/sin
     * rounded to f32 once. */
    float *cs = (float *)malloc((size_t)n_ctx * half * 4), *sn = (float *)malloc((size_t)n_ctx * half * 4);
    if (cs == NULL || sn == NULL) ok = 0;
    for (uint32_t i = 0; ok && i < half; i++) {
        const double inv = 1.0 / pow((double)c->rope_theta, (2.0 * (double)i) / (double)hd);
        for (uint32_t p = 0; p < n_ctx; p++) {
            const double a = (double)p * inv;
            cs[(size_t)p * half + i] = (float)cos(a);
            sn[(size_t)p * half + i] = (float)sin(a);
        }
    }
    if (ok && (hipMemcpy(s->rope_cos, cs, (size_t)n_ctx * half * 4, hipMemcpyHostToDevice) != hipSuccess ||
               hipMemcpy(s->rope_sin, sn, (size_t)n_ctx * half * 4, hipMemcpyHostToDevice) != hipSuccess ||
               hipMemset(s->counters, 0, 16) != hipSuccess ||
               hipMemset(s->k_cache, 0, kv * 4) != hipSuccess ||
               hipMemset(s->v_cache, 0, kv * 4) != hipSuccess))
        ok = 0;
    free(cs);
    free(sn);
    if (!ok) {
        fail(err, errsz, "state initialisation failed", NULL);
        mynah_hip_qwen3_free(s);
        return NULL;
    }
    return s;
}

/* ── the step ────────────────────────────────────────────────────────────── */

static int gemv_desc(mynah_gemv_desc *g, const dtensor *w, const float *x, float *y) {
    return mynah_gemv_desc_init(g, w->type, w->dev, w->rows, w->cols, x, y);
}

/* The grouped GEMV launches of layer l: LG_QKV q/k/v with the attention
 * norm in front and K/V written into the cache slot at the position,
 * LG_O the output projection onto the residual, LG_FFN gate/up with the FFN
 * norm in front and SwiGLU behind, LG_DOWN the down projection onto the
 * residual. */
enum { LG_QKV, LG_O, LG_FFN, LG_DOWN, LG_COUNT };

static int layer_group(const mynah_qwen3 *s, uint32_t l, int which, mynah_gemv_group *g) {
    const mynah_qwen3_shape *c = &s->c;
    const dlayer *L = &s->layers[l];
    const size_t per_layer = (size_t)s->n_ctx * s->kv_dim;
    int rc;
    memset(g, 0, sizeof *g);
    g->n = 1;
    switch (which) {
    case LG_QKV: {
        float *kl = s->k_cache + l * per_layer, *vl = s->v_cache + l * per_layer;
        uint32_t *pos = POS(s);
        g->n = 3;
        rc = gemv_desc(&g->d[0], &L->wq, s->x, s->q);
        rc = rc ? rc : gemv_desc(&g->d[1], &L->wk, s->x, kl);
        rc = rc ? rc : gemv_desc(&g->d[2], &L->wv, s->x, vl);
        if (rc) return rc;
        for (int k = 0; k < 3; k++) {      /* src/arch_qwen3.c:201 folded in */
            g->d[k].norm_w = (const float *)L->attn_norm.dev;
            g->d[k].eps = c->rms_eps;
        }
        g->d[1].ypos = pos;
        g->d[1].ystride = s->kv_dim;
        g->d[2].ypos = pos;
        g->d[2].ystride = s->kv_dim;
        return 0;
    }
    case LG_O:
        rc = gemv_desc(&g->d[0], &L->wo, s->attn, s->x);
        g->d[0].res = s->x;
        return rc;
    case LG_FFN:
        rc = gemv_desc(&g->d[0], &L->gate, s->x, s->act);
        g->d[0].w2 = L->up.dev;
        g->d[0].norm_w = (const float *)L->ffn_norm.dev;     /* src/arch_qwen3.c:226 */
        g->d[0].eps = c->rms_eps;
        return rc;
    default:
        rc = gemv_desc(&g->d[0], &L->down, s->act, s->x);
        g->d[0].res = s->x;
        return rc;
    }
}

static long env_or(const char *name, long dflt) {
    const char *e = getenv(name);
    return (e != NULL && e[0] != '\0') ? strtol(e, NULL, 10) : dflt;
}

/* L2 prefetch of the decode GEMVs' weights: each grouped launch of a step
 * carries one workgroup per MYNAH_PREFETCH_BPW bytes (default 8192; 0
 * none), or MYNAH_PREFETCH_WGS workgroups (a multiple of 8), that pull a
 * later GEMV's weights into the L2 of the XCDs that will read them, one
 * byte touched per 2^MYNAH_PREFETCH_STEP bytes (default 7, the L2 line):
 * the same GEMV of the next layer when a layer fits the L2s (below), else
 * the next GEMV, skipping those above MYNAH_PREFETCH_MAX bytes (default
 * 6 MiB, about what the L2s keep beside the K/V traffic; measured, 0.6B
 * decode 974 -> 993 tok/s, the 4B's larger GEMVs lost a little). */
static uint32_t prefetch_wgs(void) {
    const long v = env_or("MYNAH_PREFETCH_WGS", 0);
    return v > 0 && v <= 4096 ? (uint32_t)(v & ~7L) : 0u;
}

/* Chunk size of the split attention for a launch sized for `cap`
 * positions, and its kernel: the kernels for 2 and 4 query heads per key
 * head take 32 positions up to 32768 (1,024 chunks), 64 up to 65536 and 128
 * beyond (MYNAH_AS_CH=32|64|128 forces one); other groups take the generic
 * kernel's 32. More, smaller chunks run faster while the combine stays
 * small: Qwen3-4B decode at context 2048, split mode, 467.6 tok/s with 32
 * positions, 456.7 with 64, 446.8 with 128. */
static uint32_t split_chunk(const mynah_qwen3 *s, uint32_t cap, int *kernel) {
    const uint32_t group = s->c.n_heads / s->c.n_kv_heads;
    uint32_t ch = cap <= 32768u ? 32u : cap <= 65536u ? 64u : 128u;
    const uint32_t want = (uint32_t)env_or("MYNAH_AS_CH", 0);
    if (want == 32u || want == 64u || want == 128u) ch = want;
    if (group != 2u && group != 4u) {
        if (kernel) *kernel = MYNAH_K_ATTN_SPLIT;
        return MYNAH_AS_CH;
    }
    static const int k2[3] = {MYNAH_K_ATTN_SPLIT_G2_32, MYNAH_K_ATTN_SPLIT_G2_64,
                              MYNAH_K_ATTN_SPLIT_G2_128};
    static const int k4[3] = {MYNAH_K_ATTN_SPLIT_G4_32, MYNAH_K_ATTN_SPLIT_G4_64,
                              MYNAH_K_ATTN_SPLIT_G4_128};
    const int i = ch == 32u ? 0 : ch == 64u ? 1 : 2;
    if (kernel) *kernel = group == 2u ? k2[i] : k4[i];
    return ch;
}

static uint32_t bucket_cap(uint32_t b) {
    static const uint32_t caps[6] = {256u, 512u, 1024u, 2048u, 3072u, 4096u};
    return b < 6u ? caps[b] : 8192u << (b - 6u);
}

/* The bucket of a launch whose last step attends n_kv positions, and its
 * capacity (MYNAH_CTX_BUCKETS=0: one bucket, the whole context). */
static uint32_t ctx_bucket(const mynah_qwen3 *s, uint32_t n_kv, uint32_t *cap) {
    uint32_t b = 0;
    if (!s->buckets) {
        *cap = s->n_ctx;
        return 0;
    }
    while (bucket_cap(b) < n_kv && bucket_cap(b) < s->n_ctx) b++;
    *cap = bucket_cap(b) < s->n_ctx ? bucket_cap(b) : s->n_ctx;
    return b;
}

/* The exact attention's PV kernel for a launch sized for `cap` positions,
 * or -1 for the eight-lane kernels (MYNAH_ATTN_PV=0, or head_dim other than
 * 128). Up to 4 columns of 256 * MYNAH_PV_LW scores (one float4 per loader
 * thread and column) the softmax runs inside it; longer contexts read the
 * probabilities from the scores rows, normalised in place first. */
static int pv_kernel(const mynah_qwen3 *s, uint32_t cap) {
    const uint32_t col = 256u * MYNAH_PV_LW;
    if (env_or("MYNAH_ATTN_PV", 1) == 0 || s->c.head_dim != 128) return -1;
    if (cap > 4u * col) return MYNAH_K_ATTN_PV_M;
    static const int by_cols[4] = {MYNAH_K_ATTN_PV_1, MYNAH_K_ATTN_PV_2, MYNAH_K_ATTN_PV_3,
                                   MYNAH_K_ATTN_PV_4};
    return by_cols[(cap - 1u) / col];
}

static uint32_t prefetch_step(void) {
    const long v = env_or("MYNAH_PREFETCH_STEP", 7);
    return v >= 2 && v <= 12 ? (uint32_t)v : 7u;
}

/* One step of variant `variant` whose attention launches are sized for
 * `cap` positions; p0 is the first position the launch (its graph) runs at. */
static int enqueue_step(mynah_qwen3 *s, mynah_device *d, hipStream_t st, int variant,
                        uint32_t p0, uint32_t cap) {
    const mynah_qwen3_shape *c = &s->c;
    const size_t per_layer = (size_t)s->n_ctx * s->kv_dim;
    uint32_t *tok = TOKEN(s), *pos = POS(s), *step = STEP(s);
    uint32_t head_tiles = 0;
    const uint32_t pf_wgs = prefetch_wgs(), pf_step = prefetch_step();
    const long pf_bpw = env_or("MYNAH_PREFETCH_BPW", 8192);
    const long pf_max = env_or("MYNAH_PREFETCH_MAX", 6L << 20);
    const uint32_t pf_b = pf_bpw > 0 && pf_bpw < (1L << 30) ? (uint32_t)pf_bpw : 0u;
    const uint64_t pf_m = pf_max > 0 ? (uint64_t)pf_max : UINT64_MAX;
    mynah_gemv_group lg[LG_COUNT], next_qkv;
    int rc = 0;
    for (int k = 0; k < LG_COUNT && rc == 0; k++) rc = layer_group(s, 0, k, &lg[k]);
    /* Whole layers of at most MYNAH_PREFETCH_LAYER_MAX bytes (default
     * 16 MiB, half the eight L2s) are prefetched a layer ahead, larger ones
     * GEMV by GEMV (0.6B: 1,017 -> 1,028 tok/s; at 4B's 67 MB layers a
     * layer ahead lost 1-2 %). */
    uint64_t layer_bytes = 0;
    for (int k = 0; k < LG_COUNT; k++)
        for (uint32_t i = 0; i < lg[k].n; i++)
            layer_bytes += (uint64_t)lg[k].d[i].rows * lg[k].d[i].row_bytes *
                           (lg[k].d[i].w2 ? 2u : 1u);
    const long pf_lmax = env_or("MYNAH_PREFETCH_LAYER_MAX", 16L << 20);
    const int pf_ahead = (pf_wgs || pf_b) && c->n_layers > 1 && pf_lmax > 0 &&
                         layer_bytes <= (uint64_t)pf_lmax;
    for (uint32_t l = 0; l < c->n_layers && rc == 0; l++) {
        const dlayer *L = &s->layers[l];
        float *kl = s->k_cache + l * per_layer, *vl = s->v_cache + l * per_layer;
        const int more = l + 1 < c->n_layers;
        if (l > 0) {
            lg[LG_QKV] = next_qkv;
            for (int k = LG_O; k < LG_COUNT && rc == 0; k++) rc = layer_group(s, l, k, &lg[k]);
        }
        if (rc == 0 && more) rc = layer_group(s, l + 1, LG_QKV, &next_qkv);
        if (pf_ahead && more) {
            /* A layer ahead: each launch fetches the same launch of the next
             * layer, whose weights then wait in the L2s for a whole layer. */
            for (int k = 0; k < LG_COUNT && rc == 0; k++) {
                mynah_gemv_group nxl;
                rc = k == LG_QKV ? 0 : layer_group(s, l + 1, k, &nxl);
                if (rc == 0)
                    rc = mynah_gemv_prefetch_plan(k == LG_QKV ? &next_qkv : &nxl, -1, pf_wgs,
                                                  pf_b, UINT64_MAX, pf_step, &lg[k].pf);
            }
        }
        for (int k = 0; k < LG_COUNT && rc == 0 && !pf_ahead && (pf_wgs || pf_b); k++) {
            const mynah_gemv_group *nx = k + 1 < LG_COUNT ? &lg[k + 1] : more ? &next_qkv : NULL;
            if (nx) rc = mynah_gemv_prefetch_plan(nx, -1, pf_wgs, pf_b, pf_m, pf_step, &lg[k].pf);
        }
        if (rc) break;
        rc = mynah_gemv_group_launch(d, &lg[LG_QKV], st, NULL, -1);
        if (rc) break;
        if (s->attn_mode == MYNAH_ATTN_SPLIT) {
            const float *q = s->q, *qn = (const float *)L->q_norm.dev;
            const float *kn = (const float *)L->k_norm.dev;
            const float *rnow = s->rope_now;
            float *pm = s->pm, *po = s->po, *out = s->attn;
            double *pl = s->pl;
            int kernel = 0;
            uint32_t ch = split_chunk(s, cap, &kernel);
            uint32_t nchm = (cap + ch - 1) / ch, kvd = s->kv_dim;
            uint32_t group = c->n_heads / c->n_kv_heads;
            float eps = c->rms_eps, scale = s->scale;
            /* Chunks live at the launch's first position stay live in every
             * later step (the graphs replay forward), so they load K/V
             * before the position arrives. */
            uint32_t nctx = cap;
            uint32_t spec = (p0 + ch) / ch;
            if (spec > nchm) spec = nchm;
            if (nchm > s->nch_max) {
                mynah_set_error("split launch of %u chunks exceeds the partials", nchm);
                rc = -1;
                break;
            }
            void *args[] = {&q, &kl, &vl, &qn, &kn, &rnow, &pos, &pm, &pl, &po, &nchm, &kvd,
                            &group, &eps, &scale, &nctx, &spec};
            rc = mynah_launch(d, kernel, c->n_kv_heads, nchm, 128 * group, 0, st, args);
            if (rc) break;
            const float *cpm = pm, *cpo = po;
            const double *cpl = pl;
            /* The four-wave combine finds M and L in wave 0 up to 128 chunks
             * (MYNAH_COMBINE_WAVE0=0: never; same bits). */
            uint32_t w0max = env_or("MYNAH_COMBINE_WAVE0", 1) != 0 ? 128u : 0u;
            void *args2[] = {&pos, &cpm, &cpl, &cpo, &out, &nchm, &group, &w0max, &ch};
            void *args2w[] = {&pos, &cpm, &cpl, &cpo, &out, &nchm, &group, &ch};
            /* Up to MYNAH_AC1_MAX chunks one wave per query head combines
             * (no barrier), past that four (MYNAH_ATTN_COMBINE1=0: always
             * four); same bits. */
            if (nchm <= MYNAH_AC1_MAX && env_or("MYNAH_ATTN_COMBINE1", 1) != 0)
                rc = mynah_launch(d, MYNAH_K_ATTN_COMBINE1, c->n_heads, 1, 64, 0, st, args2w);
            else
                rc = mynah_launch(d, MYNAH_K_ATTN_COMBINE, c->n_heads, 1, 256,
                                  (size_t)nchm * sizeof(float), st, args2);
        } else {
            const float *q = s->q, *qn = (const float *)L->q_norm.dev;
            const float *kn = (const float *)L->k_norm.dev;
            const float *rnow = s->rope_now;
            float *sc = s->scores;
            uint32_t nctx = cap, kvd = s->kv_dim, sstride = s->sstride;
            uint32_t group = c->n_heads / c->n_kv_heads;
            float eps = c->rms_eps, scale = s->scale;
            /* 16-position chunks live at the launch's first position stay
             * live in every later step (the graphs replay forward), so they
             * load their key rows before the position arrives. */
            const uint32_t nsc = (cap + 15) / 16;
            uint32_t spec = (p0 + 16) / 16;
            if (spec > nsc) spec = nsc;
            void *args[] = {&q, &kl, &qn, &kn, &rnow, &pos, &sc, &nctx, &sstride, &kvd,
                            &group, &eps, &scale, &spec};
            rc = mynah_launch(d, MYNAH_K_ATTN_SCORES, c->n_kv_heads, nsc, 256, 0, st, args);
            if (rc) break;
            float *out = s->attn;
            const float *scc = s->scores;
            void *args2[] = {&vl, &scc, &pos, &out, &sstride, &kvd, &group};
            const int pv = pv_kernel(s, cap);
            if (pv >= 0) {
                /* A PV chain in every lane (MYNAH_ATTN_PV=0: the eight-lane
                 * kernels below; same bits). */
                uint32_t nkv = c->n_kv_heads;
                void *args3[] = {&vl, &scc, &pos, &out, &sstride, &kvd, &nkv, &group};
                if (pv == MYNAH_K_ATTN_PV_M) {
                    void *args1[] = {&sc, &pos, &sstride};
                    rc = mynah_launch(d, MYNAH_K_ATTN_SOFTMAX, c->n_heads, 1, 64, 0, st, args1);
                }
                rc = rc ? rc : mynah_launch(d, pv, c->n_heads * (128u / MYNAH_PV_SW), 1,
                                            64u * (1u + MYNAH_PV_LW), 0,
                                            st, args3);
            } else if ((size_t)group * sstride * 4 <= EXACT_LDS_SCORES) {
                rc = mynah_launch(d, MYNAH_K_ATTN_OUT, c->n_kv_heads, c->head_dim / 8, 64 * group,
                                  (size_t)group * sstride * 4, st, args2);
            } else {
                void *args1[] = {&sc, &pos, &sstride};
                rc = mynah_launch(d, MYNAH_K_ATTN_SOFTMAX, c->n_heads, 1, 64, 0, st, args1);
                rc = rc ? rc : mynah_launch(d, MYNAH_K_ATTN_OUT_LONG, c->n_kv_heads,
                                            c->head_dim / 8, 64 * group,
                                            (size_t)group * 1024 * 4, st, args2);
            }
        }
        if (rc) break;
        rc = mynah_gemv_group_launch(d, &lg[LG_O], st, NULL, -1);
        rc = rc ? rc : mynah_gemv_group_launch(d, &lg[LG_FFN], st, NULL, -1);
        rc = rc ? rc : mynah_gemv_group_launch(d, &lg[LG_DOWN], st, NULL, -1);
    }
    if (rc == 0 && (variant == STEP_FULL || variant == STEP_SAMPLE)) {
        /* The final norm (src/arch_qwen3.c:239) runs inside the head GEMV. */
        mynah_gemv_group g;
        /* The exact kernel is also the faster one for the head (its fused
         * norm costs the reordered kernel more), so the head always runs in
         * the reference's order. Its workgroups each write one key: the
         * launch is planned and checked against the key buffer before it is
         * enqueued. */
        rc = head_group(s, &g);
        rc = rc ? rc : mynah_gemv_group_geometry(&g, MYNAH_GEMV_EXACT, NULL, &head_tiles);
        if (rc == 0 && head_tiles > s->n_keys) {
            mynah_set_error("head launch of %u workgroups exceeds the key buffer", head_tiles);
            rc = -1;
        }
        rc = rc ? rc : mynah_gemv_group_launch(d, &g, st, &head_tiles, MYNAH_GEMV_EXACT);
    }
    const unsigned long long *keys = s->keys;
    uint32_t n = head_tiles;
    if (rc == 0 && variant == STEP_SAMPLE) {
        /* src/sampler.c:116-187 on the head's logits; the advance then takes
         * the sampled id as its only key. */
        rc = samp_enqueue(d, st, s->samp_st, &s->samp_sc, s->logits, c->vocab, 1u);
        keys = s->samp_sc.key;
        n = 1;
    }
    if (rc == 0) {
        uint32_t maxs = s->n_ctx;
        uint32_t *toks = s->tokens;
        const unsigned char *tab = s->embed.dev;
        float *x = s->x;
        uint32_t dm = c->d_model, ty = (uint32_t)s->embed.type, rb = (uint32_t)s->embed.row_bytes;
        const uint32_t *forced = s->forced, *nforced = NFORCED(s);
        uint32_t vocab = c->vocab;
        const float *rcos = s->rope_cos, *rsin = s->rope_sin;
        float *rnow = s->rope_now;
        void *args[] = {&keys, &n, &tok, &toks, &pos, &step, &maxs, &tab, &x, &dm, &ty, &rb,
                        &forced, &nforced, &vocab, &rcos, &rsin, &rnow};
        rc = mynah_launch(d, MYNAH_K_ARGMAX, 1, 1, 1024, 0, st, args);
    }
    return rc;
}

/* The embedding of the current token (device counter) into x: the start of a
 * sequence of steps; every step's argmax embeds the token it picks. */
static int embed_current(mynah_qwen3 *s, mynah_device *d) {
    const unsigned char *tab = s->embed.dev;
    uint32_t *tok = TOKEN(s);
    float *x = s->x;
    uint32_t dm = s->c.d_model, ty = (uint32_t)s->embed.type, rb = (uint32_t)s->embed.row_bytes;
    const uint32_t *pos = POS(s);
    const float *rcos = s->rope_cos, *rsin = s->rope_sin;
    float *rnow = s->rope_now;
    uint32_t nctx = s->n_ctx;
    void *args[] = {&tab, &tok, &x, &dm, &ty, &rb, &pos, &rcos, &rsin, &rnow, &nctx};
    return mynah_launch(d, MYNAH_K_EMBED, (dm / 32 + 255) / 256, 1, 256, 0, d->stream, args);
}

/* Steps in one launch of variant v. */
static uint32_t launch_steps(int v) { return v >= STEP_MULTI ? STEP_BATCH : 1u; }

/* Capture variant v for the bucket of a launch starting at position p0 once
 * (or again after the GEMV order or attention mode changed); leaves its
 * state -1 when capture is unavailable. Returns the bucket. */
static uint32_t ensure_graph(mynah_qwen3 *s, mynah_device *d, int v, uint32_t p0) {
    hipStream_t st = d->stream;
    uint32_t cap = 0;
    const uint32_t b = ctx_bucket(s, p0 + launch_steps(v), &cap);
    if (s->graph_state[v][b] == 1 && (s->graph_order[v][b] != mynah_hip_gemv_order() ||
                                      s->graph_attn[v][b] != s->attn_mode)) {
        (void)hipGraphExecDestroy(s->exec[v][b]);
        (void)hipGraphDestroy(s->graph[v][b]);
        s->exec[v][b] = NULL;
        s->graph[v][b] = NULL;
        s->graph_state[v][b] = 0;
    }
    if (s->graph_state[v][b] == 0 && getenv("MYNAH_HIP_NO_GRAPH") == NULL) {
        s->graph_state[v][b] = -1;
        if (hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal) == hipSuccess) {
            int rc = 0;
            for (uint32_t r = 0; r < launch_steps(v) && rc == 0; r++)
                rc = enqueue_step(s, d, st, v % STEP_MULTI, p0, cap);
            hipGraph_t g = NULL;
            const hipError_t e = hipStreamEndCapture(st, &g);
            if (rc == 0 && e == hipSuccess && g != NULL &&
                hipGraphInstantiate(&s->exec[v][b], g, NULL, NULL, 0) == hipSuccess) {
                s->graph[v][b] = g;
                s->graph_state[v][b] = 1;
                s->graph_order[v][b] = mynah_hip_gemv_order();
                s->graph_attn[v][b] = s->attn_mode;
            } else if (g != NULL) {
                (void)hipGraphDestroy(g);
            }
        }
        (void)hipGetLastError();
    }
    return b;
}

/* One launch of variant v starting at position p0: its bucket's graph, or
 * direct launches without one. */
static int run_step(mynah_qwen3 *s, mynah_device *d, int v, uint32_t p0) {
    hipStream_t st = d->stream;
    const uint32_t b = ensure_graph(s, d, v, p0);
    if (s->graph_state[v][b] == 1) {
        if (hipGraphLaunch(s->exec[v][b], st) != hipSuccess) {
            mynah_set_error("hipGraphLaunch failed");
            return -1;
        }
        return 0;
    }
    uint32_t cap = 0;
    (void)ctx_bucket(s, p0 + launch_steps(v), &cap);
    int rc = 0;
    for (uint32_t r = 0; r < launch_steps(v) && rc == 0; r++)
        rc = enqueue_step(s, d, st, v % STEP_MULTI, p0, cap);
    return rc;
}

/* n steps of variant v from position p0: batches of STEP_BATCH, then single
 * steps. */
static int run_steps(mynah_qwen3 *s, mynah_device *d, int v, uint32_t p0, uint32_t n) {
    int rc = 0;
    uint32_t i = 0;
    for (; i + STEP_BATCH <= n && rc == 0; i += STEP_BATCH)
        rc = run_step(s, d, STEP_MULTI + v, p0 + i);
    for (; i < n && rc == 0; i++) rc = run_step(s, d, v, p0 + i);
    return rc;
}

/* Capture every graph run_steps(v, p0, n) replays (a capture leaves the
 * device idle, so callers do it before their clock starts). */
static void prepare_steps(mynah_qwen3 *s, mynah_device *d, int v, uint32_t p0, uint32_t n) {
    uint32_t i = 0;
    for (; i + STEP_BATCH <= n; i += STEP_BATCH) (void)ensure_graph(s, d, STEP_MULTI + v, p0 + i);
    for (; i < n; i++) (void)ensure_graph(s, d, v, p0 + i);
}

static int set_counters(mynah_qwen3 *s, mynah_device *d, uint32_t token, uint32_t step,
                        uint32_t n_forced) {
    uint32_t v[4] = {token, s->n_past, step, n_forced};
    if (hipMemcpyAsync(s->counters, v, sizeof v, hipMemcpyHostToDevice, d->stream) != hipSuccess ||
        hipStreamSynchronize(d->stream) != hipSuccess) {
        mynah_set_error("counter upload failed");
        return -1;
    }
    return 0;
}

int mynah_hip_qwen3_forward(mynah_qwen3 *s, uint32_t token, float *logits) {
    mynah_device *d = mynah_dev();
    if (d == NULL || s == NULL) return -1;
    if (s->n_past >= s->n_ctx) {
        mynah_set_error("context exhausted");
        return -1;
    }
    if (token >= s->c.vocab) {
        mynah_set_error("token %u out of range", token);
        return -1;
    }
    if (set_counters(s, d, token, 0, 0) != 0 || embed_current(s, d) != 0 ||
        run_step(s, d, STEP_FULL, s->n_past) != 0)
        return -1;
    s->n_past++;
    if (logits && hipMemcpyAsync(logits, s->logits, (size_t)s->c.vocab * 4,
                                 hipMemcpyDeviceToHost, d->stream) != hipSuccess) {
        mynah_set_error("logits download failed");
        return -1;
    }
    if (hipStreamSynchronize(d->stream) != hipSuccess) {
        mynah_set_error("step failed");
        return -1;
    }
    return 0;
}

/* ── batched prompt prefill ──────────────────────────────────────────────── */

/* Tokens per prefill chunk: the GEMMs work in 64-token tiles (a chunk of
 * 2048 gives even the 1024-row projections 512 workgroups), the scores
 * buffer holds chunk x n_heads x sstride floats. */
static uint32_t prefill_chunk_cap(void) {
    const char *e = getenv("MYNAH_PREFILL_CHUNK");
    long v = e ? strtol(e, NULL, 10) : 2048;
    if (v < 1) v = 1;
    if (v > 4096) v = 4096;
    return (uint32_t)v;
}

/* The prefill's score rows ([token][head][sstride] floats) for one chunk
 * stay within 2 GiB: long contexts take shorter chunks. */
static uint32_t prefill_cap_for(const mynah_qwen3 *s, uint32_t want) {
    const size_t per_token = (size_t)s->c.n_heads * s->sstride * 4;
    const size_t most = ((size_t)2 << 30) / per_token;
    if (most < 1) return 1;
    return want < most ? want : (uint32_t)most;
}

static int prefill_alloc(mynah_qwen3 *s, uint32_t cap) {
    cap = prefill_cap_for(s, cap);
    if (s->pf_cap >= cap) return 0;
    void *bufs[] = {s->pf_x, s->pf_xn, s->pf_q, s->pf_att, s->pf_g, s->pf_u, s->pf_s, s->pf_tok};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++)
        if (bufs[i]) (void)hipFree(bufs[i]);
    const mynah_qwen3_shape *c = &s->c;
    int ok = 1;
    s->pf_x = (float *)dalloc((size_t)cap * c->d_model * 4, &ok);
    s->pf_xn = (float *)dalloc((size_t)cap * c->d_model * 4, &ok);
    s->pf_q = (float *)dalloc((size_t)cap * s->q_dim * 4, &ok);
    s->pf_att = (float *)dalloc((size_t)cap * s->q_dim * 4, &ok);
    s->pf_g = (float *)dalloc((size_t)cap * c->d_ff * 4, &ok);
    s->pf_u = (float *)dalloc((size_t)cap * c->d_ff * 4, &ok);
    s->pf_s = (float *)dalloc((size_t)cap * c->n_heads * s->sstride * 4, &ok);
    s->pf_tok = (uint32_t *)dalloc((size_t)cap * 4, &ok);
    if (!ok) {
        mynah_set_error("out of device memory for a %u-token prefill chunk", cap);
        s->pf_cap = 0;
        return -1;
    }
    s->pf_cap = cap;
    return 0;
}

/* The block size of the decode step's grouped launch whose fused RMSNorm
 * the prefill's row norm must reproduce (the q/k/v group when gate is NULL,
 * else the gate/up pair), always in the exact order. */
static int norm_threads(const mynah_qwen3 *s, const dlayer *L, int ffn, uint32_t *thr) {
    mynah_gemv_group g;
    memset(&g, 0, sizeof g);
    float *x = s->x;
    int rc;
    if (!ffn) {
        g.n = 3;
        rc = gemv_desc(&g.d[0], &L->wq, x, s->q);
        rc = rc ? rc : gemv_desc(&g.d[1], &L->wk, x, s->q);
        rc = rc ? rc : gemv_desc(&g.d[2], &L->wv, x, s->q);
        for (int k = 0; k < 3; k++) g.d[k].norm_w = (const float *)L->attn_norm.dev;
    } else {
        g.n = 1;
        rc = gemv_desc(&g.d[0], &L->gate, x, s->act);
        g.d[0].w2 = L->up.dev;
        g.d[0].norm_w = (const float *)L->ffn_norm.dev;
    }
    return rc ? rc : mynah_gemv_group_threads(&g, MYNAH_GEMV_EXACT, thr);
}

/* T tokens (already in pf_tok) at positions s->n_past .. + T - 1 through
 * every layer, filling the cache; no head. */
static int enqueue_prefill_chunk(mynah_qwen3 *s, mynah_device *d, hipStream_t st, uint32_t T) {
    const mynah_qwen3_shape *c = &s->c;
    const size_t per_layer = (size_t)s->n_ctx * s->kv_dim;
    uint32_t p0 = s->n_past, dm = c->d_model;
    const uint32_t group = c->n_heads / c->n_kv_heads;
    int rc;
    {
        const unsigned char *tab = s->embed.dev;
        const uint32_t *tk = s->pf_tok;
        float *x = s->pf_x;
        uint32_t ty = (uint32_t)s->embed.type, rb = (uint32_t)s->embed.row_bytes;
        void *args[] = {&tab, &tk, &x, &dm, &ty, &rb};
        rc = mynah_launch(d, MYNAH_K_EMBED_ROWS, (dm / 32 + 255) / 256, T, 256, 0, st, args);
    }
    for (uint32_t l = 0; l < c->n_layers && rc == 0; l++) {
        const dlayer *L = &s->layers[l];
        float *kl = s->k_cache + l * per_layer, *vl = s->v_cache + l * per_layer;
        uint32_t thr_attn = 0, thr_ffn = 0;
        rc = norm_threads(s, L, 0, &thr_attn);
        rc = rc ? rc : norm_threads(s, L, 1, &thr_ffn);
        if (rc) break;
        float eps = c->rms_eps;
        {   /* src/arch_qwen3.c:201 */
            const float *x = s->pf_x, *w = (const float *)L->attn_norm.dev;
            float *o = s->pf_xn;
            void *args[] = {&x, &w, &o, &dm, &eps};
            rc = mynah_launch(d, MYNAH_K_RMSNORM_ROWS, T, 1, thr_attn, 0, st, args);
        }
        /* src/arch_qwen3.c:194-199: q, and k / v straight into the cache. */
        rc = rc ? rc : mynah_matmat_mv_launch(d, L->wq.type, L->wq.dev, L->wq.rows, L->wq.cols,
                                              s->pf_xn, s->pf_q, T, NULL, st);
        rc = rc ? rc : mynah_matmat_mv_launch(d, L->wk.type, L->wk.dev, L->wk.rows, L->wk.cols,
                                              s->pf_xn, kl + (size_t)p0 * s->kv_dim, T, NULL, st);
        rc = rc ? rc : mynah_matmat_mv_launch(d, L->wv.type, L->wv.dev, L->wv.rows, L->wv.cols,
                                              s->pf_xn, vl + (size_t)p0 * s->kv_dim, T, NULL, st);
        if (rc) break;
        {   /* src/arch_qwen3.c:209-218 */
            float *q = s->pf_q;
            const float *qn = (const float *)L->q_norm.dev, *kn = (const float *)L->k_norm.dev;
            const float *rcos = s->rope_cos, *rsin = s->rope_sin;
            uint32_t nh = c->n_heads, kvd = s->kv_dim;
            void *args[] = {&q, &kl, &qn, &kn, &rcos, &rsin, &p0, &nh, &kvd, &eps};
            rc = mynah_launch(d, MYNAH_K_PREFILL_ROPE, T, c->n_heads + c->n_kv_heads, 64, 0, st,
                              args);
        }
        if (rc) break;
        {   /* src/kernels.c:228-293 (src/arch_qwen3.c:219-222) */
            const float *qn = s->pf_q;
            const float *kc = kl;
            float *sc = s->pf_s, scale = s->scale;
            uint32_t sstride = s->sstride, kvd = s->kv_dim, grp = group;
            uint32_t tt = T;
            void *args[] = {&qn, &kc, &sc, &p0, &tt, &sstride, &kvd, &grp, &scale};
            /* 256 positions by 16 queries per workgroup, the queries in LDS */
            rc = mynah_launch3(d, MYNAH_K_PREFILL_SCORES, c->n_kv_heads, (p0 + T + 255) / 256,
                               (T + 15) / 16, 256, (size_t)16 * group * 512, st, args);
            if (rc) break;
            uint32_t nh = c->n_heads;
            void *args2[] = {&sc, &p0, &sstride, &nh};
            rc = mynah_launch(d, MYNAH_K_PREFILL_SOFTMAX, T, (nh + 3) / 4, 256, 0, st, args2);
            if (rc) break;
            const float *vc = vl, *pr = s->pf_s;
            float *out = s->pf_att;
            void *args3[] = {&vc, &pr, &out, &p0, &tt, &sstride, &kvd, &grp};
            rc = mynah_launch(d, MYNAH_K_PREFILL_PV, c->n_kv_heads, (T + 7) / 8, 512, 0, st, args3);
        }
        if (rc) break;
        /* src/arch_qwen3.c:223-224: x += Wo attn */
        rc = mynah_matmat_mv_launch(d, L->wo.type, L->wo.dev, L->wo.rows, L->wo.cols, s->pf_att,
                                    s->pf_x, T, s->pf_x, st);
        if (rc) break;
        {   /* src/arch_qwen3.c:226 */
            const float *x = s->pf_x, *w = (const float *)L->ffn_norm.dev;
            float *o = s->pf_xn;
            void *args[] = {&x, &w, &o, &dm, &eps};
            rc = mynah_launch(d, MYNAH_K_RMSNORM_ROWS, T, 1, thr_ffn, 0, st, args);
        }
        /* src/arch_qwen3.c:227-233: gate, up, SwiGLU, down + residual */
        rc = rc ? rc : mynah_matmat_mv_launch(d, L->gate.type, L->gate.dev, L->gate.rows,
                                              L->gate.cols, s->pf_xn, s->pf_g, T, NULL, st);
        rc = rc ? rc : mynah_matmat_mv_launch(d, L->up.type, L->up.dev, L->up.rows, L->up.cols,
                                              s->pf_xn, s->pf_u, T, NULL, st);
        if (rc) break;
        {
            const float *g = s->pf_g, *u = s->pf_u;
            float *a = s->pf_g;
            uint32_t n = T * c->d_ff;
            void *args[] = {&g, &u, &a, &n};
            rc = mynah_launch(d, MYNAH_K_SWIGLU_ROWS, (n + 255) / 256, 1, 256, 0, st, args);
        }
        rc = rc ? rc : mynah_matmat_mv_launch(d, L->down.type, L->down.dev, L->down.rows,
                                              L->down.cols, s->pf_g, s->pf_x, T, s->pf_x, st);
    }
    return rc;
}

int mynah_hip_qwen3_prefill(mynah_qwen3 *s, const uint32_t *tokens, uint32_t n) {
    mynah_device *d = mynah_dev();
    if (d == NULL || s == NULL || (tokens == NULL && n > 0)) {
        mynah_set_error("bad prefill arguments");
        return -1;
    }
    if (n > s->n_ctx - s->n_past) {
        mynah_set_error("%u prefill tokens do not fit the context (%u of %u used)", n, s->n_past,
                        s->n_ctx);
        return -1;
    }
    for (uint32_t i = 0; i < n; i++)
        if (tokens[i] >= s->c.vocab) {
            mynah_set_error("token %u out of range", tokens[i]);
            return -1;
        }
    const uint32_t cap = prefill_chunk_cap();
    if (n > 0 && prefill_alloc(s, n < cap ? n : cap) != 0) return -1;
    hipStream_t st = d->stream;
    for (uint32_t done = 0; done < n;) {
        const uint32_t T = n - done < s->pf_cap ? n - done : s->pf_cap;
        if (hipMemcpyAsync(s->pf_tok, tokens + done, (size_t)T * 4, hipMemcpyHostToDevice, st) !=
            hipSuccess) {
            mynah_set_error("prefill token upload failed");
            return -1;
        }
        if (enqueue_prefill_chunk(s, d, st, T) != 0) return -1;
        s->n_past += T;
        done += T;
        /* the token buffer is reused by the next chunk */
        if (done < n && hipStreamSynchronize(st) != hipSuccess) {
            mynah_set_error("prefill failed");
            return -1;
        }
    }
    if (hipStreamSynchronize(st) != hipSuccess) {
        mynah_set_error("prefill failed");
        return -1;
    }
    return 0;
}

int mynah_hip_qwen3_set_prefill(mynah_qwen3 *s, int mode) {
    if (s == NULL || (mode != MYNAH_PREFILL_BATCHED && mode != MYNAH_PREFILL_STEPS)) {
        mynah_set_error("prefill mode %d", mode);
        return -1;
    }
    s->prefill_mode = mode;
    return 0;
}

/* src/generate.c:13-86 with the prompt's cache-filling tokens prefilled in
 * batches (bit-identical to filling them one decode step at a time), then
 * the greedy steps from the last prompt token. */
static int prompt_batched(mynah_qwen3 *s, mynah_device *d, const uint32_t *prompt,
                          uint32_t n_prompt, uint32_t n_steps, uint32_t *tokens_out,
                          float *prefill_ms, float *decode_ms) {
    const uint32_t cap = prefill_chunk_cap();
    if (prefill_alloc(s, n_prompt - 1u < cap ? n_prompt - 1u : cap) != 0) return -1;
    const uint32_t start = s->n_past;
    prepare_steps(s, d, STEP_FULL, start + (n_prompt - 1u), n_steps);
    hipEvent_t ev[4] = {NULL, NULL, NULL, NULL};
    for (int i = 0; i < 4; i++)
        if (hipEventCreate(&ev[i]) != hipSuccess) {
            mynah_set_error("hipEventCreate failed");
            for (int j = 0; j < i; j++) (void)hipEventDestroy(ev[j]);
            return -1;
        }
    (void)hipEventRecord(ev[0], d->stream);
    int rc = mynah_hip_qwen3_prefill(s, prompt, n_prompt - 1u);
    (void)hipEventRecord(ev[1], d->stream);
    if (rc == 0) rc = set_counters(s, d, prompt[n_prompt - 1u], 0, 0);
    (void)hipEventRecord(ev[2], d->stream);
    if (rc == 0) rc = embed_current(s, d);
    if (rc == 0) rc = run_steps(s, d, STEP_FULL, start + (n_prompt - 1u), n_steps);
    (void)hipEventRecord(ev[3], d->stream);
    if (rc == 0 && hipStreamSynchronize(d->stream) != hipSuccess) {
        mynah_set_error("decode failed");
        rc = -1;
    }
    if (rc == 0 && prefill_ms) (void)hipEventElapsedTime(prefill_ms, ev[0], ev[1]);
    if (rc == 0 && decode_ms) (void)hipEventElapsedTime(decode_ms, ev[2], ev[3]);
    for (int i = 0; i < 4; i++) (void)hipEventDestroy(ev[i]);
    if (rc != 0) return -1;
    s->n_past = start + (n_prompt - 1u) + n_steps;
    if (hipMemcpy(tokens_out, s->tokens, (size_t)n_steps * 4, hipMemcpyDeviceToHost) != hipSuccess) {
        mynah_set_error("token download failed");
        return -1;
    }
    return 0;
}

int mynah_hip_qwen3_prompt(mynah_qwen3 *s, const uint32_t *prompt, uint32_t n_prompt,
                           uint32_t n_steps, uint32_t *tokens_out, float *prefill_ms,
                           float *decode_ms) {
    mynah_device *d = mynah_dev();
    if (d == NULL || s == NULL || prompt == NULL || tokens_out == NULL || n_prompt == 0) {
        mynah_set_error("bad prompt arguments");
        return -1;
    }
    if (n_steps == 0 || n_prompt - 1u > s->n_ctx - s->n_past ||
        n_steps > s->n_ctx - s->n_past - (n_prompt - 1u)) {
        mynah_set_error("%u prompt tokens and %u steps do not fit the context (%u of %u used)",
                        n_prompt, n_steps, s->n_past, s->n_ctx);
        return -1;
    }
    for (uint32_t i = 0; i < n_prompt; i++)
        if (prompt[i] >= s->c.vocab) {
            mynah_set_error("token %u out of range", prompt[i]);
            return -1;
        }
    if (n_prompt > 1 && s->prefill_mode == MYNAH_PREFILL_BATCHED)
        return prompt_batched(s, d, prompt, n_prompt, n_steps, tokens_out, prefill_ms, decode_ms);
    if (n_prompt > 1 &&
        hipMemcpy(s->forced, prompt, (size_t)n_prompt * 4, hipMemcpyHostToDevice) != hipSuccess) {
        mynah_set_error("prompt upload failed");
        return -1;
    }
    if (set_counters(s, d, prompt[0], 0, n_prompt > 1 ? n_prompt : 0) != 0) return -1;
    hipEvent_t a = NULL, m = NULL, b = NULL;
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&m) != hipSuccess ||
        hipEventCreate(&b) != hipSuccess) {
        mynah_set_error("hipEventCreate failed");
        if (a) (void)hipEventDestroy(a);
        if (m) (void)hipEventDestroy(m);
        return -1;
    }
    /* Capture before the clock starts: a capture leaves the device idle. */
    const uint32_t p_first = s->n_past + (n_prompt - 1u);
    if (n_prompt > 1) prepare_steps(s, d, STEP_PREFILL, s->n_past, n_prompt - 1u);
    prepare_steps(s, d, STEP_FULL, p_first, n_steps);
    (void)hipEventRecord(a, d->stream);
    int rc = embed_current(s, d);
    /* src/generate.c:33-36: every prompt token but the last only fills the
     * cache; its logits are never produced. */
    if (rc == 0 && n_prompt > 1) rc = run_steps(s, d, STEP_PREFILL, s->n_past, n_prompt - 1u);
    (void)hipEventRecord(m, d->stream);
    if (rc == 0) rc = run_steps(s, d, STEP_FULL, p_first, n_steps);
    (void)hipEventRecord(b, d->stream);
    if (rc == 0 && hipStreamSynchronize(d->stream) != hipSuccess) {
        mynah_set_error("decode failed");
        rc = -1;
    }
    if (rc == 0 && prefill_ms) (void)hipEventElapsedTime(prefill_ms, a, m);
    if (rc == 0 && decode_ms) (void)hipEventElapsedTime(decode_ms, m, b);
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(m);
    (void)hipEventDestroy(b);
    if (rc != 0) return -1;
    s->n_past += n_prompt - 1u + n_steps;
    if (hipMemcpy(tokens_out, s->tokens + (n_prompt - 1u), (size_t)n_steps * 4,
                  hipMemcpyDeviceToHost) != hipSuccess) {
        mynah_set_error("token download failed");
        return -1;
    }
    return 0;
}

int mynah_hip_qwen3_generate(mynah_qwen3 *s, uint32_t first_token, uint32_t n_steps,
                             uint32_t *tokens_out, float *ms) {
    return mynah_hip_qwen3_prompt(s, &first_token, 1, n_steps, tokens_out, NULL, ms);
}

/* Teacher forcing through the same captured steps the greedy loop replays:
 * the forced-token list makes the argmax kernel embed inputs[i + 1] after
 * step i instead of its choice, and still record the choice. */
int mynah_hip_qwen3_forced(mynah_qwen3 *s, const uint32_t *inputs, uint32_t n,
                           uint32_t *greedy_out, float *last_logits) {
    mynah_device *d = mynah_dev();
    if (d == NULL || s == NULL || inputs == NULL || greedy_out == NULL || n == 0) {
        mynah_set_error("bad teacher-forcing arguments");
        return -1;
    }
    if (n > s->n_ctx - s->n_past) {
        mynah_set_error("%u forced steps do not fit the context (%u of %u used)", n, s->n_past,
                        s->n_ctx);
        return -1;
    }
    for (uint32_t i = 0; i < n; i++)
        if (inputs[i] >= s->c.vocab) {
            mynah_set_error("token %u out of range", inputs[i]);
            return -1;
        }
    if (hipMemcpy(s->forced, inputs, (size_t)n * 4, hipMemcpyHostToDevice) != hipSuccess) {
        mynah_set_error("forced-token upload failed");
        return -1;
    }
    if (set_counters(s, d, inputs[0], 0, n) != 0) return -1;
    prepare_steps(s, d, STEP_FULL, s->n_past, n);
    if (embed_current(s, d) != 0 || run_steps(s, d, STEP_FULL, s->n_past, n) != 0) return -1;
    if (hipStreamSynchronize(d->stream) != hipSuccess) {
        mynah_set_error("forced decode failed");
        return -1;
    }
    s->n_past += n;
    if (hipMemcpy(greedy_out, s->tokens, (size_t)n * 4, hipMemcpyDeviceToHost) != hipSuccess ||
        (last_logits && hipMemcpy(last_logits, s->logits, (size_t)s->c.vocab * 4,
                                  hipMemcpyDeviceToHost) != hipSuccess)) {
        mynah_set_error("forced decode download failed");
        return -1;
    }
    return 0;
}

/* ── the reference's sampler on the device (sample.hip) ──────────────────── */

struct mynah_hip_sampler {
    uint32_t vocab;
    SampState *st;                  /* device: what the kernels read and update */
    SampState h;                    /* host mirror */
    samp_scratch sc;                /* for mynah_hip_sample */
};

static uint32_t samp_nwg(uint32_t vocab) { return (vocab + SP_CH - 1u) / SP_CH; }
static uint32_t samp_nwg_tk(uint32_t vocab) { return (vocab + SP_TK_CH - 1u) / SP_TK_CH; }

static void samp_scratch_free(samp_scratch *sc) {
    void *b[] = {sc->e, sc->logits, sc->wkey, sc->cand, sc->key, sc->wsum};
    for (size_t i = 0; i < sizeof b / sizeof b[0]; i++)
        if (b[i]) (void)hipFree(b[i]);
    memset(sc, 0, sizeof *sc);
}

static int samp_scratch_alloc(samp_scratch *sc, uint32_t vocab, int with_logits) {
    if (sc->e != NULL && (!with_logits || sc->logits != NULL)) return 0;
    samp_scratch_free(sc);
    const uint32_t nwg = samp_nwg(vocab);
    int ok = 1;
    sc->nwg = nwg;
    sc->e = (float *)dalloc((size_t)vocab * 4, &ok);
    if (with_logits) sc->logits = (float *)dalloc((size_t)vocab * 4, &ok);
    sc->wkey = (unsigned long long *)dalloc((size_t)nwg * 8, &ok);
    sc->cand = (unsigned long long *)dalloc((size_t)SP_TK_MAXWG * SP_KMAX * 8, &ok);
    sc->key = (unsigned long long *)dalloc(8, &ok);
    sc->wsum = (double *)dalloc((size_t)nwg * 16, &ok);
    if (!ok) {
        samp_scratch_free(sc);
        mynah_set_error("out of device memory for the sampler");
        return -1;
    }
    return 0;
}

/* The four launches of one draw over `logits` (device), state `state`;
 * `accept`: the id also enters the window. */
static int samp_enqueue(mynah_device *d, hipStream_t st, SampState *state, const samp_scratch *sc,
                        float *logits, uint32_t vocab, uint32_t accept) {
    const float *clogits = logits, *ce = sc->e;
    const SampState *cstate = state;
    float *e = sc->e;
    unsigned long long *wkey = sc->wkey, *cand = sc->cand, *key = sc->key;
    const unsigned long long *cwkey = wkey, *ccand = cand;
    double *wsum = sc->wsum;
    const double *cwsum = wsum;
    uint32_t nwg = sc->nwg, nwg_tk = samp_nwg_tk(vocab);
    void *a1[] = {&logits, &vocab, &cstate, &wkey};
    void *a2[] = {&clogits, &vocab, &cstate, &cwkey, &nwg, &e, &wsum};
    void *a3[] = {&ce, &vocab, &cstate, &cwsum, &nwg, &cand};
    void *a4[] = {&state, &vocab, &cwkey, &ccand, &nwg, &nwg_tk, &key, &accept};
    int rc = mynah_launch(d, MYNAH_K_SAMP_PENALIZE, nwg, 1, SP_T, 0, st, a1);
    rc = rc ? rc : mynah_launch(d, MYNAH_K_SAMP_EXP, nwg, 1, SP_T, 0, st, a2);
    rc = rc ? rc : mynah_launch(d, MYNAH_K_SAMP_TOPK, nwg_tk, 1, SP_TK_T, 0, st, a3);
    rc = rc ? rc : mynah_launch(d, MYNAH_K_SAMP_PICK, 1, 1, 64, 0, st, a4);
    return rc;
}

/* What the device sampler takes (include/mynah_generate.h). */
static int samp_check(const mynah_hip_sampler_params *p, uint32_t vocab) {
    if (p == NULL || vocab == 0) {
        mynah_set_error("sampler: null parameters or empty vocabulary");
        return -1;
    }
    if (samp_nwg_tk(vocab) > SP_TK_MAXWG) {
        mynah_set_error("sampler: vocabulary of %u exceeds %u", vocab, SP_TK_MAXWG * SP_TK_CH);
        return -1;
    }
    if (p->penalty_window > SP_WMAX) {
        mynah_set_error("sampler: penalty window %u exceeds %u", p->penalty_window, SP_WMAX);
        return -1;
    }
    if (p->temp > 0.0f && (p->top_k == 0 || p->top_k > SP_KMAX || p->top_k >= vocab)) {
        mynah_set_error("sampler: with temp > 0 the device sampler takes 1 <= top_k <= %u "
                        "(below the vocabulary), not %u; sample on the host instead",
                        SP_KMAX, p->top_k);
        return -1;
    }
    return 0;
}

/* src/sampler.c:73-78. */
static void samp_push(SampState *h, uint32_t token) {
    if (h->window == 0) return;
    h->ring[h->head] = token;
    h->head = (h->head + 1u) % h->window;
    if (h->n_recent < h->window) h->n_recent++;
}

/* Bytes of the state that matter: everything before the window, and the
 * window's slots. */
static size_t samp_bytes(const SampState *h) {
    return offsetof(SampState, ring) + (size_t)h->window * sizeof(uint32_t);
}

mynah_hip_sampler *mynah_hip_sampler_new(const mynah_hip_sampler_params *p, uint32_t vocab) {
    mynah_device *d = mynah_dev();
    if (d == NULL || samp_check(p, vocab) != 0) return NULL;
    mynah_hip_sampler *s = (mynah_hip_sampler *)calloc(1, sizeof *s);
    if (s == NULL) {
        mynah_set_error("out of host memory");
        return NULL;
    }
    s->vocab = vocab;
    SampState *h = &s->h;
    h->temp = p->temp;
    h->top_k = p->top_k;
    h->top_p = p->top_p;
    h->min_p = p->min_p;
    h->repeat_penalty = p->repeat_penalty;
    h->freq_penalty = p->freq_penalty;
    h->presence_penalty = p->presence_penalty;
    h->window = p->penalty_window;
    h->seed = p->seed;
    h->rng = p->seed ? p->seed : 0x853C49E6748FEA9Bull;       /* src/sampler.c:55 */
    /* MYNAH_SAMPLE_SEQ_SUM=1: always the index-order double sum (tests). */
    h->flags = env_or("MYNAH_SAMPLE_SEQ_SUM", 0) != 0 ? SP_FLAG_SEQ_SUM : 0u;
    int ok = 1;
    s->st = (SampState *)dalloc(sizeof(SampState), &ok);
    if (!ok || hipMemcpy(s->st, h, samp_bytes(h), hipMemcpyHostToDevice) != hipSuccess) {
        mynah_set_error("sampler state upload failed");
        mynah_hip_sampler_free(s);
        return NULL;
    }
    return s;
}

void mynah_hip_sampler_free(mynah_hip_sampler *s) {
    if (s == NULL) return;
    samp_scratch_free(&s->sc);
    if (s->st) (void)hipFree(s->st);
    free(s);
}

/* The host mirror into the device state. */
static int samp_upload(mynah_hip_sampler *s) {
    if (hipMemcpy(s->st, &s->h, samp_bytes(&s->h), hipMemcpyHostToDevice) != hipSuccess) {
        mynah_set_error("sampler state upload failed");
        return -1;
    }
    return 0;
}

int mynah_hip_sampler_accept(mynah_hip_sampler *s, uint32_t token) {
    if (s == NULL) {
        mynah_set_error("null sampler");
        return -1;
    }
    samp_push(&s->h, token);
    return s->h.window ? samp_upload(s) : 0;
}

int mynah_hip_sample(mynah_hip_sampler *s, float *logits, uint32_t *id) {
    mynah_device *d = mynah_dev();
    if (d == NULL || s == NULL || logits == NULL || id == NULL) {
        mynah_set_error("bad sample arguments");
        return -1;
    }
    if (samp_scratch_alloc(&s->sc, s->vocab, 1) != 0) return -1;
    const size_t bytes = (size_t)s->vocab * 4;
    unsigned long long key = 0;
    if (hipMemcpyAsync(s->sc.logits, logits, bytes, hipMemcpyHostToDevice, d->stream) != hipSuccess ||
        samp_enqueue(d, d->stream, s->st, &s->sc, s->sc.logits, s->vocab, 0u) != 0 ||
        hipMemcpyAsync(logits, s->sc.logits, bytes, hipMemcpyDeviceToHost, d->stream) != hipSuccess ||
        hipMemcpyAsync(&key, s->sc.key, 8, hipMemcpyDeviceToHost, d->stream) != hipSuccess ||
        hipMemcpyAsync(&s->h, s->st, samp_bytes(&s->h), hipMemcpyDeviceToHost, d->stream) !=
            hipSuccess ||
        hipStreamSynchronize(d->stream) != hipSuccess) {
        mynah_set_error("device sampling failed");
        return -1;
    }
    *id = ~(uint32_t)(key & 0xffffffffull);
    return 0;
}

/* ── the generation loop (src/generate.c:13-86) ──────────────────────────── */

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + (double)ts.tv_nsec * 1e-9;
}

static int is_eos(const mynah_hip_gen_params *p, uint32_t id) {
    for (size_t i = 0; i < p->n_eos; i++)
        if (p->eos[i] == id) return 1;
    return 0;
}

/* src/timing.c:48-55: the first generated token stamps TTFT (prefill plus
 * the decode time so far), every token counts. */
static void timing_token(mynah_hip_timing *t, double t0) {
    if (!t->ttft_done) {
        t->ttft_s = t->prefill_s + (now_s() - t0);
        t->ttft_done = 1;
    }
    t->n_gen++;
}

/* What the loop does with one sampled id (src/generate.c:50-77): 1 to go on,
 * 0 to stop after it. The id counts as produced either way. */
static int take_token(const mynah_hip_gen_params *p, mynah_hip_timing *t, double t0,
                      uint32_t id, long *produced) {
    if (p->accept) p->accept(p->sampler, id);
    (*produced)++;
    timing_token(t, t0);
    if (is_eos(p, id)) return 0;
    if (p->on_token && p->on_token(p->token_ctx, id) != 0) return 0;
    return 1;
}

/* A failed call still leaves the caller's sampler with the ids it took. */
static long gen_fail(mynah_hip_sampler *sm) {
    if (sm != NULL) (void)samp_upload(sm);
    return -1;
}

long mynah_hip_qwen3_generate_tokens(mynah_qwen3 *s, const mynah_hip_gen_params *pp,
                                     mynah_hip_timing *t) {
    mynah_device *d = mynah_dev();
    mynah_hip_timing scratch_t;
    if (t == NULL) t = &scratch_t;
    memset(t, 0, sizeof *t);
    if (d == NULL || s == NULL || pp == NULL || pp->prompt == NULL || pp->n_prompt == 0 ||
        (pp->n_eos > 0 && pp->eos == NULL) || pp->n_prompt > 0xffffffffu) {
        mynah_set_error("bad generation arguments");
        return -1;
    }
    /* With the device sampler the host sampler's hooks are not used. */
    mynah_hip_gen_params q = *pp;
    mynah_hip_sampler *sm = q.device_sampler;
    if (sm != NULL) {
        q.sample = NULL;
        q.accept = NULL;
        if (sm->vocab != s->c.vocab) {
            mynah_set_error("sampler vocabulary %u, model %u", sm->vocab, s->c.vocab);
            return -1;
        }
    }
    const mynah_hip_gen_params *p = &q;
    for (size_t i = 0; i < p->n_prompt; i++)
        if (p->prompt[i] >= s->c.vocab) {
            mynah_set_error("token %u out of range", p->prompt[i]);
            return -1;
        }
    const uint32_t n_prompt = (uint32_t)p->n_prompt;
    double t0 = now_s();
    /* src/generate.c:26-33: every prompt token but the last only fills the
     * cache (batched here; the same bits as one step per token). */
    if (n_prompt > 1) {
        if (s->prefill_mode == MYNAH_PREFILL_BATCHED) {
            if (mynah_hip_qwen3_prefill(s, p->prompt, n_prompt - 1u) != 0) return -1;
        } else {
            for (uint32_t i = 0; i + 1 < n_prompt; i++)
                if (mynah_hip_qwen3_forward(s, p->prompt[i], NULL) != 0) return -1;
        }
    }
    if (p->accept)
        for (uint32_t i = 0; i + 1 < n_prompt; i++) p->accept(p->sampler, p->prompt[i]);
    if (sm != NULL)
        for (uint32_t i = 0; i + 1 < n_prompt; i++) samp_push(&sm->h, p->prompt[i]);
    {   /* src/timing.c:30-35 */
        const double now = now_s();
        t->prefill_s = now - t0;
        t->n_prompt = n_prompt;
        t0 = now;
    }
    uint32_t next = p->prompt[n_prompt - 1u];
    if (p->accept) p->accept(p->sampler, next);
    if (sm != NULL) samp_push(&sm->h, next);
    long produced = 0;
    if (p->sample != NULL) {
        /* Host sampling: every step's logits come back to the host and the
         * caller's sampler (the reference's mynah_slm_sample, say) picks. */
        if (s->host_logits == NULL &&
            hipHostMalloc((void **)&s->host_logits, (size_t)s->c.vocab * 4, 0) != hipSuccess) {
            s->host_logits = NULL;
            mynah_set_error("cannot allocate the host logits buffer");
            return -1;
        }
        for (uint32_t step = 0; step < p->max_new; step++) {
            /* src/generate.c:48: a full context ends the loop, not the call. */
            if (s->n_past >= s->n_ctx) break;
            if (mynah_hip_qwen3_forward(s, next, s->host_logits) != 0) return -1;
            const uint32_t id = p->sample(p->sampler, s->host_logits);
            if (!take_token(p, t, t0, id, &produced)) break;
            next = id;
        }
    } else {
        /* Greedy, or the device sampler, on the device: up to `chunk` steps
         * replay as graphs per host round trip (the first step alone, so
         * TTFT is one step), then the ids come back and run through the
         * loop's checks in order. A stop inside a chunk rewinds the position
         * to just after the stopping step: the cache slots past it are
         * rewritten before any later step reads them. The sampler's device
         * copy may run ahead of the stop; the caller's sampler is brought to
         * exactly the ids taken, below. Greedy without penalties is the
         * reference's sampler at temp <= 0 and takes the plain greedy steps. */
        int variant = STEP_FULL;
        if (sm != NULL) {
            const SampState *h = &sm->h;
            if (h->temp > 0.0f || h->repeat_penalty != 1.0f || h->freq_penalty != 0.0f ||
                h->presence_penalty != 0.0f) {
                int ok = 1;
                if (s->samp_st == NULL) s->samp_st = (SampState *)dalloc(sizeof(SampState), &ok);
                if (!ok || samp_scratch_alloc(&s->samp_sc, s->c.vocab, 0) != 0 ||
                    hipMemcpy(s->samp_st, h, samp_bytes(h), hipMemcpyHostToDevice) != hipSuccess) {
                    mynah_set_error("device sampler set-up failed");
                    return gen_fail(sm);
                }
                variant = STEP_SAMPLE;
            }
        }
        const uint32_t chunk = p->chunk ? p->chunk : STEP_BATCH;
        uint32_t done = 0;
        int go = 1;
        while (go && done < p->max_new && s->n_past < s->n_ctx) {
            uint32_t c = done == 0 ? 1u : chunk;
            if (c > p->max_new - done) c = p->max_new - done;
            if (c > s->n_ctx - s->n_past) c = s->n_ctx - s->n_past;
            if (set_counters(s, d, next, 0, 0) != 0) return gen_fail(sm);
            prepare_steps(s, d, variant, s->n_past, c);
            if (embed_current(s, d) != 0 || run_steps(s, d, variant, s->n_past, c) != 0)
                return gen_fail(sm);
            uint32_t ids[64];
            uint32_t *buf = c <= 64u ? ids : (uint32_t *)malloc((size_t)c * 4);
            if (buf == NULL ||
                hipMemcpyAsync(buf, s->tokens, (size_t)c * 4, hipMemcpyDeviceToHost, d->stream) !=
                    hipSuccess ||
                hipStreamSynchronize(d->stream) != hipSuccess) {
                if (buf != ids) free(buf);
                mynah_set_error("greedy decode failed");
                return gen_fail(sm);
            }
            uint32_t used = 0;
            while (used < c && go) {
                const uint32_t id = buf[used++];
                go = take_token(p, t, t0, id, &produced);
                next = id;
                if (sm != NULL) {
                    /* src/generate.c:51-52: the id entered the window and,
                     * at temp > 0, took one splitmix64 draw. */
                    samp_push(&sm->h, id);
                    if (sm->h.temp > 0.0f) sm->h.rng += 0x9E3779B97F4A7C15ull;
                }
            }
            if (buf != ids) free(buf);
            s->n_past += used;
            done += used;
        }
    }
    if (sm != NULL && samp_upload(sm) != 0) return -1;
    t->decode_s = now_s() - t0;        /* src/timing.c:57-59 */
    return produced;
}

int mynah_hip_qwen3_set_kv(mynah_qwen3 *s, const float *k, const float *v, uint32_t n_pos) {
    mynah_device *d = mynah_dev();
    if (d == NULL || s == NULL || k == NULL || v == NULL || n_pos > s->n_ctx) {
        mynah_set_error("bad KV prefill");
        return -1;
    }
    const size_t row = (size_t)n_pos * s->kv_dim, per_layer = (size_t)s->n_ctx * s->kv_dim;
    for (uint32_t l = 0; l < s->c.n_layers; l++) {
        if (hipMemcpy(s->k_cache + l * per_layer, k + l * row, row * 4, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(s->v_cache + l * per_layer, v + l * row, row * 4, hipMemcpyHostToDevice) != hipSuccess) {
            mynah_set_error("KV upload failed");
            return -1;
        }
    }
    s->n_past = n_pos;
    return 0;
}

int mynah_hip_qwen3_get_kv(const mynah_qwen3 *s, float *k, float *v, uint32_t n_pos) {
    mynah_device *d = mynah_dev();
    if (d == NULL || s == NULL || k == NULL || v == NULL || n_pos > s->n_ctx) {
        mynah_set_error("bad KV download");
        return -1;
    }
    if (hipStreamSynchronize(d->stream) != hipSuccess) {
        mynah_set_error("stream failed");
        return -1;
    }
    const size_t row = (size_t)n_pos * s->kv_dim, per_layer = (size_t)s->n_ctx * s->kv_dim;
    for (uint32_t l = 0; l < s->c.n_layers; l++) {
        if (hipMemcpy(k + l * row, s->k_cache + l * per_layer, row * 4, hipMemcpyDeviceToHost) != hipSuccess ||
            hipMemcpy(v + l * row, s->v_cache + l * per_layer, row * 4, hipMemcpyDeviceToHost) != hipSuccess) {
            mynah_set_error("KV download failed");
            return -1;
        }
    }
    return 0;
}

uint32_t mynah_hip_qwen3_n_past(const mynah_qwen3 *s) { return s ? s->n_past : 0; }

int mynah_hip_qwen3_read_attn(const mynah_qwen3 *s, float *out) {
    if (s == NULL || out == NULL) {
        mynah_set_error("null argument");
        return -1;
    }
    mynah_device *d = mynah_dev();
    if (d == NULL) return -1;
    if (hipStreamSynchronize(d->stream) != hipSuccess ||
        hipMemcpy(out, s->attn, (size_t)s->q_dim * 4, hipMemcpyDeviceToHost) != hipSuccess) {
        mynah_set_error("attention output download failed");
        return -1;
    }
    return 0;
}

void mynah_hip_qwen3_reset(mynah_qwen3 *s) {
    if (s) s->n_past = 0;
}

int mynah_hip_qwen3_uses_graph(const mynah_qwen3 *s) {
    if (s == NULL) return 0;
    for (uint32_t b = 0; b < N_BUCKETS; b++)
        if (s->graph_state[STEP_FULL][b] == 1 || s->graph_state[STEP_MULTI + STEP_FULL][b] == 1)
            return 1;
    return 0;
}

int mynah_hip_qwen3_set_attention(mynah_qwen3 *s, int mode) {
    if (s == NULL || (mode != MYNAH_ATTN_EXACT && mode != MYNAH_ATTN_SPLIT)) {
        mynah_set_error("attention mode %d", mode);
        return -1;
    }
    /* The combine keeps one weight per chunk in LDS (64 KiB: 16,384 chunks). */
    if (mode == MYNAH_ATTN_SPLIT && (size_t)s->nch_max * sizeof(float) > 64u * 1024u) {
        mynah_set_error("split attention holds at most %u positions (n_ctx %u)",
                        16384u * s->as_ch, s->n_ctx);
        return -1;
    }
    s->attn_mode = mode;
    return 0;
}
