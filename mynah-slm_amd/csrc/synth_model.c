/* synth_model.c — layout and contents of a random-init Qwen3 in the Q4_K_M
 * type mix (see include/mynah_synth.h).
 *
 * SPDX-License-Identifier: MIT */
#include "mynah_synth.h"

#include <stdio.h>
#include <string.h>

int mynah_synth_q4_k_m_bumped(uint32_t i, uint32_t n) {
    const uint32_t a = n / 8, b = 7 * n / 8;
    return i < a || i >= b || (i >= a && (i - a) % 3 == 2);
}

static uint64_t type_bytes(int type, uint64_t rows, uint64_t cols) {
    switch (type) {
    case 0:  return rows * cols * 4;
    case 12: return rows * (cols / 256) * 144;
    case 14: return rows * (cols / 256) * 210;
    case 8:  return rows * (cols / 32) * 34;
    default: return 0;
    }
}

typedef struct {
    mynah_synth_tensor *table;
    size_t cap, n;
    uint64_t off;
} builder;

static void add(builder *b, const char *name, int type, uint32_t rank,
                uint64_t rows, uint64_t cols) {
    if (b->n < b->cap) {
        mynah_synth_tensor *t = &b->table[b->n];
        memset(t, 0, sizeof *t);
        snprintf(t->name, sizeof t->name, "%s", name);
        t->type = type;
        t->rank = rank;
        t->rows = rows;
        t->cols = cols;
        t->offset = b->off;
        t->nbytes = type_bytes(type, rows, cols);
    }
    b->off += (type_bytes(type, rows, cols) + 255u) & ~(uint64_t)255u;
    b->n++;
}

int mynah_synth_qwen3_layout(const mynah_qwen3_shape *s, mynah_synth_tensor *table,
                             size_t cap, size_t *count, uint64_t *total) {
    if (s == NULL || count == NULL || total == NULL || s->n_layers == 0 ||
        s->d_model % 256 || s->d_ff % 256 || s->n_kv_heads == 0 ||
        s->n_heads % s->n_kv_heads || (s->n_heads * s->head_dim) % 256 || s->vocab == 0)
        return -1;
    builder b = { table, table ? cap : 0, 0, 0 };
    const uint64_t d = s->d_model, q = (uint64_t)s->n_heads * s->head_dim;
    const uint64_t kv = (uint64_t)s->n_kv_heads * s->head_dim, ff = s->d_ff;
    char name[48];
    add(&b, "token_embd.weight", 14, 2, s->vocab, d);
    for (uint32_t l = 0; l < s->n_layers; l++) {
        const int bumped = mynah_synth_q4_k_m_bumped(l, s->n_layers);
#define NAME(suffix) (snprintf(name, sizeof name, "blk.%u." suffix, l), name)
        add(&b, NAME("attn_norm.weight"), 0, 1, 1, d);
        add(&b, NAME("attn_q.weight"), 12, 2, q, d);
        add(&b, NAME("attn_k.weight"), 12, 2, kv, d);
        add(&b, NAME("attn_v.weight"), bumped ? 14 : 12, 2, kv, d);
        add(&b, NAME("attn_q_norm.weight"), 0, 1, 1, s->head_dim);
        add(&b, NAME("attn_k_norm.weight"), 0, 1, 1, s->head_dim);
        add(&b, NAME("attn_output.weight"), 12, 2, d, q);
        add(&b, NAME("ffn_norm.weight"), 0, 1, 1, d);
        add(&b, NAME("ffn_gate.weight"), 12, 2, ff, d);
        add(&b, NAME("ffn_up.weight"), 12, 2, ff, d);
        add(&b, NAME("ffn_down.weight"), bumped ? 14 : 12, 2, d, ff);
#undef NAME
    }
    add(&b, "output_norm.weight", 0, 1, 1, d);
    *count = b.n;
    *total = b.off;
    return (table != NULL && cap < b.n) ? -1 : 0;
}

int mynah_synth_qwen3_fill(const mynah_qwen3_shape *s, uint64_t seed,
                           const mynah_synth_tensor *table, size_t count,
                           void *blob, int threads) {
    if (s == NULL || table == NULL || blob == NULL) return -1;
    unsigned char *base = (unsigned char *)blob;
    for (size_t i = 0; i < count; i++) {
        const mynah_synth_tensor *t = &table[i];
        const uint64_t ts = mynah_synth_substream(seed, i);
        int rc;
        if (t->type == 0)
            rc = mynah_synth_normal(ts, (size_t)(t->rows * t->cols), 1.0f, 0.02f,
                                    (float *)(base + t->offset), threads);
        else
            rc = mynah_synth_blocks(t->type, ts, 0, (size_t)t->rows, (size_t)t->cols,
                                    base + t->offset, threads);
        if (rc != 0) return -1;
    }
    return 0;
}
