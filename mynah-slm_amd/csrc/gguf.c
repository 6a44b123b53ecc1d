/* gguf.c — GGUF checkpoints for the resident decoder (C11 host code).
 *
 * Reads the GGUF v2 / v3 container (the format third_party/ingot/src/gguf.c
 * reads for the reference): a little-endian header ("GGUF", version, tensor
 * count, metadata count), the metadata entries (key string, value type,
 * value; strings are a u64 length and bytes, arrays an element type, a u64
 * count and the elements), the tensor infos (name, rank, ne[0..rank), ggml
 * type, offset), then the data section at the next multiple of
 * general.alignment (default 32). Every length, count and offset is checked
 * against the mapping before use; a malformed file is refused with a
 * message, never read past.
 *
 * The config and tensor binding follow src/model.c:71-228 (see
 * include/mynah_gguf.h); the data section goes unchanged to
 * mynah_hip_qwen3_new.
 *
 * SPDX-License-Identifier: MIT */
#define _GNU_SOURCE
#include "mynah_gguf.h"
#include "runtime_internal.h"

#include <ctype.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#define GG_MAGIC 0x46554747u           /* "GGUF" little-endian */
#define GG_MAX_STRING (16u << 20)
#define GG_MAX_COUNT (1u << 28)
#define GG_MAX_DIMS 8              /* ingot's INGOT_MAX_RANK */

enum {
    KV_U8 = 0, KV_I8 = 1, KV_U16 = 2, KV_I16 = 3, KV_U32 = 4, KV_I32 = 5, KV_F32 = 6,
    KV_BOOL = 7, KV_STRING = 8, KV_ARRAY = 9, KV_U64 = 10, KV_I64 = 11, KV_F64 = 12
};

typedef struct {
    const char *key;
    uint64_t klen;
    uint32_t type;
    const unsigned char *val;   /* scalar payload, string length field, or array elements */
    uint32_t arr_type;
    uint64_t arr_len;
} gg_kv;

typedef struct {
    const char *name;
    uint64_t nlen;
    uint32_t rank, type, shard;
    uint64_t ne[GG_MAX_DIMS];
    uint64_t offset, nbytes;        /* offset within its shard's data section */
} gg_tensor;

/* One mapped file of a checkpoint; `concat` is where its data section sits
 * in the concatenation of all shards' data sections (mynah_gguf_shard_data). */
typedef struct {
    unsigned char *map;
    size_t size;
    uint32_t version;
    uint64_t alignment;
    const unsigned char *data;
    uint64_t data_bytes, concat;
} gg_shard;

struct mynah_gguf {
    gg_shard *sh;
    uint32_t n_sh;
    uint64_t n_kv, n_tensors, concat_bytes;
    gg_kv *kv;                      /* the first shard's metadata */
    gg_tensor *t;                   /* every shard's tensors, in shard order */
};

static void gg_err(char *err, size_t errsz, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (err && errsz) snprintf(err, errsz, "%s", buf);
    mynah_set_error("%s", buf);
}

/* ── bounds-checked cursor ──────────────────────────────────────────────── */

typedef struct {
    const unsigned char *p, *end;
} gg_cur;

static uint32_t ld_u32(const unsigned char *p) {
    return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}
static uint64_t ld_u64(const unsigned char *p) {
    return (uint64_t)ld_u32(p) | (uint64_t)ld_u32(p + 4) << 32;
}

static int rd_bytes(gg_cur *c, uint64_t n, const unsigned char **out) {
    if ((uint64_t)(c->end - c->p) < n) return -1;
    *out = c->p;
    c->p += n;
    return 0;
}
static int rd_le32(gg_cur *c, uint32_t *v) {
    const unsigned char *p;
    if (rd_bytes(c, 4, &p)) return -1;
    *v = ld_u32(p);
    return 0;
}
static int rd_le64(gg_cur *c, uint64_t *v) {
    const unsigned char *p;
    if (rd_bytes(c, 8, &p)) return -1;
    *v = ld_u64(p);
    return 0;
}
static int rd_string(gg_cur *c, const char **s, uint64_t *len) {
    const unsigned char *p;
    if (rd_le64(c, len) || *len > GG_MAX_STRING || rd_bytes(c, *len, &p)) return -1;
    *s = (const char *)p;
    return 0;
}

static int scalar_bytes(uint32_t type, uint64_t *n) {
    switch (type) {
    case KV_U8: case KV_I8: case KV_BOOL: *n = 1; return 0;
    case KV_U16: case KV_I16: *n = 2; return 0;
    case KV_U32: case KV_I32: case KV_F32: *n = 4; return 0;
    case KV_U64: case KV_I64: case KV_F64: *n = 8; return 0;
    default: return -1;
    }
}

/* Block geometry (values, bytes) of every ggml type id the reference's
 * reader knows (third_party/ingot/src/dtype.c:37-83): a file is accepted or
 * refused on exactly this table, so it is the same list, Q8_1 at 40 bytes
 * included. */
static int type_geometry(uint32_t type, uint64_t *elems, uint64_t *bytes) {
    static const struct { uint32_t type, elems, bytes; } tab[] = {
        {0, 1, 4},      /* F32 */     {1, 1, 2},       /* F16 */
        {30, 1, 2},     /* BF16 */    {28, 1, 8},      /* F64 */
        {24, 1, 1},     /* I8 */      {25, 1, 2},      /* I16 */
        {26, 1, 4},     /* I32 */     {27, 1, 8},      /* I64 */
        {2, 32, 18},    /* Q4_0 */    {3, 32, 20},     /* Q4_1 */
        {6, 32, 22},    /* Q5_0 */    {7, 32, 24},     /* Q5_1 */
        {8, 32, 34},    /* Q8_0 */    {9, 32, 40},     /* Q8_1 */
        {20, 32, 18},   /* IQ4_NL */
        {10, 256, 84},  /* Q2_K */    {11, 256, 110},  /* Q3_K */
        {12, 256, 144}, /* Q4_K */    {13, 256, 176},  /* Q5_K */
        {14, 256, 210}, /* Q6_K */    {15, 256, 292},  /* Q8_K */
        {16, 256, 66},  /* IQ2_XXS */ {17, 256, 74},   /* IQ2_XS */
        {22, 256, 82},  /* IQ2_S */   {18, 256, 98},   /* IQ3_XXS */
        {21, 256, 110}, /* IQ3_S */   {19, 256, 50},   /* IQ1_S */
        {29, 256, 56},  /* IQ1_M */   {23, 256, 136},  /* IQ4_XS */
        {34, 256, 54},  /* TQ1_0 */   {35, 256, 66},   /* TQ2_0 */
        {39, 32, 17},   /* MXFP4 */   {40, 64, 36},    /* NVFP4 */
        {41, 128, 18},  /* Q1_0 */
    };
    for (size_t i = 0; i < sizeof tab / sizeof tab[0]; i++)
        if (tab[i].type == type) {
            *elems = tab[i].elems;
            *bytes = tab[i].bytes;
            return 0;
        }
    return -1;
}

/* ── parsing ────────────────────────────────────────────────────────────── */

static int read_entry(gg_cur *c, gg_kv *kv, uint64_t index, char *err, size_t errsz) {
    if (rd_string(c, &kv->key, &kv->klen) || rd_le32(c, &kv->type)) {
        gg_err(err, errsz, "metadata entry %llu is cut short by the end of the file", (unsigned long long)index);
        return -1;
    }
    const int kl = (int)(kv->klen < 200 ? kv->klen : 200);
    uint64_t n;
    if (kv->type == KV_STRING) {
        const char *s;
        uint64_t len;
        kv->val = c->p;
        if (rd_string(c, &s, &len)) {
            gg_err(err, errsz, "string of key '%.*s' is cut short", kl, kv->key);
            return -1;
        }
        return 0;
    }
    if (kv->type == KV_ARRAY) {
        if (rd_le32(c, &kv->arr_type) || rd_le64(c, &kv->arr_len) || kv->arr_len > GG_MAX_COUNT) {
            gg_err(err, errsz, "key '%.*s': bad array element type or length", kl, kv->key);
            return -1;
        }
        kv->val = c->p;
        if (kv->arr_type == KV_ARRAY) {
            gg_err(err, errsz, "key '%.*s' holds an array of arrays, which GGUF readers refuse", kl, kv->key);
            return -1;
        }
        if (kv->arr_type == KV_STRING) {
            for (uint64_t i = 0; i < kv->arr_len; i++) {
                const char *s;
                uint64_t len;
                if (rd_string(c, &s, &len)) {
                    gg_err(err, errsz, "key '%.*s': string element %llu is cut short", kl, kv->key,
                           (unsigned long long)i);
                    return -1;
                }
            }
            return 0;
        }
        const unsigned char *p;
        if (scalar_bytes(kv->arr_type, &n)) {
            gg_err(err, errsz, "key '%.*s': array element type %u is unknown", kl, kv->key, kv->arr_type);
            return -1;
        }
        if (rd_bytes(c, n * kv->arr_len, &p)) {
            gg_err(err, errsz, "key '%.*s': array data ends past the file", kl, kv->key);
            return -1;
        }
        return 0;
    }
    if (scalar_bytes(kv->type, &n)) {
        gg_err(err, errsz, "key '%.*s': value type %u is unknown", kl, kv->key, kv->type);
        return -1;
    }
    if (rd_bytes(c, n, &kv->val)) {
        gg_err(err, errsz, "key '%.*s': value is cut short", kl, kv->key);
        return -1;
    }
    return 0;
}

/* Names compare as C strings (ingot keeps NUL-terminated copies, so a name
 * ends at its first NUL byte); the first entry of a repeated name wins. */
static int name_is(const char *s, uint64_t len, const char *want, size_t n) {
    return strnlen(s, (size_t)len) == n && memcmp(s, want, n) == 0;
}

static const gg_kv *find_kv(const mynah_gguf *g, const char *key) {
    const size_t n = strlen(key);
    for (uint64_t i = 0; i < g->n_kv; i++)
        if (name_is(g->kv[i].key, g->kv[i].klen, key, n)) return &g->kv[i];
    return NULL;
}

static const gg_tensor *find_tensor(const mynah_gguf *g, const char *name) {
    const size_t n = strlen(name);
    for (uint64_t i = 0; i < g->n_tensors; i++)
        if (name_is(g->t[i].name, g->t[i].nlen, name, n)) return &g->t[i];
    return NULL;
}

/* One decoder for every scalar width, like ingot's (gguf.c kv_read_scalar). */
static int read_scalar(uint32_t type, const unsigned char *p, uint64_t *u, double *f) {
    int64_t i;
    switch (type) {
    case KV_U8: *u = p[0]; *f = (double)p[0]; return 0;
    case KV_BOOL: *u = p[0] ? 1u : 0u; *f = (double)*u; return 0;
    case KV_I8: i = (int8_t)p[0]; break;
    case KV_U16: *u = (uint64_t)p[0] | (uint64_t)p[1] << 8; *f = (double)*u; return 0;
    case KV_I16: i = (int16_t)(uint16_t)((uint32_t)p[0] | (uint32_t)p[1] << 8); break;
    case KV_U32: *u = ld_u32(p); *f = (double)*u; return 0;
    case KV_I32: i = (int32_t)ld_u32(p); break;
    case KV_U64: *u = ld_u64(p); *f = (double)*u; return 0;
    case KV_I64: i = (int64_t)ld_u64(p); break;
    case KV_F32: {
        float v;
        const uint32_t b = ld_u32(p);
        memcpy(&v, &b, 4);
        *f = (double)v;
        *u = !(v > 0.0f) ? 0u : v >= 18446744073709551616.0f ? UINT64_MAX : (uint64_t)v;
        return 0;
    }
    case KV_F64: {
        double v;
        const uint64_t b = ld_u64(p);
        memcpy(&v, &b, 8);
        *f = v;
        *u = !(v > 0.0) ? 0u : v >= 18446744073709551616.0 ? UINT64_MAX : (uint64_t)v;
        return 0;
    }
    default: return -1;
    }
    *u = (uint64_t)i;
    *f = (double)i;
    return 0;
}

void mynah_gguf_close(mynah_gguf *g) {
    if (g == NULL) return;
    for (uint32_t i = 0; i < g->n_sh; i++)
        if (g->sh[i].map) munmap(g->sh[i].map, g->sh[i].size);
    free(g->sh);
    free(g->kv);
    free(g->t);
    free(g);
}

/* The last general.alignment among kv[0 .. n) that reads as a number, else
 * `dflt` (ingot's header scan). */
static uint64_t alignment_of(const gg_kv *kv, uint64_t n, uint64_t dflt) {
    uint64_t a = dflt;
    for (uint64_t i = 0; i < n; i++) {
        uint64_t v;
        double f;
        if (name_is(kv[i].key, kv[i].klen, "general.alignment", 17) &&
            read_scalar(kv[i].type, kv[i].val, &v, &f) == 0)
            a = v;
    }
    return a;
}

/* Map `path` as shard `index` of g and parse it: header, metadata (kept for
 * the first shard; a later shard's is read with the same checks and only its
 * general.alignment used, a missing or zero one meaning 32, as ingot's
 * shard_parse does), tensor infos appended to g's table, data section. */
static int parse_shard(mynah_gguf *g, uint32_t index, const char *path, char *err,
                       size_t errsz) {
    gg_shard *sh = &g->sh[index];
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        gg_err(err, errsz, "cannot open '%s'", path);
        return -1;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        close(fd);
        gg_err(err, errsz, "'%s' is shorter than a GGUF header", path);
        return -1;
    }
    sh->size = (size_t)st.st_size;
    void *m = mmap(NULL, sh->size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) {
        gg_err(err, errsz, "cannot map '%s'", path);
        return -1;
    }
    sh->map = (unsigned char *)m;
    g->n_sh = index + 1;
    gg_cur c = {sh->map, sh->map + sh->size};
    uint32_t magic;
    uint64_t n_tensors, n_kv;
    if (rd_le32(&c, &magic) || magic != GG_MAGIC) {
        gg_err(err, errsz, "'%s' does not start with the GGUF magic", path);
        return -1;
    }
    if (rd_le32(&c, &sh->version) || sh->version < 2 || sh->version > 3) {
        gg_err(err, errsz, "'%s': GGUF version %u (this reader takes 2 and 3)", path, sh->version);
        return -1;
    }
    /* A metadata entry takes at least 13 bytes and a tensor info 24, so the
     * counts are bounded by the file before anything is allocated for them. */
    if (rd_le64(&c, &n_tensors) || rd_le64(&c, &n_kv) || n_tensors > GG_MAX_COUNT ||
        n_kv > GG_MAX_COUNT || n_kv * 13 + n_tensors * 24 > sh->size - 24) {
        gg_err(err, errsz, "'%s': the header counts more entries than the file can hold", path);
        return -1;
    }
    gg_kv *kv = (gg_kv *)calloc(n_kv ? n_kv : 1, sizeof *kv);
    gg_tensor *grown = (gg_tensor *)realloc(g->t, (size_t)(g->n_tensors + n_tensors + 1) *
                                                      sizeof *g->t);
    if (kv == NULL || grown == NULL) {
        free(kv);
        if (grown) g->t = grown;
        gg_err(err, errsz, "out of memory");
        return -1;
    }
    g->t = grown;
    for (uint64_t i = 0; i < n_kv; i++)
        if (read_entry(&c, &kv[i], i, err, errsz)) {
            free(kv);
            return -1;
        }
    sh->alignment = alignment_of(kv, n_kv, 32);
    if (index == 0) {
        g->kv = kv;
        g->n_kv = n_kv;
    } else {
        free(kv);
        if (sh->alignment == 0) sh->alignment = 32;
    }
    /* Checked here rather than where ingot checks it (when the data section
     * is placed); a file is refused either way. */
    if (sh->alignment == 0 || sh->alignment > (1u << 20) ||
        (sh->alignment & (sh->alignment - 1))) {
        gg_err(err, errsz, "'%s': general.alignment %llu is not a power of two up to 1 MiB",
               path, (unsigned long long)sh->alignment);
        return -1;
    }
    const uint64_t base = g->n_tensors;
    for (uint64_t i = 0; i < n_tensors; i++) {
        gg_tensor *t = &g->t[base + i];
        memset(t, 0, sizeof *t);
        t->shard = index;
        if (rd_string(&c, &t->name, &t->nlen) || rd_le32(&c, &t->rank)) {
            gg_err(err, errsz, "tensor entry %llu is cut short by the end of the file", (unsigned long long)i);
            return -1;
        }
        const int nl = (int)(t->nlen < 200 ? t->nlen : 200);
        if (t->rank > GG_MAX_DIMS) {
            gg_err(err, errsz, "tensor '%.*s': rank %u is above %d", nl, t->name, t->rank,
                   GG_MAX_DIMS);
            return -1;
        }
        uint64_t nelem = 1;
        for (uint32_t d = 0; d < t->rank; d++) {
            if (rd_le64(&c, &t->ne[d]) || t->ne[d] == 0 || nelem > UINT64_MAX / t->ne[d]) {
                gg_err(err, errsz, "tensor '%.*s': a zero or overflowing dimension", nl, t->name);
                return -1;
            }
            nelem *= t->ne[d];
        }
        for (uint32_t d = t->rank; d < GG_MAX_DIMS; d++) t->ne[d] = 1;
        if (rd_le32(&c, &t->type) || rd_le64(&c, &t->offset)) {
            gg_err(err, errsz, "tensor '%.*s': its entry is cut short", nl, t->name);
            return -1;
        }
        uint64_t be, bb;
        if (type_geometry(t->type, &be, &bb)) {
            gg_err(err, errsz, "tensor '%.*s': ggml type %u is unknown", nl, t->name, t->type);
            return -1;
        }
        /* Quantized blocks lie along ne[0] and may not straddle rows. */
        if ((be > 1 && (t->rank == 0 || t->ne[0] % be != 0)) || (nelem / be) > UINT64_MAX / bb) {
            gg_err(err, errsz, "tensor '%.*s': %llu values is not whole blocks of type %u", nl,
                   t->name, (unsigned long long)t->ne[0], t->type);
            return -1;
        }
        t->nbytes = nelem / be * bb;
        if (t->offset % sh->alignment != 0) {
            gg_err(err, errsz, "tensor '%.*s': data offset %llu is off the %llu-byte alignment", nl, t->name,
                   (unsigned long long)t->offset, (unsigned long long)sh->alignment);
            return -1;
        }
        g->n_tensors = base + i + 1;
    }
    const uint64_t head = (uint64_t)(c.p - sh->map);
    const uint64_t data_off = (head + sh->alignment - 1) & ~(sh->alignment - 1);
    if (data_off > sh->size) {
        gg_err(err, errsz, "'%s': the data section starts past the end of the file", path);
        return -1;
    }
    sh->data = sh->map + data_off;
    sh->data_bytes = sh->size - data_off;
    for (uint64_t i = base; i < g->n_tensors; i++) {
        const gg_tensor *t = &g->t[i];
        if (t->offset > sh->data_bytes || t->nbytes > sh->data_bytes - t->offset) {
            gg_err(err, errsz, "tensor '%.*s': data ends past the end of '%s'",
                   (int)(t->nlen < 200 ? t->nlen : 200), t->name, path);
            return -1;
        }
    }
    return 0;
}

/* 1 (with the message) when two tensors share a name, compared as C strings
 * (up to a first NUL); an open-addressing hash of the names, so a table of
 * millions of entries costs linear time. */
static int dup_name(const mynah_gguf *g, char *err, size_t errsz) {
    if (g->n_tensors < 2) return 0;
    uint64_t cap = 16;
    while (cap < 2 * g->n_tensors) cap *= 2;
    uint64_t *slot = (uint64_t *)calloc((size_t)cap, sizeof *slot);   /* index + 1 */
    if (slot == NULL) {
        gg_err(err, errsz, "out of memory");
        return 1;
    }
    int dup = 0;
    for (uint64_t i = 0; i < g->n_tensors && !dup; i++) {
        const gg_tensor *t = &g->t[i];
        const size_t tl = strnlen(t->name, (size_t)t->nlen);
        uint64_t h = 0xcbf29ce484222325ull;
        for (size_t k = 0; k < tl; k++) h = (h ^ (unsigned char)t->name[k]) * 0x100000001b3ull;
        for (uint64_t p = h & (cap - 1);; p = (p + 1) & (cap - 1)) {
            if (slot[p] == 0) {
                slot[p] = i + 1;
                break;
            }
            const gg_tensor *o = &g->t[slot[p] - 1];
            if (strnlen(o->name, (size_t)o->nlen) == tl && memcmp(o->name, t->name, tl) == 0) {
                gg_err(err, errsz, "tensor '%.*s' appears more than once",
                       (int)(tl < 200 ? tl : 200), t->name);
                dup = 1;
                break;
            }
        }
    }
    free(slot);
    return dup;
}

/* Open the `n` files of one checkpoint as shards 0 .. n - 1. A tensor name
 * present twice (in one file or across shards) makes every lookup
 * ambiguous, and the reference's reader refuses it; so does this one. */
static mynah_gguf *open_paths(char *const *paths, uint32_t n, char *err, size_t errsz) {
    mynah_gguf *g = (mynah_gguf *)calloc(1, sizeof *g);
    if (g == NULL || (g->sh = (gg_shard *)calloc(n, sizeof *g->sh)) == NULL) {
        free(g);
        gg_err(err, errsz, "out of memory");
        return NULL;
    }
    for (uint32_t i = 0; i < n; i++)
        if (parse_shard(g, i, paths[i], err, errsz)) goto fail;
    if (dup_name(g, err, errsz)) goto fail;
    /* The shards' data sections laid end to end, each from a multiple of 256
     * bytes and of its own alignment. */
    uint64_t at = 0;
    for (uint32_t i = 0; i < n; i++) {
        const uint64_t a = g->sh[i].alignment > 256 ? g->sh[i].alignment : 256;
        at = (at + a - 1) & ~(a - 1);
        g->sh[i].concat = at;
        at += g->sh[i].data_bytes;
    }
    g->concat_bytes = at;
    return g;
fail:
    mynah_gguf_close(g);
    return NULL;
}

mynah_gguf *mynah_gguf_open(const char *path, char *err, size_t errsz) {
    if (path == NULL) {
        gg_err(err, errsz, "null path");
        return NULL;
    }
    char *one = (char *)path;
    return open_paths(&one, 1, err, errsz);
}

/* Shard names end in "-NNNNN-of-MMMMM.gguf": shard NNNNN of MMMMM, both
 * zero-padded five-digit decimals, shards counted from 1, at most 999 of them
 * (llama.cpp's gguf-split naming, which third_party/ingot/src/gguf.c:466-509
 * accepts). A name that is not of this form, or names one shard of one, is a
 * plain single file. Returns the shard count and the prefix length, else 0. */
static int five_digits(const char *s, unsigned *v) {
    unsigned x = 0;
    for (int i = 0; i < 5; i++) {
        if (!isdigit((unsigned char)s[i])) return 0;
        x = 10u * x + (unsigned)(s[i] - '0');
    }
    *v = x;
    return 1;
}

static uint32_t split_name(const char *path, size_t *prefix) {
    static const char of[] = "-of-", ext[] = ".gguf";
    enum { OF = sizeof of - 1, EXT = sizeof ext - 1, TAIL = 1 + 5 + OF + 5 + EXT };
    const size_t len = strlen(path);
    if (len < TAIL) return 0;
    const char *p = path + len - TAIL;        /* '-' NNNNN "-of-" MMMMM ".gguf" */
    unsigned shard, count;
    if (*p != '-' || !five_digits(p + 1, &shard) || memcmp(p + 6, of, OF) != 0 ||
        !five_digits(p + 6 + OF, &count) || memcmp(p + 11 + OF, ext, EXT) != 0)
        return 0;
    if (count < 2 || count > 999 || shard < 1 || shard > count) return 0;
    *prefix = len - TAIL;
    return count;
}

mynah_gguf *mynah_gguf_open_split(const char *path, char *err, size_t errsz) {
    if (path == NULL) {
        gg_err(err, errsz, "null path");
        return NULL;
    }
    size_t prefix = 0;
    const uint32_t n = split_name(path, &prefix);
    if (n == 0) return mynah_gguf_open(path, err, errsz);
    char **paths = (char **)calloc(n, sizeof *paths);
    const size_t plen = strlen(path) + 1;     /* every shard name is as long */
    mynah_gguf *g = NULL;
    if (paths == NULL) goto oom;
    for (uint32_t i = 0; i < n; i++) {
        if ((paths[i] = (char *)malloc(plen)) == NULL) goto oom;
        memcpy(paths[i], path, prefix);
        snprintf(paths[i] + prefix, plen - prefix, "-%05u-of-%05u.gguf", i + 1, n);
    }
    g = open_paths(paths, n, err, errsz);
    goto done;
oom:
    gg_err(err, errsz, "out of memory");
done:
    if (paths)
        for (uint32_t i = 0; i < n; i++) free(paths[i]);
    free(paths);
    return g;
}

/* ── queries ────────────────────────────────────────────────────────────── */

uint32_t mynah_gguf_version(const mynah_gguf *g) { return g ? g->sh[0].version : 0; }
uint64_t mynah_gguf_alignment(const mynah_gguf *g) { return g ? g->sh[0].alignment : 0; }
uint32_t mynah_gguf_n_shards(const mynah_gguf *g) { return g ? g->n_sh : 0; }
uint64_t mynah_gguf_n_kv(const mynah_gguf *g) { return g ? g->n_kv : 0; }
uint64_t mynah_gguf_n_tensors(const mynah_gguf *g) { return g ? g->n_tensors : 0; }

int mynah_gguf_kv_u64(const mynah_gguf *g, const char *key, uint64_t *out) {
    const gg_kv *kv = g && key && out ? find_kv(g, key) : NULL;
    double f;
    return kv ? read_scalar(kv->type, kv->val, out, &f) : -1;
}

int mynah_gguf_kv_f64(const mynah_gguf *g, const char *key, double *out) {
    const gg_kv *kv = g && key && out ? find_kv(g, key) : NULL;
    uint64_t u;
    return kv ? read_scalar(kv->type, kv->val, &u, out) : -1;
}

int mynah_gguf_kv_str(const mynah_gguf *g, const char *key, const char **out, size_t *len) {
    const gg_kv *kv = g && key && out && len ? find_kv(g, key) : NULL;
    if (kv == NULL || kv->type != KV_STRING) return -1;
    *len = (size_t)ld_u64(kv->val);
    *out = (const char *)(kv->val + 8);
    return 0;
}

int mynah_gguf_kv_arr_len(const mynah_gguf *g, const char *key, uint64_t *out) {
    const gg_kv *kv = g && key && out ? find_kv(g, key) : NULL;
    if (kv == NULL || kv->type != KV_ARRAY) return -1;
    *out = kv->arr_len;
    return 0;
}

static int req_u32(const mynah_gguf *g, const char *arch, size_t alen, const char *suffix,
                   uint32_t *out, char *err, size_t errsz) {
    char key[160];
    snprintf(key, sizeof key, "%.*s.%s", (int)alen, arch, suffix);
    uint64_t v;
    if (find_kv(g, key) == NULL) {
        gg_err(err, errsz, "missing metadata key: %s", key);
        return -1;
    }
    if (mynah_gguf_kv_u64(g, key, &v)) {
        gg_err(err, errsz, "key %s does not hold an integer", key);
        return -1;
    }
    *out = (uint32_t)v;                  /* truncated, as src/model.c:50 does */
    return 0;
}

static int req_f32(const mynah_gguf *g, const char *arch, size_t alen, const char *suffix,
                   float *out, char *err, size_t errsz) {
    char key[160];
    snprintf(key, sizeof key, "%.*s.%s", (int)alen, arch, suffix);
    double v;
    if (find_kv(g, key) == NULL) {
        gg_err(err, errsz, "missing metadata key: %s", key);
        return -1;
    }
    if (mynah_gguf_kv_f64(g, key, &v)) {
        gg_err(err, errsz, "key %s does not hold a number", key);
        return -1;
    }
    *out = (float)v;
    return 0;
}

int mynah_gguf_qwen3_shape(const mynah_gguf *g, mynah_qwen3_shape *out, uint32_t *n_ctx_train,
                           char *err, size_t errsz) {
    if (g == NULL || out == NULL) {
        gg_err(err, errsz, "null argument");
        return -1;
    }
    const char *arch;
    size_t alen;
    if (mynah_gguf_kv_str(g, "general.architecture", &arch, &alen) || alen == 0) {
        gg_err(err, errsz, "general.architecture is missing or not a string");
        return -1;
    }
    if (alen >= 32) {                    /* mynah_slm_config.arch[32] */
        gg_err(err, errsz, "architecture name longer than 31 bytes: %.*s", (int)(alen < 200 ? alen : 200),
               arch);
        return -1;
    }
    mynah_qwen3_shape s;
    memset(&s, 0, sizeof s);
    uint32_t n_ctx = 0;
    if (req_u32(g, arch, alen, "block_count", &s.n_layers, err, errsz) ||
        req_u32(g, arch, alen, "embedding_length", &s.d_model, err, errsz) ||
        req_u32(g, arch, alen, "feed_forward_length", &s.d_ff, err, errsz) ||
        req_u32(g, arch, alen, "attention.head_count", &s.n_heads, err, errsz) ||
        req_u32(g, arch, alen, "attention.head_count_kv", &s.n_kv_heads, err, errsz) ||
        req_u32(g, arch, alen, "attention.key_length", &s.head_dim, err, errsz) ||
        req_u32(g, arch, alen, "context_length", &n_ctx, err, errsz) ||
        req_f32(g, arch, alen, "attention.layer_norm_rms_epsilon", &s.rms_eps, err, errsz) ||
        req_f32(g, arch, alen, "rope.freq_base", &s.rope_theta, err, errsz))
        return -1;
    if (s.n_heads == 0 || s.n_kv_heads == 0) {
        gg_err(err, errsz, "a head count is zero");
        return -1;
    }
    if (s.n_heads % s.n_kv_heads != 0) {
        gg_err(err, errsz, "n_heads (%u) is not a multiple of n_kv_heads (%u)", s.n_heads,
               s.n_kv_heads);
        return -1;
    }
    {
        /* Checked only when it reads as an integer (src/model.c:106-111). */
        char key[160];
        snprintf(key, sizeof key, "%.*s.attention.value_length", (int)alen, arch);
        uint64_t v;
        if (mynah_gguf_kv_u64(g, key, &v) == 0 && (uint32_t)v != s.head_dim) {
            gg_err(err, errsz, "value_length (%u) != key_length (%u), unsupported", (uint32_t)v,
                   s.head_dim);
            return -1;
        }
    }
    /* The vocabulary is the embedding's row count, else the tokenizer's
     * length (src/model.c:113-118, 209-222). */
    const gg_tensor *e = find_tensor(g, "token_embd.weight");
    if (e == NULL) {
        gg_err(err, errsz, "missing tensor: token_embd.weight");
        return -1;
    }
    uint64_t n_tok = 0;
    (void)mynah_gguf_kv_arr_len(g, "tokenizer.ggml.tokens", &n_tok);
    s.vocab = (uint32_t)(e->rank >= 2 ? e->ne[1] : n_tok);
    *out = s;
    if (n_ctx_train) *n_ctx_train = n_ctx;
    return 0;
}

int mynah_gguf_tensor_table(const mynah_gguf *g, mynah_synth_tensor *table, size_t cap,
                            size_t *count) {
    if (g == NULL || count == NULL) return -1;
    size_t n = 0;
    for (uint64_t i = 0; i < g->n_tensors; i++) {
        const gg_tensor *t = &g->t[i];
        if (t->nlen >= sizeof table[0].name) continue;
        if (table != NULL && n < cap) {
            mynah_synth_tensor *d = &table[n];
            memset(d, 0, sizeof *d);
            memcpy(d->name, t->name, (size_t)t->nlen);
            d->type = (int)t->type;
            d->rank = t->rank;
            d->cols = t->ne[0];
            d->rows = 1;
            for (uint32_t k = 1; k < GG_MAX_DIMS; k++) d->rows *= t->ne[k];
            d->offset = g->sh[t->shard].concat + t->offset;
            d->nbytes = t->nbytes;
        }
        n++;
    }
    *count = n;
    return 0;
}

const void *mynah_gguf_data(const mynah_gguf *g, uint64_t *bytes) {
    if (g == NULL || g->n_sh != 1) return NULL;
    if (bytes) *bytes = g->sh[0].data_bytes;
    return g->sh[0].data;
}

const void *mynah_gguf_shard_data(const mynah_gguf *g, uint32_t shard, uint64_t *bytes,
                                  uint64_t *concat) {
    if (g == NULL || shard >= g->n_sh) return NULL;
    if (bytes) *bytes = g->sh[shard].data_bytes;
    if (concat) *concat = g->sh[shard].concat;
    return g->sh[shard].data;
}

int mynah_gguf_tensor_place(const mynah_gguf *g, uint64_t index, uint32_t *shard,
                            uint64_t *offset) {
    if (g == NULL || index >= g->n_tensors) return -1;
    if (shard) *shard = g->t[index].shard;
    if (offset) *offset = g->t[index].offset;
    return 0;
}

mynah_qwen3 *mynah_hip_qwen3_from_gguf(const char *path, uint32_t n_ctx, char *err, size_t errsz) {
    /* src/model.c:183 opens every checkpoint through the split-aware open. */
    mynah_gguf *g = mynah_gguf_open_split(path, err, errsz);
    if (g == NULL) return NULL;
    mynah_qwen3_shape shape;
    uint32_t n_train = 0;
    mynah_qwen3 *s = NULL;
    if (mynah_gguf_qwen3_shape(g, &shape, &n_train, err, errsz) == 0) {
        size_t count = 0;
        mynah_gguf_tensor_table(g, NULL, 0, &count);
        mynah_synth_tensor *table = (mynah_synth_tensor *)calloc(count ? count : 1, sizeof *table);
        const void **parts = (const void **)calloc(g->n_sh, sizeof *parts);
        uint64_t *bytes = (uint64_t *)calloc(g->n_sh, sizeof *bytes);
        uint64_t *at = (uint64_t *)calloc(g->n_sh, sizeof *at);
        if (table == NULL || parts == NULL || bytes == NULL || at == NULL) {
            gg_err(err, errsz, "out of memory");
        } else {
            mynah_gguf_tensor_table(g, table, count, &count);
            for (uint32_t i = 0; i < g->n_sh; i++)
                parts[i] = mynah_gguf_shard_data(g, i, &bytes[i], &at[i]);
            /* The state's context as src/arch_qwen3.c:94 sets it: 0 or more
             * than the file's context_length takes context_length (a zero
             * context_length leaves no position, which the decoder refuses
             * like any empty context). */
            if (n_ctx == 0 || n_ctx > n_train) n_ctx = n_train;
            s = mynah_qwen3_new_parts(&shape, table, count, parts, bytes, at, g->n_sh,
                                      g->concat_bytes, n_ctx, err, errsz);
        }
        free(table);
        free(parts);
        free(bytes);
        free(at);
    }
    mynah_gguf_close(g);
    return s;
}
