/* gguf_shim.c — TEST INFRASTRUCTURE ONLY: a stand-in for the host process's
 * GGUF reader, so the tests can drive libmynah_hip.so's ingot_gguf_matvec /
 * _matmat / _dequant_matrix, which find a tensor's bytes through the
 * process's ingot_gguf_data(). Loaded RTLD_GLOBAL before libmynah_hip.so.
 *
 * The contract is the reference reader's (third_party/ingot/src/gguf.c:
 * 601-608): NULL for a NULL handle or tensor or a shard out of range, NULL
 * when offset + nbytes overflows or leaves the mapping, else mapping base +
 * data base + offset. The handle here is a plain {base, size, data_base}
 * triple for one shard; the tensor is ingot_tensor's layout
 * (third_party/ingot/include/ingot/gguf.h:41-50).
 *
 * SPDX-License-Identifier: MIT */
#include <stddef.h>
#include <stdint.h>

typedef struct {
    const unsigned char *base;
    uint64_t size, data_base;
} shim_gguf;

typedef struct {
    const char *name;
    int type;
    uint32_t rank;
    uint64_t ne[8];
    uint64_t nelem, nbytes, offset;
    uint32_t shard;
} shim_tensor;

const void *ingot_gguf_data(const void *g, const void *t) {
    const shim_gguf *h = (const shim_gguf *)g;
    const shim_tensor *x = (const shim_tensor *)t;
    if (h == NULL || x == NULL || x->shard != 0) return NULL;
    const uint64_t abs = h->data_base + x->offset;
    if (abs < x->offset || abs + x->nbytes < abs || abs + x->nbytes > h->size) return NULL;
    return h->base + abs;
}
