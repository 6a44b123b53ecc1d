/* mynah_gguf.h — real checkpoints: a GGUF file's Qwen3 config and tensor
 * table, and the resident decoder built from them.
 *
 * The reference opens a checkpoint with ingot's GGUF reader and binds its
 * tensors in src/model.c:71-228 (mynah_slm_load): the config comes from the
 * "<arch>.*" metadata keys, the tensors by their GGUF names, the head is tied
 * to token_embd when output.weight is absent, and the vocabulary is the
 * embedding's row count. This header is that path for the GPU decoder: the
 * file is memory-mapped, parsed (GGUF v2 / v3, bounds-checked), and its data
 * section is handed unchanged to mynah_hip_qwen3_new, which uploads it to HBM
 * once — the tensors are read in place, never repacked.
 *
 * SPDX-License-Identifier: MIT */
#ifndef MYNAH_GGUF_H
#define MYNAH_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "mynah_decode.h"
#include "mynah_synth.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mynah_gguf mynah_gguf;

/* Map and parse `path` (third_party/ingot/src/gguf.c's reader, v2 / v3;
 * gguf.h ingot_gguf_open): header, metadata (every value type, arrays of
 * scalars and strings; strings up to 16 MiB, counts up to 2^28), tensor
 * infos (up to 8 non-zero dimensions, quantized rows made of whole blocks,
 * offsets aligned to general.alignment, default 32, data inside the file,
 * no tensor name twice). NULL on any malformed input, with the reason in
 * err. */
mynah_gguf *mynah_gguf_open(const char *path, char *err, size_t errsz);
/* gguf.h:62-66 (ingot_gguf_open_split): `path` may be any shard of a split
 * checkpoint named <prefix>-00001-of-000NN.gguf (llama.cpp's convention, 2
 * to 999 shards): every shard is opened and checked, the metadata is the
 * first shard's (a later shard's is read with the same checks, only its
 * general.alignment applies to it, 32 when missing or 0), and the tensor
 * tables are merged in shard order; a name in two shards is refused. Any
 * other path opens as mynah_gguf_open does. */
mynah_gguf *mynah_gguf_open_split(const char *path, char *err, size_t errsz);
void mynah_gguf_close(mynah_gguf *g);

/* Shards of the handle (1 unless opened from a split checkpoint); shard i's
 * data section, its size and where it sits in the concatenation of every
 * shard's data section (each from a multiple of 256 bytes and of its
 * alignment; the offsets mynah_gguf_tensor_table reports are into that
 * concatenation); tensor i's shard and offset within that shard's data
 * section (gguf.h:41-50 ingot_tensor.shard / .offset). */
uint32_t mynah_gguf_n_shards(const mynah_gguf *g);
const void *mynah_gguf_shard_data(const mynah_gguf *g, uint32_t shard, uint64_t *bytes,
                                  uint64_t *concat);
int mynah_gguf_tensor_place(const mynah_gguf *g, uint64_t index, uint32_t *shard,
                            uint64_t *offset);

/* GGUF version, the numbers of metadata entries and tensors, and the data
 * alignment in force, of the first shard (gguf.h ingot_gguf_version /
 * _kv_count / _count / _alignment; the tensor count is the merged table's). */
uint32_t mynah_gguf_version(const mynah_gguf *g);
uint64_t mynah_gguf_alignment(const mynah_gguf *g);
uint64_t mynah_gguf_n_kv(const mynah_gguf *g);
uint64_t mynah_gguf_n_tensors(const mynah_gguf *g);

/* Scalar metadata by key (src/model.c:39-69 kv_u32 / kv_f32): any integer,
 * float or bool scalar converts (saturating); 0, or -1 when the key is
 * absent or not a scalar. mynah_gguf_kv_str: a string value (not
 * NUL-terminated) and its length. mynah_gguf_kv_arr_len: an array's length. */
int mynah_gguf_kv_u64(const mynah_gguf *g, const char *key, uint64_t *out);
int mynah_gguf_kv_f64(const mynah_gguf *g, const char *key, double *out);
int mynah_gguf_kv_str(const mynah_gguf *g, const char *key, const char **out, size_t *len);
int mynah_gguf_kv_arr_len(const mynah_gguf *g, const char *key, uint64_t *out);

/* The architecture config the way mynah-slm reads it (src/model.c:71-130):
 * general.architecture gives the key prefix; block_count, embedding_length,
 * feed_forward_length, attention.head_count, attention.head_count_kv,
 * attention.key_length, context_length, attention.layer_norm_rms_epsilon and
 * rope.freq_base are required; attention.value_length, when present, must
 * equal key_length; the vocabulary is token_embd's row count. *n_ctx_train
 * (optional) gets context_length. 0, or -1 with the missing key in err. */
int mynah_gguf_qwen3_shape(const mynah_gguf *g, mynah_qwen3_shape *out, uint32_t *n_ctx_train,
                           char *err, size_t errsz);

/* Tensor descriptors (name, ggml type, rank, cols = ne[0], rows = the
 * product of ne[1..] (1 for rank 1), offset within the data section (of a
 * split checkpoint: within the concatenation above), bytes):
 * up to `cap` written, *count gets the number of tensors whose names fit the
 * descriptor (< 48 bytes, the others are skipped). */
int mynah_gguf_tensor_table(const mynah_gguf *g, mynah_synth_tensor *table, size_t cap,
                            size_t *count);

/* The data section: base address in the mapping and its size (NULL for a
 * split checkpoint: see mynah_gguf_shard_data). */
const void *mynah_gguf_data(const mynah_gguf *g, uint64_t *bytes);

/* mynah_slm_load + mynah_slm_state_init (src/model.c:177-228,
 * src/arch_qwen3.c:89-131) for the GPU: open `path` (split-aware, as
 * src/model.c:183 opens it), read the config and
 * tensors, build the resident decoder for n_ctx positions (0 or above the
 * file's context_length: context_length, as src/arch_qwen3.c:94 sets it; the
 * KV cache takes n_layers * n_ctx * kv_dim * 8 bytes of HBM, 12 GB for a 4B
 * model at 40960), unmap. NULL with the reason in err. */
mynah_qwen3 *mynah_hip_qwen3_from_gguf(const char *path, uint32_t n_ctx, char *err, size_t errsz);

#ifdef __cplusplus
}
#endif
#endif
