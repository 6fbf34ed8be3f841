/*
 * mq_gguf.h -- GGUF v3 model files for the runners in libmq.so: a reader and the loaders that
 * build an encoder (mq_bert.h) or decoder embedder (mq_decoder.h) from a CrispEmbed GGUF.
 *
 * Reader.  Stands in for the gguf_* API that CrispEmbed's loaders call through
 * src/core/gguf_loader.h:54-137 (open_metadata, kv_u32 / kv_i32 / kv_f32 / kv_bool / kv_str and
 * the array readers) and for the tensor map load_weights builds (src/core/gguf_loader.h:140-200).
 * The file is memory-mapped read-only; every length, count and offset is checked against the
 * file size before use, so a truncated or malformed file fails mq_gguf_open with MQ_EINVAL and
 * a message (mq_last_error), never a crash.  Versions 2 and 3 (same layout, little-endian) are
 * accepted.  Tensor data pointers point into the mapping and stay valid until mq_gguf_close.
 *
 * Typed scalar readers return `def` when the key is absent or holds a type the reader does not
 * convert, with the conversions of core_gguf's readers (src/core/gguf_loader.cpp:72-137):
 * get_u32 accepts any integer type (truncating), get_i32 the 32/64-bit integer types, get_f32
 * FLOAT32 and FLOAT64, get_bool BOOL, get_str STRING.
 *
 * Loaders.  mq_bert_load reads CrispEmbed's BERT hyper-parameter keys with their fallbacks
 * (bert.*, xlmr.*, <arch>.*; src/crispembed.cpp:437-470) and tensors enc.N.* or blk.N.*
 * (src/crispembed.cpp:748-845); mq_decoder_load reads decoder.* then <arch>.* keys
 * (src/decoder_embed.cpp:96-175) and tensors dec.N.* or blk.N.* (src/decoder_embed.cpp:253-315).
 * Variants the runners do not implement (pre-LN or RoPE encoders, gated or MoE FFNs, CLS or
 * last-token pooling on the encoder, biased or Gemma-style decoders, RoPE scaling, dense
 * output heads, F32 or mixed-type linear weights) fail with MQ_EUNSUPPORTED and a message
 * naming the feature.  Embedding tables in F32, F16, Q8_0, Q4_K or Q6_K are dequantized on the
 * host, as ggml's get_rows does.
 */
#ifndef MQ_GGUF_H
#define MQ_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "mq_bert.h"
#include "mq_decoder.h"

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF metadata value types (the file format's ids) */
#define MQ_GGUF_UINT8 0
#define MQ_GGUF_INT8 1
#define MQ_GGUF_UINT16 2
#define MQ_GGUF_INT16 3
#define MQ_GGUF_UINT32 4
#define MQ_GGUF_INT32 5
#define MQ_GGUF_FLOAT32 6
#define MQ_GGUF_BOOL 7
#define MQ_GGUF_STRING 8
#define MQ_GGUF_ARRAY 9
#define MQ_GGUF_UINT64 10
#define MQ_GGUF_INT64 11
#define MQ_GGUF_FLOAT64 12

typedef struct mq_gguf mq_gguf;

mq_gguf *mq_gguf_open(const char *path);
void mq_gguf_close(mq_gguf *g);

uint32_t mq_gguf_version(const mq_gguf *g);
size_t mq_gguf_alignment(const mq_gguf *g);   /* general.alignment, default 32 */
size_t mq_gguf_data_offset(const mq_gguf *g); /* file offset of the tensor data section */

int64_t mq_gguf_n_kv(const mq_gguf *g);
int64_t mq_gguf_find_key(const mq_gguf *g, const char *key); /* -1 when absent */
const char *mq_gguf_kv_key(const mq_gguf *g, int64_t i);
int mq_gguf_kv_type(const mq_gguf *g, int64_t i); /* MQ_GGUF_*, -1 for a bad index */
int mq_gguf_arr_type(const mq_gguf *g, int64_t i);
int64_t mq_gguf_arr_n(const mq_gguf *g, int64_t i);
const void *mq_gguf_arr_data(const mq_gguf *g, int64_t i); /* numeric arrays (NULL for strings) */
const void *mq_gguf_kv_data(const mq_gguf *g, int64_t i);  /* a numeric or BOOL scalar's bytes (little-endian) */
const char *mq_gguf_arr_str(const mq_gguf *g, int64_t i, int64_t j); /* NUL-terminated, owned by g */

uint32_t mq_gguf_get_u32(const mq_gguf *g, const char *key, uint32_t def);
int32_t mq_gguf_get_i32(const mq_gguf *g, const char *key, int32_t def);
float mq_gguf_get_f32(const mq_gguf *g, const char *key, float def);
int mq_gguf_get_bool(const mq_gguf *g, const char *key, int def);
const char *mq_gguf_get_str(const mq_gguf *g, const char *key, const char *def); /* owned by g */

int64_t mq_gguf_n_tensors(const mq_gguf *g);
int64_t mq_gguf_find_tensor(const mq_gguf *g, const char *name); /* -1 when absent */
const char *mq_gguf_tensor_name(const mq_gguf *g, int64_t i);
/* type: the ggml type id (MQ_TYPE_* where this library has one); ne[0] is the fastest axis
 * (ne[i] = 1 past n_dims); offset: relative to mq_gguf_data_offset. */
int mq_gguf_tensor_info(const mq_gguf *g, int64_t i, int *type, int *n_dims, int64_t ne[4], size_t *offset,
                        size_t *nbytes);
const void *mq_gguf_tensor_data(const mq_gguf *g, int64_t i);

/* Build a runner on the current device from a GGUF file (weights copied; the file is closed on
 * return).  NULL on failure with mq_last_error().  The hyper-parameters read are returned by
 * mq_bert_get_hparams / mq_decoder_get_hparams. */
mq_bert *mq_bert_load(const char *path);
mq_decoder *mq_decoder_load(const char *path);
int mq_bert_get_hparams(const mq_bert *m, mq_bert_hparams *hp);
int mq_decoder_get_hparams(const mq_decoder *m, mq_decoder_hparams *hp);

#ifdef __cplusplus
}
#endif
#endif
