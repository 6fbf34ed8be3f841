/*
 * mq_bert.h -- C ABI of the MI355X BERT-encoder runner in libmq.so.
 *
 * It runs CrispEmbed's post-LN BERT encoder graph (src/crispembed.cpp:1043-1468: token +
 * position + type embeddings and LayerNorm; per layer q/k/v, attention, o, residual
 * LayerNorm, GELU-erf FFN, residual LayerNorm) on one GPU, with every linear layer's
 * GGML_OP_MUL_MAT on the quantized path of mq.h and the other ops as fused fp32 kernels,
 * followed by mean pooling and L2 normalisation (pool_and_norm, src/crispembed.cpp:2024-2045).
 * It stands in for crispembed_encode's batch path (src/crispembed.cpp:2137-2153 builds the
 * same graph for B sequences of T tokens with a full attention mask).
 *
 * Conventions as in mq.h: 0 / negative MQ_E* codes, mq_last_error() for the message.
 * Weights are given as HOST pointers and copied to the device; ids and outputs are
 * DEVICE pointers.  Linear weights are GGUF bytes of mq type `wtype` (Q8_0, Q4_K, Q6_K
 * or F16), rows = out-features, k = in-features (ggml layout).
 */
#ifndef MQ_BERT_H
#define MQ_BERT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mq_bert mq_bert;

/* Hyper-parameters as read from a CrispEmbed GGUF (src/crispembed.cpp:437-470). */
typedef struct mq_bert_hparams {
    int n_layer, n_embd, n_head, n_ff;
    int n_vocab, n_max_pos, n_type;  /* n_type 0: no token-type embedding */
    float layer_norm_eps;
    int wtype;                       /* MQ_TYPE_* of the linear weights */
} mq_bert_hparams;

mq_bert *mq_bert_create(const mq_bert_hparams *hp);
void mq_bert_free(mq_bert *m);

/* token_embd [n_vocab][n_embd], position_embd [n_max_pos][n_embd], token_type_embd
 * [n_type][n_embd] (may be NULL when n_type == 0), embd_ln weight and bias [n_embd]; fp32. */
int mq_bert_set_embeddings(mq_bert *m, const float *tok, const float *pos, const float *type, const float *ln_w,
                           const float *ln_b);

/* Layer il: q, k, v, o [n_embd x n_embd], fc1 [n_ff x n_embd], fc2 [n_embd x n_ff] as GGUF
 * bytes; biases and LayerNorm parameters fp32 (ln1 after attention, ln2 after the FFN). */
int mq_bert_set_layer(mq_bert *m, int il, const void *wq, const void *wk, const void *wv, const void *wo,
                      const void *w1, const void *w2, const float *bq, const float *bk, const float *bv,
                      const float *bo, const float *b1, const float *b2, const float *ln1_w, const float *ln1_b,
                      const float *ln2_w, const float *ln2_b);

/* Encode B sequences of T tokens each (full attention mask, positions 0..T-1).
 * ids / types: device int32 [B*T] (types may be NULL: type 0).  out: device fp32 [B][n_embd],
 * mean-pooled and L2-normalised.  hidden (optional, may be NULL): device fp32 [B*T][n_embd]
 * receives the last layer's output.  Enqueued on `stream`. */
int mq_bert_encode(mq_bert *m, const int32_t *ids, const int32_t *types, int B, int T, float *out, float *hidden,
                   void *stream);

#ifdef __cplusplus
}
#endif
#endif
