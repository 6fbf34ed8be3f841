/*
 * mq_decoder.h -- C ABI of the MI355X decoder-embedder runner in libmq.so.
 *
 * It runs CrispEmbed's decoder embedding graph for the Qwen3 family
 * (src/decoder_embed.cpp:565-830: token embedding; per layer RMS norm, q/k/v projections,
 * per-head q/k RMS norms, NEOX RoPE, causal grouped-query attention, o projection and
 * residual, RMS norm, SwiGLU FFN and residual; output RMS norm) followed by last-token or
 * mean pooling and L2 normalisation (src/decoder_embed.cpp:1044-1100).  It stands in for
 * decoder_encode_tokens (src/decoder_embed.cpp:565) over B sequences of T tokens each,
 * every sequence attending causally to its own tokens only.  Every linear layer's
 * GGML_OP_MUL_MAT runs on the quantized path of mq.h; the other ops are fp32 kernels.
 *
 * Conventions as in mq.h: 0 / negative MQ_E* codes, mq_last_error() for the message.
 * Weights are HOST pointers (copied to the device); ids and outputs are DEVICE pointers.
 * Linear weights are GGUF bytes of mq type `wtype`, rows = out-features (ggml layout).
 */
#ifndef MQ_DECODER_H
#define MQ_DECODER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mq_decoder mq_decoder;

/* Hyper-parameters as read from a CrispEmbed decoder GGUF (src/decoder_embed.cpp:96-175). */
typedef struct mq_decoder_hparams {
    int n_layer, n_embd, n_head, n_kv_head, head_dim, n_ff, n_vocab;
    float rms_norm_eps, rope_theta;
    int causal;   /* 1: causal mask (Qwen3); 0: bidirectional */
    int pooling;  /* 2: last token (Qwen3), 1: mean over the sequence */
    int wtype;    /* MQ_TYPE_* of the linear weights */
} mq_decoder_hparams;

mq_decoder *mq_decoder_create(const mq_decoder_hparams *hp);
void mq_decoder_free(mq_decoder *m);

/* token_embd [n_vocab][n_embd] and output_norm [n_embd], fp32. */
int mq_decoder_set_embeddings(mq_decoder *m, const float *tok, const float *out_norm);

/* Layer il: q [n_head*head_dim x n_embd], k and v [n_kv_head*head_dim x n_embd],
 * o [n_embd x n_head*head_dim], gate and up [n_ff x n_embd], down [n_embd x n_ff] as GGUF
 * bytes; attn_norm, ffn_norm [n_embd] and q_norm, k_norm [head_dim] fp32 (q_norm / k_norm
 * may be NULL: no per-head norm). */
int mq_decoder_set_layer(mq_decoder *m, int il, const void *wq, const void *wk, const void *wv, const void *wo,
                         const void *wgate, const void *wup, const void *wdown, const float *attn_norm,
                         const float *ffn_norm, const float *q_norm, const float *k_norm);

/* Encode B sequences of T tokens (positions 0..T-1 each).  ids: device int32 [B*T].
 * out: device fp32 [B][n_embd], pooled and L2-normalised.  hidden (optional, may be NULL):
 * device fp32 [B*T][n_embd] receives the last layer's residual stream (before the output
 * norm).  Enqueued on `stream`. */
int mq_decoder_encode(mq_decoder *m, const int32_t *ids, int B, int T, float *out, float *hidden, void *stream);

/* An observer of the runner's intermediate tensors: the runner's form of the scheduler eval
 * callback CrispEmbed installs to read every MUL_MAT's input (the imatrix collector,
 * src/imatrix.cpp:57-99, installed at src/crispembed.cpp:723 and :2483).  With an observer set,
 * mq_decoder_encode synchronises its stream after each tensor below is final and calls
 *   cb(name, layer, x, rows, cols, xq, xq_bytes, user)
 * with x a DEVICE fp32 tensor of rows x cols (dense rows) and xq the quantized activation the
 * following mat-mul reads (DEVICE, in the layout mq_quantize_act_ex writes for the path
 * mq_mul_mat_path(wtype, n, cols, rows) of that mat-mul) or NULL:
 *   "attn_norm"  layer il's normed input, the src1 of the q/k/v mat-muls (xq: its quantization)
 *   "attn_out"   the attention output rows, the src1 of the o projection (xq: its quantization)
 *   "ffn_norm"   the normed input of the FFN, the src1 of gate/up (xq: its quantization)
 *   "ffn_gate_up" the gate and up projections side by side (cols = 2 n_ff); the src1 of the
 *                down projection is silu(gate) * up, which the quantizer forms (xq: its
 *                quantization, cols n_ff)
 *   "l_out"      the residual stream after layer il (xq NULL)
 * The tensors are only valid during the call.  Observing makes the runner also write the
 * normed rows it otherwise leaves only in quantized form, and the gate and up projections that
 * large batches otherwise never write (silu(gate) * up then formed in the gate|up GEMM's store,
 * mq_mul_mat_q_swiglu); the quantized bytes do not change.
 * cb NULL removes the observer. */
typedef void (*mq_decoder_observer)(const char *name, int layer, const float *x, int64_t rows, int64_t cols,
                                    const void *xq, size_t xq_bytes, void *user);
int mq_decoder_set_observer(mq_decoder *m, mq_decoder_observer cb, void *user);

/* The runner's non-MUL_MAT ops on caller buffers (device pointers, fp32), for callers that
 * build their own graph.  qkv holds B*T rows of ld floats: n_head query heads, then
 * n_kv_head key heads, then n_kv_head value heads, head_dim values each (ld a multiple of 4,
 * the buffer 16-byte aligned).
 *
 * mq_qk_norm_rope: in place on the query and key heads, per head RMS norm times q_norm /
 * k_norm (each may be NULL: no norm) then NEOX RoPE at positions row % T with base theta
 * (the ggml_rms_norm + ggml_mul + ggml_rope_ext mode 2 nodes, src/decoder_embed.cpp:735-766).
 *
 * mq_attention: out[row][h*head_dim + d] = softmax(scale * q k^T + mask) v per sequence and
 * query head h, key/value head h / (n_head / n_kv_head), mask causal or none
 * (ggml_flash_attn_ext, src/decoder_embed.cpp:769-777).  workspace: device memory of at least
 * mq_attention_workspace_bytes(B, T, n_kv_head, head_dim) bytes, 16-byte aligned (the keys and
 * values re-laid as matrix-core operands; B * n_kv_head * ceil(T/32) * 32 KB at head_dim 128). */
int mq_qk_norm_rope(float *qkv, int64_t ld, const float *q_norm, const float *k_norm, float eps, int n_head,
                    int n_kv_head, int head_dim, int T, float theta, int64_t rows, void *stream);
size_t mq_attention_workspace_bytes(int B, int T, int n_kv_head, int head_dim);
int mq_attention(const float *qkv, int64_t ld, float *out, int64_t ldo, int B, int T, int n_head, int n_kv_head,
                 int head_dim, float scale, int causal, void *workspace, size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif
