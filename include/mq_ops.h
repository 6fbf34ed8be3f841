/*
 * mq_ops.h -- the non-matmul graph ops of CrispEmbed's encoder and decoder graphs on MI355X
 * (libmq.so), on strided tensor views with ggml's metadata (type, ne[4], nb[4] in bytes).
 *
 * These are the ops the MI355X ggml backend executes besides GGML_OP_MUL_MAT, so that the
 * graph built by build_encoder_graph (src/crispembed.cpp:1043-1468) runs on the GPU without
 * the scheduler splitting it at every non-matmul node:
 *   ggml_get_rows        (src/crispembed.cpp:1068-1078)       mq_op_get_rows
 *   ggml_add / ggml_mul  (src/crispembed.cpp:1071,1137,1301)  mq_op_binary
 *   ggml_norm            (src/crispembed.cpp:1135,1321,1446)  mq_op_norm (also ggml_rms_norm,
 *                                                             src/decoder_embed.cpp:717)
 *   ggml_gelu_erf        (src/crispembed.cpp:1415)            mq_op_unary (also silu, relu, gelu)
 *   ggml_cont / ggml_cpy (src/crispembed.cpp:1164-1166)       mq_op_cpy
 *   ggml_flash_attn_ext  (src/crispembed.cpp:1293)            mq_op_flash_attn
 *   ggml_rope_ext        (src/decoder_embed.cpp:756-759)      mq_op_rope
 *   ggml_mul_mat_id      (src/crispembed.cpp:1365,1371)       mq_op_mul_mat_id
 *   ggml_soft_max, ggml_top_k (argsort), ggml_repeat, F32 ggml_mul_mat: the rest of the MoE
 *   FFN block (src/crispembed.cpp:1327-1382)                  mq_op_soft_max, _argsort, _repeat,
 *                                                             _mul_mat_f32
 * The semantics (shapes, broadcasting, op_params) are ggml's, as its CPU backend computes them
 * (ggml-cpu ops.cpp, the ggml submodule pinned in .gitmodules): the ggml backend passes each
 * node's tensors straight through.
 *
 * Conventions are mq.h's: device pointers, `stream` is a hipStream_t, 0 or a negative MQ_E*
 * code with mq_last_error().  A view element (i0, i1, i2, i3) is at
 * data + i0*nb[0] + i1*nb[1] + i2*nb[2] + i3*nb[3]; unused trailing dims have ne = 1.
 * Shapes a kernel does not handle fail with MQ_EUNSUPPORTED before any launch, and
 * mq_op_supported answers the same question without launching (the backend's supports_op).
 */
#ifndef MQ_OPS_H
#define MQ_OPS_H

#include <stddef.h>
#include <stdint.h>

#include "mq.h"

#ifdef __cplusplus
extern "C" {
#endif

#define MQ_TYPE_I32 26 /* ggml GGML_TYPE_I32: row ids of get_rows */

typedef struct mq_view {
    void *data;
    int type; /* MQ_TYPE_* */
    int64_t ne[4];
    size_t nb[4]; /* bytes */
} mq_view;

/* op ids of mq_op_binary / mq_op_unary / mq_op_norm */
#define MQ_BIN_ADD 0
#define MQ_BIN_SUB 1
#define MQ_BIN_MUL 2
#define MQ_BIN_DIV 3

#define MQ_UNARY_GELU_ERF 0 /* 0.5 x (1 + erf(x / sqrt 2))              ggml_gelu_erf */
#define MQ_UNARY_GELU 1     /* 0.5 x (1 + tanh(sqrt(2/pi)(x + 0.044715 x^3)))  ggml_gelu */
#define MQ_UNARY_SILU 2     /* x / (1 + exp(-x))                         ggml_silu */
#define MQ_UNARY_RELU 3     /* max(x, 0)                                 ggml_relu */

#define MQ_NORM_LAYER 0 /* (x - mean) / sqrt(var + eps)   ggml_norm */
#define MQ_NORM_RMS 1   /* x / sqrt(mean(x^2) + eps)      ggml_rms_norm */

/* dst[:, i10, i11, i12] = dequantized row ids[i10, i11, i12] of src plane (i11, i12).
 * src F32, F16, Q8_0, Q4_K or Q6_K (rows contiguous); ids I32; dst F32 [src.ne0, ids.ne0,
 * ids.ne1, ids.ne2].  Quantized rows are dequantized with ggml's dequantize_row arithmetic
 * (bit-identical).  A row id outside [0, src.ne1) is an error the kernel cannot report: the
 * row is written as zeros instead of reading out of bounds. */
int mq_op_get_rows(const mq_view *src, const mq_view *ids, const mq_view *dst, void *stream);

/* dst = get_rows(srcs[0], ids[0]) + get_rows(srcs[1], ids[1]) [+ get_rows(srcs[2], ids[2])],
 * added in that order: the token + position [+ token-type] embedding sum of
 * src/crispembed.cpp:1068-1078 (GET_ROWS, GET_ROWS, ADD, GET_ROWS, ADD) in one pass.  n = 2 or 3
 * F32 tables [ne0, rows_t] with contiguous rows, I32 id vectors of dst's row count, dst dense F32
 * [ne0, rows].  An id outside its table adds a zero row (as mq_op_get_rows gathers one). */
int mq_op_get_rows_sum(int n, const mq_view *const *srcs, const mq_view *const *ids, const mq_view *dst,
                       void *stream);

/* dst = a (op) b, F32, with b broadcast over a (b.ne[i] divides a.ne[i]); dst has a's shape. */
int mq_op_binary(int op, const mq_view *a, const mq_view *b, const mq_view *dst, void *stream);

/* dst = f(x) elementwise, F32, same shape. */
int mq_op_unary(int op, const mq_view *x, const mq_view *dst, void *stream);

/* Row normalisation over ne0, F32, of x (plus `add`, a second F32 tensor of x's shape, when
 * given: the residual ADD that feeds a post-LN block's norm); then, if given, times w and plus b
 * (F32 vectors of ne0 floats, broadcast over rows).  The ADD -> NORM -> MUL -> ADD chain of a
 * post-LN layer norm (src/crispembed.cpp:1320-1323) in one pass; with add, w and b NULL it is
 * ggml_norm / ggml_rms_norm. */
int mq_op_norm(int kind, const mq_view *x, const mq_view *add, const mq_view *dst, float eps, const float *w,
               const float *b, void *stream);

/* mq_op_norm whose result also leaves quantized for the mat-mul that reads it: dst as
 * mq_op_norm writes it (the sums taken in another lane order, so the last bit may differ), and
 * dst's rows quantized to Q8_0 in the GEMM-path activation layout -- the bytes
 * mq_quantize_act_ex(MQ_TYPE_Q8_0, dst, ..., MQ_PATH_GEMM) would write -- into workspace
 * (>= mq_workspace_bytes(MQ_TYPE_Q8_0, rows, ne0)).  The post-LN norm of
 * src/crispembed.cpp:1320-1323 and the from_float quantization of the q/k/v or FFN-up
 * MUL_MAT that reads it (src/crispembed.cpp:1168-1170,1410), in one pass.  x, add and dst
 * have dense, 16-byte aligned rows of ne0 floats, ne0 a multiple of 128 and at most 1024. */
int mq_op_norm_q8_0(int kind, const mq_view *x, const mq_view *add, const mq_view *dst, float eps, const float *w,
                    const float *b, void *workspace, size_t workspace_bytes, void *stream);

/* The decoder's form of mq_op_norm_q8_0, for mat-muls on K-quant weights (Q4_K / Q6_K, whose
 * activations are Q8_K): sum = x + add (add NULL: sum = x; sum NULL: not written; sum may alias
 * x), dst = rms_norm(sum) * w (dst NULL: not written), and the normed rows quantized to Q8_K
 * in the GEMM-path activation layout -- the bytes mq_quantize_act_ex(MQ_TYPE_Q4_K, dst, ...,
 * MQ_PATH_GEMM) writes for them -- into workspace (>= mq_workspace_bytes(MQ_TYPE_Q4_K, rows,
 * ne0)).  The residual ADD, the rms_norm helper (ggml_rms_norm + ggml_mul,
 * src/decoder_embed.cpp:680-683,722,789-790) and the from_float quantization of the q/k/v or
 * gate/up MUL_MAT that reads its result (:724-728,793-795) in one pass.  kind must be
 * MQ_NORM_RMS; x, add, sum and dst are dense, 16-byte aligned rows of ne0 floats, ne0 a
 * multiple of 256 and at most 2048; w 16-byte aligned, the workspace 256-byte aligned. */
int mq_op_norm_q8_K(int kind, const mq_view *x, const mq_view *add, const mq_view *sum, const mq_view *dst, float eps,
                    const float *w, void *workspace, size_t workspace_bytes, void *stream);

/* Copies src into dst element by element in logical (row-major over ne0..ne3) order; the two
 * views hold the same number of elements and may differ in shape and strides (ggml_cpy,
 * ggml_cont, ggml_dup).  F32 / F16 either side (F32 -> F16 rounds to nearest even). */
int mq_op_cpy(const mq_view *src, const mq_view *dst, void *stream);

/* Multi-head attention, ggml_flash_attn_ext semantics without ALiBi or soft-capping:
 *   q [hd, Tq, nh, B], k and v [hd, Tk, nkv, B] (F32, any strides that are multiples of 16
 *   bytes with nb[0] = 4; nh a multiple of nkv: query head h reads kv head h / (nh / nkv)),
 *   mask NULL or F16 [>= Tk, >= Tq, 1 or nh, 1 or B] added to the scaled scores (-inf masks),
 *   dst F32 [hd, nh, Tq, B] (strides as q's rules).  hd 32, 64 or 128.
 * Softmax(scale * q k^T + mask) v in fp32-accurate arithmetic (split-fp16 MFMA products); a
 * query whose keys are all masked gets a zero row.  workspace: mq_op_flash_attn_workspace_bytes
 * of device memory (16-byte aligned) for the K/V operand fragments. */
size_t mq_op_flash_attn_workspace_bytes(const mq_view *k);
int mq_op_flash_attn(const mq_view *q, const mq_view *k, const mq_view *v, const mq_view *mask, const mq_view *dst,
                     float scale, void *workspace, size_t workspace_bytes, void *stream);

/* mq_op_flash_attn that also leaves its result quantized for the output projection that reads
 * it: dst as mq_op_flash_attn writes it, and dst's B * Tq rows of n_head * head_dim values
 * quantized to Q8_0 in the GEMM-path activation layout -- the bytes
 * mq_quantize_act_ex(MQ_TYPE_Q8_0, dst rows, ..., MQ_PATH_GEMM) would write -- into
 * act_workspace (256-byte aligned, >= mq_workspace_bytes(MQ_TYPE_Q8_0, B * Tq, n_head *
 * head_dim)).  The attention of src/crispembed.cpp:1293 and the from_float quantization of the
 * output-projection MUL_MAT after it (src/crispembed.cpp:1300) in one kernel when the 8-wave
 * form runs (head_dim 32 or 64); otherwise the quantizer runs after the attention.  dst must
 * hold dense rows (nb[1] = 4 head_dim, nb[2] = 4 n_head head_dim, nb[3] = nb[2] Tq), n_head *
 * head_dim a multiple of 128. */
int mq_op_flash_attn_q8_0(const mq_view *q, const mq_view *k, const mq_view *v, const mq_view *mask,
                          const mq_view *dst, float scale, void *workspace, size_t workspace_bytes,
                          void *act_workspace, size_t act_workspace_bytes, void *stream);

/* The attention's K/V operand fragments are already in workspace (written by
 * mq_mul_mat_q_qkv): the attention skips its K/V pass and reads k and v for their shapes only. */
#define MQ_ATTN_KV_READY 1

/* mq_op_flash_attn (act_workspace NULL) or mq_op_flash_attn_q8_0 (act_workspace given), with
 * flags: 0 or MQ_ATTN_KV_READY. */
int mq_op_flash_attn_ex(const mq_view *q, const mq_view *k, const mq_view *v, const mq_view *mask,
                        const mq_view *dst, float scale, void *workspace, size_t workspace_bytes,
                        void *act_workspace, size_t act_workspace_bytes, int flags, void *stream);

/* ggml_rope_ext: rotates dimension pairs of x [ne0 >= n_dims, n_head, T, B] by the angles of
 * positions pos[i2] (I32 [T]): pair i < n_dims/2 is (2i, 2i+1) for mode 0 and (i, i + n_dims/2)
 * for MQ_ROPE_NEOX; dimensions from n_dims on are copied.  The angle of pair i at position p is
 * theta_i = p * s * s ... (i products, s = freq_base^(-2/n_dims), fp32), divided by
 * freq_factors[i] when given (F32 [n_dims/2], else NULL), then YaRN-mixed as ggml's rope_yarn:
 * theta = freq_scale * theta_i, and when ext_factor != 0 the interpolation ramp between the
 * correction dimensions of (n_ctx_orig, beta_fast, beta_slow) mixes in theta_i and the
 * magnitude is scaled by 1 + 0.1 ln(1 / freq_scale); cos and sin are scaled by attn_factor.
 * x and dst F32 with contiguous rows (may be the same tensor). */
#define MQ_ROPE_NORMAL 0
#define MQ_ROPE_NEOX 2
int mq_op_rope(const mq_view *x, const mq_view *pos, const mq_view *freq_factors, const mq_view *dst, int n_dims,
               int mode, int n_ctx_orig, float freq_base, float freq_scale, float ext_factor, float attn_factor,
               float beta_fast, float beta_slow, void *stream);

/* mq_op_rope of rms_norm(x) * w: the decoder's per-head q / k norm (ggml_rms_norm over ne0, then
 * ggml_mul by the F32 row w [ne0]) and rotation (src/decoder_embed.cpp:737-759) in one pass,
 * equal bit for bit to mq_op_norm(MQ_NORM_RMS, x, NULL, tmp, eps, w, NULL) followed by
 * mq_op_rope(tmp, ...).  mode MQ_ROPE_NEOX with n_dims = ne0 = 128 only. */
int mq_op_rms_norm_rope(const mq_view *x, float eps, const float *w, const mq_view *pos, const mq_view *freq_factors,
                        const mq_view *dst, int n_dims, int mode, int n_ctx_orig, float freq_base, float freq_scale,
                        float ext_factor, float attn_factor, float beta_fast, float beta_slow, void *stream);

/* The rope cache of mq_op_rope's angles: cs[2 (t n_dims/2 + i)] = cos(theta) attn_factor' and
 * cs[2 (t n_dims/2 + i) + 1] = sin(theta) attn_factor' for position pos[t] (I32 [T]) and pair
 * i < n_dims/2, with theta and the YaRN magnitude factor exactly as mq_op_rope computes them
 * (the angles of the ggml_rope_ext nodes of src/decoder_embed.cpp:758-763).  cs: device memory
 * of T n_dims floats; n_dims even, at most 128. */
int mq_op_rope_cache(const mq_view *pos, const mq_view *freq_factors, int n_dims, int n_ctx_orig, float freq_base,
                     float freq_scale, float ext_factor, float attn_factor, float beta_fast, float beta_slow,
                     float *cs, void *stream);

/* mq_op_flash_attn_ex (flags 0) whose q and k are taken before the decoder's per-head q / k
 * norm and rotation (src/decoder_embed.cpp:735-763): the attention reads
 *   q' = rope(rms_norm(q) * q_norm_w),  k' = rope(rms_norm(k) * k_norm_w)
 * (RMS norm over head_dim with eps, weights F32 [head_dim], NEOX rotation of all head_dim
 * dimensions by the angles of cs, the mq_op_rope_cache table with n_dims = head_dim over the
 * Tq = Tk positions) -- the ROPE(MUL(RMS_NORM)) nodes of q and k and the attention in two
 * kernels.  Equal to those ops followed by mq_op_flash_attn_ex up to the norm's summation order. */
int mq_op_flash_attn_qk_norm_rope(const mq_view *q, const mq_view *k, const mq_view *v, const mq_view *mask,
                                  const mq_view *dst, float scale, const float *q_norm_w, const float *k_norm_w,
                                  float eps, const float *cs, void *workspace, size_t workspace_bytes,
                                  void *act_workspace, size_t act_workspace_bytes, void *stream);

/* Block lists of an attention mask, for the batched decoder's T_total x T_total F16 mask
 * (decoder_encode_tokens_batch, src/decoder_embed.cpp:1406-1443 builds it, :1517 passes it to
 * every layer's ggml_flash_attn_ext): for each tile of 32 query rows, the 32-key blocks in
 * which some row of the tile has a finite mask value, and whether the block's values are all
 * zero.  The attention then runs only those blocks (an all-zero block with no mask reads),
 * instead of classifying the whole mask in every workgroup of every layer: one pass over the
 * mask per graph.  mq_op_mask_blocks_bytes is 0 when the attention of these q / k / mask
 * operands (as mq_op_flash_attn takes them) reads no block lists: no mask, a mask that differs
 * per head, or an attention form that classifies per block itself; else the bytes of device
 * memory mq_op_mask_blocks fills (4-byte aligned).  The lists stay valid while the mask's
 * values and the operands' shapes do. */
size_t mq_op_mask_blocks_bytes(const mq_view *q, const mq_view *k, const mq_view *mask);
int mq_op_mask_blocks(const mq_view *q, const mq_view *k, const mq_view *mask, void *blocks, size_t blocks_bytes,
                      void *stream);

/* The structure of a batched decoder's mask (decoder_encode_tokens_batch without a shared prefix,
 * every item T_max long: src/decoder_embed.cpp:1429-1437): seg_len = S when the T x T mask of q
 * and k (T positions, one batch, the mask shared by every head) is exactly block-diagonal causal
 * over segments of S rows -- 0 on keys from the row's segment start up to the row itself, -inf
 * on every other key, every value -- else 0.  One pass over the mask and a T x 4-byte readback:
 * the call synchronizes the stream (not for HIP graph capture).  scratch: device memory of
 * mq_op_mask_segments_bytes (0: these operands have no such form).  The attention of such a mask
 * is the per-segment causal attention, with no mask reads (mq_op_flash_attn_blocks'
 * causal_segment). */
size_t mq_op_mask_segments_bytes(const mq_view *q, const mq_view *k, const mq_view *mask);
int mq_op_mask_segments(const mq_view *q, const mq_view *k, const mq_view *mask, void *scratch, size_t scratch_bytes,
                        int64_t *seg_len, void *stream);

/* Whether an attention's F16 mask adds nothing: *is_zero = 1 when every value of the Tq x Tk region
 * (Tq = q->ne[1], Tk = k->ne[1]) of each of the mask's planes is +-0 -- an equal-length batch's
 * padding mask (src/crispembed.cpp:2052-2135) -- so the attention may run unmasked with the same
 * scores.  scratch: 4 bytes of device memory.  Synchronizes the stream (one flag read back): not
 * for capture. */
int mq_op_mask_is_zero(const mq_view *q, const mq_view *k, const mq_view *mask, void *scratch, size_t scratch_bytes,
                       int *is_zero, void *stream);

/* The general attention entry point: mq_op_flash_attn_ex with flags, plus the q / k norm and
 * rotation of mq_op_flash_attn_qk_norm_rope when q_norm_w, k_norm_w and cs are given (all three,
 * or all NULL), plus mask_blocks: NULL, or mq_op_mask_blocks' lists for these q, k and mask
 * (ignored when mq_op_mask_blocks_bytes of the operands is 0), plus causal_segment: 0, or the
 * seg_len mq_op_mask_segments found for this mask (a multiple of 32): each segment then runs as a
 * causal sequence of its own and the mask is not read; plus act_type: the weight type of the
 * projection that reads the result when act_workspace is given (MQ_TYPE_Q8_0, or MQ_TYPE_Q4_K /
 * MQ_TYPE_Q6_K for their Q8_K activations: n_head * head_dim a multiple of 256), whose activation
 * workspace receives the rows quantized as mq_quantize_act_ex(act_type, ..., MQ_PATH_GEMM) writes
 * them.  Results equal those entry points' up to the order in which the waves of a query tile
 * share out its key blocks. */
int mq_op_flash_attn_blocks(const mq_view *q, const mq_view *k, const mq_view *v, const mq_view *mask,
                            const mq_view *dst, float scale, const float *q_norm_w, const float *k_norm_w, float eps,
                            const float *cs, const void *mask_blocks, int64_t causal_segment, void *workspace,
                            size_t workspace_bytes, void *act_workspace, size_t act_workspace_bytes, int act_type,
                            int flags, void *stream);

/* ggml_mul_mat_id, the mixture-of-experts mat-mul (src/crispembed.cpp:1365,1371):
 *   experts: n_exp prepared weight images of `type` (n x k each, as mq_weight_prepare builds
 *            them), expert e at expert_images + e * expert_stride bytes;
 *   b   F32 [k, nb1, T] (rows contiguous): slot i of token t reads row i % nb1 of token t
 *       (nb1 = 1: every slot reads the token's one row);
 *   ids I32 [n_used, T] (any row stride): the expert of slot i of token t;
 *   dst F32 [n, n_used, T] (rows contiguous): dst[:, i, t] = W_{ids[i, t]} b[:, i % nb1, t].
 * The routing is read back to the host (the stream is synchronized once, as ggml's GPU
 * backends do for ids), the rows are gathered by expert in one pass, every used expert runs one
 * activation quantization and one GEMM or GEMV (mq_mul_mat_path) over its rows, and one pass
 * scatters the results.  An id outside [0, n_exp) fails with MQ_EINVAL (after the sync).
 * workspace: mq_op_mul_mat_id_workspace_bytes(type, n, k, n_used * T) bytes, 256-aligned. */
size_t mq_op_mul_mat_id_workspace_bytes(int type, int64_t n, int64_t k, int64_t rows);
int mq_op_mul_mat_id(int type, const void *expert_images, size_t expert_stride, int n_exp, int64_t n, int64_t k,
                     const mq_view *b, const mq_view *ids, const mq_view *dst, void *workspace, size_t workspace_bytes,
                     void *stream);

/* ggml_mul_mat_id (src/crispembed.cpp:1365,1371) with the routing on the device: the same
 * operands and result as mq_op_mul_mat_id, with no stream synchronization and no host copy, so
 * it can be enqueued ahead and captured in a HIP graph.  One workgroup counts the slots per
 * expert and lays the rows out by expert in segments of whole row tiles (64 or 256 rows), one
 * pass gathers them, one activation quantization and one GEMM launch cover every expert (each
 * row tile reads its expert's weights from a device table; tiles past the used ones exit), and
 * one pass scatters the results.  A slot whose id lies outside [0, n_exp) gets a row of NaN.
 * n_exp <= 1024.  workspace: mq_op_mul_mat_id_device_workspace_bytes(type, n_exp, n, k,
 * n_used * T) bytes, 256-aligned (the rows padded to whole tiles per expert). */
size_t mq_op_mul_mat_id_device_workspace_bytes(int type, int n_exp, int64_t n, int64_t k, int64_t rows);
int mq_op_mul_mat_id_device(int type, const void *expert_images, size_t expert_stride, int n_exp, int64_t n, int64_t k,
                            const mq_view *b, const mq_view *ids, const mq_view *dst, void *workspace,
                            size_t workspace_bytes, void *stream);

/* ggml_soft_max_ext without ALiBi (src/crispembed.cpp:1267,1336): dst = softmax over ne0 of
 * x * scale + mask, mask NULL or F16/F32 [ne0, >= ne1, ...] (row i1 of x uses mask row i1; mask
 * planes broadcast over x's by index modulo), -inf entries masked; a row with every entry
 * masked gives zeros.  F32 x and dst, rows contiguous. */
int mq_op_soft_max(const mq_view *x, const mq_view *mask, const mq_view *dst, float scale, void *stream);

/* ggml_argsort (ggml_top_k takes its first k columns, src/crispembed.cpp:1339): dst I32 row =
 * the indices of x's F32 row in descending (MQ_SORT_DESC) or ascending order, equal values in
 * index order (a stable sort).  ne0 <= 1024. */
#define MQ_SORT_ASC 0
#define MQ_SORT_DESC 1
int mq_op_argsort(const mq_view *x, const mq_view *dst, int order, void *stream);

/* ggml_repeat (src/crispembed.cpp:1361): dst[i0, i1, i2, i3] = src[i0 % ne0, i1 % ne1, ...];
 * every extent of src divides dst's.  F32. */
int mq_op_repeat(const mq_view *src, const mq_view *dst, void *stream);

/* GGML_OP_MUL_MAT with an F32 first operand, for the small products of the graphs (the MoE
 * router and its weighted sum over experts, src/crispembed.cpp:1333,1378):
 * dst[i, j, b2, b3] = sum_k a[k, i, b2 / (ne12/ne02), b3 / (ne13/ne03)] * b[k, j, b2, b3] in
 * fp32 (a's batches broadcast as ggml does).  One thread per output: meant for outputs with at
 * most 2^26 multiply-adds. */
int mq_op_mul_mat_f32(const mq_view *a, const mq_view *b, const mq_view *dst, void *stream);

/* ids for mq_op_supported */
#define MQ_OP_GET_ROWS 0
#define MQ_OP_BINARY 1
#define MQ_OP_UNARY 2
#define MQ_OP_NORM 3
#define MQ_OP_CPY 4
#define MQ_OP_FLASH_ATTN 5
#define MQ_OP_ROPE 6 /* sub = mode; src0 x, src1 pos, src2 freq_factors; n_dims = x.ne0 assumed */
#define MQ_OP_SOFT_MAX 7  /* src0 x, src1 mask */
#define MQ_OP_ARGSORT 8   /* sub = order */
#define MQ_OP_REPEAT 9
#define MQ_OP_MUL_MAT_F32 10 /* src0 a, src1 b */

/* 1 when mq_op_<op> accepts these operands (srcs in the op's argument order, NULL where an
 * optional operand is absent -- for MQ_OP_NORM src1 is `add`; `sub` is the binary / unary /
 * norm op id), else 0.  Host only. */
int mq_op_supported(int op, int sub, const mq_view *src0, const mq_view *src1, const mq_view *src2,
                    const mq_view *src3, const mq_view *dst);

#ifdef __cplusplus
}
#endif
#endif
