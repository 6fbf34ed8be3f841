/*
 * mq.h -- C ABI of the MI355X (gfx950) quantized mat-mul library (libmq.so).
 *
 * This is the drop-in boundary for CrispEmbed's GGML_OP_MUL_MAT hot path on
 * GGUF block-quantized weights.  In CrispEmbed every linear layer is
 * ggml_mul_mat(W, X) (src/crispembed.cpp:1168-1170,1300,1410,1416;
 * src/decoder_embed.cpp:724-802; src/qwen2vl_ocr.cpp:2368-2452) and is executed
 * by a ggml backend's graph_compute, reached from ggml_backend_sched_graph_compute
 * (src/crispembed.cpp:1471-1483).  The ggml backend in ggml-mi355.h is built on
 * top of these entry points; callers that do not use ggml can call them directly.
 *
 * Conventions
 *   - All tensor pointers are DEVICE pointers unless the name says host.
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream).
 *     Entry points enqueue work and return; they do not synchronize.
 *   - Return value: 0 on success, a negative MQ_E* code on failure;
 *     mq_last_error() returns a message for the calling thread.
 *   - Layout follows ggml: a weight W has ne[0] = k (in-features, the axis the
 *     quant blocks run along) and ne[1] = n rows; activations X are m rows of
 *     k floats with row stride ldx (floats); Y[i*ldy + j] = sum_k W[j,k]*X[i,k].
 *   - Type ids are ggml/GGUF ids: F32 0, F16 1, Q8_0 8, Q4_K 12, Q6_K 14, Q8_K 15.
 */
#ifndef MQ_H
#define MQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MQ_TYPE_F32 0
#define MQ_TYPE_F16 1
#define MQ_TYPE_Q8_0 8
#define MQ_TYPE_Q4_K 12
#define MQ_TYPE_Q6_K 14
#define MQ_TYPE_Q8_K 15

#define MQ_OK 0
#define MQ_EINVAL (-1)      /* bad argument: shape, type, alignment, NULL pointer */
#define MQ_EUNSUPPORTED (-2) /* valid ggml input this library does not handle */
#define MQ_EHIP (-3)        /* a HIP runtime call failed */
#define MQ_ENOMEM (-4)      /* device allocation failed */
#define MQ_ENODEV (-5)      /* no gfx950 device */

/* Q8_0 activation rounding variants (the host ISA decides which one ggml-cpu runs):
 * X86 : id = 127/amax, q = round-half-even(x*id)   (AVX/AVX2/AVX-512 quantize_row_q8_0)
 * NEON: id = 1/(amax/127), q = round-half-even(x*id)
 * REF : id = 1/(amax/127), q = roundf(x*id)          (quantize_row_q8_0_ref) */
#define MQ_Q8_0_X86 0
#define MQ_Q8_0_NEON 1
#define MQ_Q8_0_REF 2

/* mq_mul_mat_ex path selection */
#define MQ_PATH_AUTO 0 /* GEMV when m <= mq_gemv_max_m(), else GEMM */
#define MQ_PATH_GEMV 1 /* weight-streaming GEMV, m <= 32 (one launch per 8 rows) */
#define MQ_PATH_GEMM 2 /* MFMA GEMM */

/* Elementwise prologue of mq_quantize_act_ex, applied to X before it is quantized. */
#define MQ_PRE_NONE 0     /* x (+ bias) */
#define MQ_PRE_GELU_ERF 1 /* gelu_erf(x + bias) */
#define MQ_PRE_SILU_MUL 2 /* silu(g) * u: row = [g (k values) | u (k values)], ldx >= 2k */

/* ---- library / device ---- */

/* Checks that the current HIP device is gfx950.  Replaces nothing in the reference
 * (ggml backends check their device inside ggml_backend_dev_init). */
int mq_init(void);
const char *mq_last_error(void);
/* Largest m routed to the GEMV path by MQ_PATH_AUTO (default 8; env MQ_FORCE_GEMV_MAX_M). */
int mq_gemv_max_m(void);
/* The device's sustained dense int8 MFMA rate, measured: one workgroup per CU, one wave per SIMD,
 * each wave issuing `iters` x 8 independent v_mfma_i32_32x32x32_i8 (no memory traffic), timed
 * with HIP events on `stream`; *tops = 2*32*32*32 ops per MFMA / time in TOP/s.  A measurement
 * aid for comparing kernels with what the chip holds under MFMA load (its clock drops below the
 * datasheet's); no counterpart in the reference. */
int mq_measure_mfma_i8(int iters, double *tops, void *stream);
/* Q8_0 activation rounding variant used by mq_mul_mat (default MQ_Q8_0_X86; env MQ_Q8_0_VARIANT). */
int mq_q8_0_variant(void);
int mq_set_q8_0_variant(int variant);

/* ---- type traits (ggml_blck_size / ggml_type_size / ggml_row_size) ---- */
int64_t mq_blck_size(int type);
size_t mq_type_size(int type);
size_t mq_row_size(int type, int64_t k);
/* ggml's vec_dot_type: the type CPU mul_mat converts X to (Q8_0->Q8_0, Q4_K/Q6_K->Q8_K, F16->F16). */
int mq_vec_dot_type(int type);
/* 1 if mq_mul_mat accepts weights of this type with this k (k % block == 0, F16 k % 32 == 0). */
int mq_supports(int type, int64_t k);

/* ---- host weight quantization (producer side) ----
 * Replaces ggml_quantize_chunk(type, src, dst, 0, nrows, k, NULL) as called by
 * tools/quantize.cpp:804-805 (no importance matrix: ggml's _ref quantizers).
 * HOST pointers.  Returns bytes written, 0 on bad type/shape. */
size_t mq_quantize_chunk(int type, const float *src_host, void *dst_host, int64_t nrows, int64_t k);

/* ---- activation quantization, GGUF block layout (device) ----
 * quantize_row_q8_0 (ggml-cpu from_float for Q8_0 weights), one row of k per x row. */
int mq_quantize_q8_0(const float *x, int64_t ldx, void *y, int64_t nrows, int64_t k, int variant, void *stream);
/* quantize_row_q8_K (from_float for Q4_K / Q6_K weights): block_q8_K {float d; int8 qs[256]; int16 bsums[16]}. */
int mq_quantize_q8_K(const float *x, int64_t ldx, void *y, int64_t nrows, int64_t k, void *stream);
/* fp32 -> fp16 round-to-nearest-even (from_float for F16 weights). */
int mq_quantize_f16(const float *x, int64_t ldx, void *y, int64_t nrows, int64_t k, void *stream);

/* ---- dequantization (ggml type_traits to_float; src/core/cpu_ops.h:63-65) ----
 * GGUF rows -> fp32.  fused=1 evaluates Q4_K's d1*q - m1 as one fma (what a
 * contracting compiler emits); fused=0 rounds the product and the difference
 * separately.  Other types are unaffected by the flag. */
int mq_dequantize(int type, const void *w, float *y, int64_t nrows, int64_t k, int fused, void *stream);

/* ---- weight images ----
 * A weight image is the GGUF bytes of an n x k tensor (row-major blocks, exactly
 * what core_gguf::load_weights uploads with ggml_backend_tensor_set,
 * src/core/gguf_loader.cpp:480), followed at mq_gguf_bytes_aligned() by derived
 * planes in the layout the GEMM / GEMV kernels read.  mq_weight_prepare() builds
 * the planes from the GGUF part; the GGUF part is never modified, so reading it
 * back returns the original bytes. */
size_t mq_gguf_bytes(int type, int64_t n, int64_t k);
size_t mq_gguf_bytes_aligned(int type, int64_t n, int64_t k);
size_t mq_weight_image_bytes(int type, int64_t n, int64_t k);
/* Rebuild planes for rows [row0, row1) after a (partial) write of the GGUF part. */
int mq_weight_prepare(int type, void *image, int64_t n, int64_t k, int64_t row0, int64_t row1, void *stream);

/* ---- mul_mat ----
 * Y = X * W^T with ggml CPU semantics: X is requantized to mq_vec_dot_type(type)
 * exactly as ggml's from_float does, the integer block dots are exact, and the
 * per-block fp16/fp32 scales are applied in fp32.
 * `w_image` is a prepared weight image.  `workspace` receives the quantized
 * activations; size it with mq_workspace_bytes().  workspace == NULL makes the
 * library use (and grow with hipMalloc) an internal buffer per (device, stream), so
 * calls on different streams never share one; calls on one stream from several threads
 * must be serialised by the caller (as ggml backends are, src/core/gpu_backend_pref.h:180-185).
 * Growing that buffer synchronizes the stream and calls hipMalloc, which HIP graph capture does
 * not allow: under capture pass a workspace, or make an equally large call on the stream before
 * capturing.  Each stream's buffer lives until mq_release_workspace(stream) or the process ends;
 * a caller that creates short-lived streams releases it before destroying the stream. */
/* The path MQ_PATH_AUTO of mq_mul_mat / mq_mul_mat_ex takes for an n x k weight and m rows:
 * MQ_PATH_GEMV up to mq_gemv_max_m() rows, and up to 32 rows while a 128 x 128 GEMM tile grid
 * would have fewer than 64 workgroups (short inputs on narrow layers); else MQ_PATH_GEMM.
 * Callers of the two-step API (mq_quantize_act_ex + mq_mul_mat_q*) pass it to both calls. */
int mq_mul_mat_path(int type, int64_t n, int64_t k, int64_t m);
size_t mq_workspace_bytes(int type, int64_t m, int64_t k);
/* Frees the internal workspace of `stream` on the current device (after synchronizing the
 * stream), if it has one.  No counterpart in the reference (ggml frees a backend's buffers with
 * the backend); for callers that create and destroy streams. */
int mq_release_workspace(void *stream);
int mq_mul_mat(int type, const void *w_image, int64_t n, int64_t k, const float *x, int64_t ldx, int64_t m, float *y,
               int64_t ldy, void *workspace, size_t workspace_bytes, void *stream);
int mq_mul_mat_ex(int type, const void *w_image, int64_t n, int64_t k, const float *x, int64_t ldx, int64_t m,
                  float *y, int64_t ldy, void *workspace, size_t workspace_bytes, int path, void *stream);

/* mq_mul_mat_ex that allocates nothing.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, serving loops and
 * harnesses that forbid hipMalloc).  The quantized activations go to a fixed device array
 * inside libmq.so of MQ_NOALLOC_SCRATCH_BYTES (64 MiB) per GPU, held until the process ends,
 * instead of a workspace argument or an internal hipMalloc'd buffer; results equal
 * mq_mul_mat_ex's bit for bit.  Calls whose mq_workspace_bytes(type, m, k) exceeds the array
 * fail with MQ_EINVAL (e.g. Q8_K activations of 8192 x 4096 need 38.4 MB and fit; 16384 x 4096
 * do not).  Every call on one GPU shares that GPU's array: calls that overlap on one GPU (two
 * streams, or two threads) race on it and must be serialised by the caller. */
#define MQ_NOALLOC_SCRATCH_BYTES (64u << 20)
int mq_mul_mat_noalloc(int type, const void *w_image, int64_t n, int64_t k, const float *x, int64_t ldx, int64_t m,
                       float *y, int64_t ldy, int path, void *stream);

/* The two halves of mq_mul_mat_ex, for callers that reuse one quantized X for
 * several weights (q, k and v share their input in every encoder layer,
 * src/crispembed.cpp:1168-1170) or time the stages separately.
 * mq_quantize_act writes X in mq_vec_dot_type(type) to `workspace`, in the layout of
 * the path that will read it (the GEMV reads row-major quants, the GEMM tiled
 * ones); mq_mul_mat_q then runs that path.  Pass the same `path` to both. */
int mq_quantize_act(int type, const float *x, int64_t ldx, int64_t m, int64_t k, void *workspace,
                    size_t workspace_bytes, int path, void *stream);
int mq_mul_mat_q(int type, const void *w_image, int64_t n, int64_t k, const void *workspace, int64_t m, float *y,
                 int64_t ldy, int path, void *stream);

/* mq_mul_mat_q with the linear layer's bias: Y = X W^T + bias, bias an fp32 [n] row (NULL:
 * none) added to every output row as the GEMM / GEMV stores it -- the MUL_MAT and the ADD of
 * its bias in the graph (src/crispembed.cpp:1168-1170,1300-1301,1410-1416) in one pass, with
 * the same fp32 rounding as the ADD node. */
int mq_mul_mat_q_ex(int type, const void *w_image, int64_t n, int64_t k, const void *workspace, int64_t m, float *y,
                    int64_t ldy, const float *bias, int path, void *stream);

/* Up to 4 mat-muls on the same quantized activation in one launch (the q, k and v projections
 * of an encoder layer read one input, src/crispembed.cpp:1168-1170): for g < n_groups,
 * Y_g = X W_g^T + bias_g (bias NULL, or bias[g] NULL: none), every W_g of `type` with k
 * in-features, n[g] out-features, output row stride ldy[g].  The GEMM walks the feature tiles
 * of all groups as one grid, so three narrow projections fill the GPU like one wide one; the
 * GEMV path runs the groups one after another.  Results equal separate mq_mul_mat_q_ex calls
 * bit for bit. */
int mq_mul_mat_q_group(int type, int n_groups, const void *const *w_images, const int64_t *n, int64_t k,
                       const void *workspace, int64_t m, float *const *y, const int64_t *ldy, const float *const *bias,
                       int path, void *stream);

/* The GEMV path with the activation quantization inside the mat-mul kernel, for decode-sized
 * inputs: m <= 8 fp32 rows, K-quant weights (Q4_K, Q6_K) with k <= 6144, up to 3 weights on one
 * activation in one launch: Y_g = op(X) W_g^T + bias_g (bias NULL, or bias[g] NULL: none).
 * Bit for bit what mq_quantize_act_ex(type, X, ..., op, MQ_PATH_GEMV) followed by
 * mq_mul_mat_q_group(..., MQ_PATH_GEMV) computes, without the separate quantization launch and
 * without a caller workspace: every workgroup quantizes the activation it reads, while that is a
 * few superblock-rows (m * k / 256, three times that with SiLU, at most 100); larger ones are
 * quantized once into the library's internal workspace of this stream (as mq_mul_mat_ex with a
 * NULL workspace) and read by the same GEMV -- whose first such call on a stream may synchronize
 * it and hipMalloc, so under HIP graph capture make one equally large call on the stream before
 * capturing.  op MQ_PRE_NONE, or
 * MQ_PRE_SILU_MUL with x2 the up-projection rows (row stride ldx2): the value quantized is then
 * silu(x) * x2, the SwiGLU input of the down projection.  These are the MUL_MATs of the decode
 * step, one to eight new tokens: q/k/v (src/qwen2vl_ocr.cpp:2368-2372), o (:2430), gate/up and
 * down (:2437-2439), the lm_head (:2452).  x and x2 16-byte aligned, ldx and ldx2 multiples of 4;
 * other shapes return MQ_EUNSUPPORTED (use the two-step form). */
int mq_mul_mat_gemv(int type, int n_groups, const void *const *w_images, const int64_t *n, int64_t k, const float *x,
                    int64_t ldx, const float *x2, int64_t ldx2, int op, int64_t m, float *const *y, const int64_t *ldy,
                    const float *const *bias, void *stream);

/* Two mat-muls in a row without the fp32 tensor between them: computes
 * V = op(X W^T + bias) on the GEMM path (workspace: X quantized with path MQ_PATH_GEMM) and
 * writes V quantized for the next product's weights, of type out_type, straight into
 * out_workspace, in the layout that mq_quantize_act_ex(out_type, V, ..., MQ_PATH_GEMM) writes --
 * the same bytes, bit for bit -- ready for mq_mul_mat_q_ex(out_type, W2, n2, n, out_workspace, m,
 * ..., MQ_PATH_GEMM).  V itself is never written.  This is the encoder FFN of
 * src/crispembed.cpp:1410-1416 (FFN-up MUL_MAT, bias ADD, ggml_gelu_erf, then the FFN-down
 * MUL_MAT, whose CPU backend quantizes its src1 through the vec_dot_type's from_float before the
 * block dots).  out_type MQ_TYPE_Q8_0 (Q8_0 activations): n a multiple of 128.  out_type
 * MQ_TYPE_Q4_K or MQ_TYPE_Q6_K (Q8_K activations): type Q4_K or Q6_K, n a multiple of 256 and
 * a product of at least 256 workgroups of 128 x 256 (MQ_EUNSUPPORTED otherwise: use
 * mq_mul_mat_q_ex and mq_quantize_act_ex).  op MQ_PRE_NONE or MQ_PRE_GELU_ERF;
 * out_workspace_bytes >= mq_workspace_bytes(out_type, m, n). */
int mq_mul_mat_q_requant(int type, const void *w_image, int64_t n, int64_t k, const void *workspace, int64_t m,
                         const float *bias, int op, int out_type, void *out_workspace, size_t out_workspace_bytes,
                         void *stream);

/* 1 when mq_mul_mat_q_requant(type, ..., n, k, ..., m, ..., out_type, ...) runs (the shape and type
 * rules above; k and the workspaces aside), else 0.  No GPU call. */
int mq_mul_mat_q_requant_supported(int type, int out_type, int64_t m, int64_t n);

/* The gate and up projections of a gated FFN and the product between them, as one GEMM: w_image
 * holds 2 n_ff rows (the gate weight's n_ff rows, then the up weight's: the gate|up product of
 * mq_mul_mat_q), the activation is quantized with path MQ_PATH_GEMM, and y (m x n_ff, row stride
 * ldy) receives silu(gate) * up -- the values mq_quantize_act_ex(..., MQ_PRE_SILU_MUL, ...) forms
 * from that product, bit for bit -- while gate and up themselves are never written.  This is the
 * decoder FFN of src/decoder_embed.cpp:793-802 (gate and up MUL_MATs, ggml_silu, ggml_mul) before
 * its down projection.  Returns MQ_EUNSUPPORTED unless n_ff is a multiple of 64 and the product
 * has at least 512 tiles of 128 x 128 (smaller shapes run faster as mq_mul_mat_q followed by the
 * quantizer's MQ_PRE_SILU_MUL prologue). */
int mq_mul_mat_q_swiglu(int type, const void *w_image, int64_t n_ff, int64_t k, const void *workspace, int64_t m,
                        float *y, int64_t ldy, void *stream);

/* 1 when mq_mul_mat_q_swiglu(type, ..., n_ff, k, ..., m, ...) runs (the type and shape rules
 * above; k and the buffers aside), else 0.  No GPU call. */
int mq_mul_mat_q_swiglu_supported(int type, int64_t n_ff, int64_t m);

/* The q, k and v projections of an attention layer (src/crispembed.cpp:1168-1170, each with its
 * bias ADD) on one activation quantized with path MQ_PATH_GEMM, as one grouped GEMM: q (n[0]
 * features) is stored to y_q as mq_mul_mat_q_group stores it, while k and v (n[1] = n[2] =
 * n_kv_head * head_dim features) never become floats -- the GEMM stores them straight into
 * kv_frags as the attention's K/V operand fragments (the bytes mq_op_flash_attn's own K/V pass
 * writes into its workspace), ready for mq_op_flash_attn_ex(..., MQ_ATTN_KV_READY) with kv_frags
 * as its workspace.  m = B * T rows (B sequences of T tokens, T a multiple of 32), head_dim 32,
 * 64 or 128; kv_frags_bytes >= mq_op_flash_attn_workspace_bytes of the [head_dim, T, n_kv_head,
 * B] k view. */
int mq_mul_mat_q_qkv(int type, const void *const *w_images, const int64_t *n, int64_t k, const void *workspace,
                     int64_t m, float *y_q, int64_t ldy_q, const float *const *bias, int T, int head_dim,
                     int n_kv_head, void *kv_frags, size_t kv_frags_bytes, void *stream);

/* mq_quantize_act with the graph's elementwise producer folded in: it quantizes
 * op(X + bias) where bias is an fp32 [k] row added to every row of X (NULL: none) and
 * op is one of MQ_PRE_*.  The value quantized is the fp32 tensor the ggml graph
 * materialises between those nodes and the MUL_MAT:
 *   MQ_PRE_GELU_ERF: the ADD of the FFN-up bias and ggml_gelu_erf feeding the encoder's
 *     FFN-down projection (src/crispembed.cpp:1410-1416), 0.5 v (1 + erf(v / sqrt 2));
 *   MQ_PRE_SILU_MUL: ggml_silu(gate) * up feeding the decoder's FFN-down projection
 *     (src/decoder_embed.cpp:793-802), v / (1 + exp(-v)) * u, with each row of x holding
 *     the gate projection (k values) followed by the up projection (k values). */
int mq_quantize_act_ex(int type, const float *x, int64_t ldx, int64_t m, int64_t k, const float *bias, int op,
                       void *workspace, size_t workspace_bytes, int path, void *stream);

/* MQ_PRE_SILU_MUL of mq_quantize_act_ex with the gate and up projections in two tensors of one
 * row stride ld (floats): quantizes silu(gate) * up, the ggml_silu and ggml_mul nodes between a
 * gated FFN's separate gate / up MUL_MATs and its down MUL_MAT (src/decoder_embed.cpp:793-802),
 * without either node's tensor.  The bytes are those mq_quantize_act_ex(type, x, ...,
 * MQ_PRE_SILU_MUL, ...) writes for the same values side by side in x. */
int mq_quantize_act_silu_mul(int type, const float *gate, const float *up, int64_t ld, int64_t m, int64_t k,
                             void *workspace, size_t workspace_bytes, int path, void *stream);

#ifdef __cplusplus
}
#endif
#endif
