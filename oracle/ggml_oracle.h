/*
 * ggml_oracle.h -- CPU restatement of ggml's block-quantized MUL_MAT semantics.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: the pytest suite, the
 * package smoke check and bench.py's cpu_baseline leg load it.  Nothing in the
 * shipped path (crispembed_amd/, include/) links or calls it.
 *
 * The arithmetic restated here lives in the ggml git submodule of CrispEmbed
 * (.gitmodules:1-4, fork pin 890278a8 per HISTORY.md:394), which is not vendored
 * in the reference tree.  The functions follow ggml's published algorithms
 * (ggml-quants.c / ggml-cpu quants.c, MIT licence) as restated in prose; the
 * call sites in the reference that reach them are:
 *   - weight quantization: ggml_quantize_chunk, tools/quantize.cpp:804-805
 *   - activation requantization inside CPU mul_mat: LEARNINGS.md:4826-4830
 *   - MUL_MAT graph nodes: src/crispembed.cpp:1168-1170,1300,1410,1416,
 *     src/decoder_embed.cpp:724-802, src/qwen2vl_ocr.cpp:2368-2452
 *   - dequantization (to_float): src/core/cpu_ops.h:63-65
 *
 * Floating-point contract: the library is compiled with -ffp-contract=off, so
 * every a*b+c below rounds twice, as ISO C without contraction does.
 *
 * Parity status per function (what pins it is in tests/test_oracle_*.py):
 *   fp16 conversion              pinned (numpy float16, exhaustive fp16 decode)
 *   nearest_int                  pinned (numpy.rint on ties and random values)
 *   quantize_row_q8_0 (3 variants) pinned (closed-form invariants, crafted ties)
 *   quantize_row_q8_K            pinned (closed form, invariants, crafted ties)
 *   dequantize q8_0/q4_K/q6_K/f16  pinned (independent packer round trips,
 *                                exhaustive scale/min unpacking)
 *   vec_dot_* and mul_mat        pinned (fp64 integer-exact product in numpy)
 *   quantize_row_q4_K_ref        pinned: the sub-block search against its definition (its
 *                                error equals the best candidate's, float64), idempotence on
 *                                representable superblocks, and the whole row's bytes against a
 *                                float64 restatement of the published wrapper (weights, search
 *                                parameters, 6-bit codes, level recomputation): identical
 *                                superblocks but for fp32 / float64 rounding ties (< 5 %); planted
 *                                mistakes in the search and at its call site fail them
 *   quantize_row_q6_K_ref        pinned: the search as an argmax over its candidates,
 *                                idempotence on representable superblocks, planted mistakes
 */
#ifndef GGML_ORACLE_H
#define GGML_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (also the GGUF on-disk ids). */
enum {
    OR_TYPE_F32  = 0,
    OR_TYPE_F16  = 1,
    OR_TYPE_Q8_0 = 8,
    OR_TYPE_Q4_K = 12,
    OR_TYPE_Q6_K = 14,
    OR_TYPE_Q8_K = 15,
};

/* Activation quantizer variants for Q8_0 (ggml-cpu picks one per host ISA):
 *   X86  : id = 127/amax, round-half-even  (AVX/AVX2/AVX-512 path)
 *   NEON : id = 1/(amax/127), round-half-even
 *   REF  : id = 1/(amax/127), roundf (half away from zero) -- quantize_row_q8_0_ref */
enum { OR_Q8_0_X86 = 0, OR_Q8_0_NEON = 1, OR_Q8_0_REF = 2 };

#define OR_QK8_0 32
#define OR_QK_K 256

#pragma pack(push, 1)
typedef struct { uint16_t d; int8_t qs[32]; } or_block_q8_0;                        /* 34 B  */
typedef struct { uint16_t d; uint16_t dmin; uint8_t scales[12]; uint8_t qs[128]; } or_block_q4_K; /* 144 B */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } or_block_q6_K; /* 210 B */
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } or_block_q8_K;       /* 292 B */
#pragma pack(pop)

/* ---- scalar helpers ---- */
uint16_t or_fp32_to_fp16(float f);
float    or_fp16_to_fp32(uint16_t h);
int      or_nearest_int(float f);
void     or_get_scale_min_k4(int j, const uint8_t *scales, uint8_t *sc, uint8_t *m);

/* ---- type traits ---- */
int64_t or_blck_size(int type);
size_t  or_type_size(int type);
size_t  or_row_size(int type, int64_t k);
int     or_vec_dot_type(int type);

/* ---- quantizers (one row of k values) ---- */
void or_quantize_row_q8_0_ref(const float *x, void *y, int64_t k);
void or_quantize_row_q8_0_act(const float *x, void *y, int64_t k, int variant);
void or_quantize_row_q8_K(const float *x, void *y, int64_t k);
void or_quantize_row_q4_K_ref(const float *x, void *y, int64_t k);
void or_quantize_row_q6_K_ref(const float *x, void *y, int64_t k);
void or_quantize_row_f16(const float *x, void *y, int64_t k);

/* The sub-block searches of the K-quant weight quantizers, exposed for the tests that pin them:
 * make_qkx2_quants (Q4_K: returns the scale, *the_min = -min, levels L in [0, nmax]) and
 * make_qx_quants with rmse_type 1 (Q6_K: returns the scale, L = level + nmax). */
float or_make_qkx2_quants(int n, int nmax, const float *x, const float *weights, uint8_t *L, float *the_min,
                          float rmin, float rdelta, int nstep);
float or_make_qx_quants(int n, int nmax, const float *x, int8_t *L);

/* Planted mistakes for the tests that show the pins above catch them (0: none). */
#define OR_MUT_NONE 0
#define OR_MUT_Q4K_NO_SEARCH 1 /* make_qkx2_quants without its refit search (nstep 0) */
#define OR_MUT_Q4K_RDELTA 2    /* the search steps by 0.2 instead of 0.1 */
#define OR_MUT_Q4K_PACK 3      /* the high bits of sub-blocks 4-7's scale and min swapped */
#define OR_MUT_Q6K_NO_SEARCH 4 /* make_qx_quants without its +-9 search */
#define OR_MUT_Q6K_STEP 5      /* the search steps by 0.2 instead of 0.1 */
#define OR_MUT_Q6K_ISCALE 6    /* the 8-bit scales against 127 instead of 128 */
/* mistakes at quantize_row_q4_K_ref's call of make_qkx2_quants (the search itself intact) */
#define OR_MUT_Q4K_CALL_NSTEP0 7       /* nstep 0: no refits */
#define OR_MUT_Q4K_CALL_UNIT_WEIGHTS 8 /* weights 1 instead of av_x + |x| */
#define OR_MUT_Q4K_CALL_RMIN 9         /* rmin -0.5 instead of -1 */
void or_set_mutation(int m);
/* ggml_quantize_chunk(type, src, dst, 0, nrows, k, NULL): weight quantization. */
size_t or_quantize_chunk(int type, const float *src, void *dst, int64_t nrows, int64_t k);

/* ---- dequantizers; fused=1 evaluates Q4_K's d1*q - m1 as one fma ---- */
void or_dequantize_row(int type, const void *x, float *y, int64_t k, int fused);

/* ---- activation requantization (src1 -> vec_dot_type), rows of k ---- */
void or_quantize_act_rows(int wtype, const float *x, int64_t ldx, void *xq, int64_t m, int64_t k,
                          int q8_0_variant);

/* ---- block dots (ggml's portable C accumulation order) ---- */
float or_vec_dot(int wtype, int64_t k, const void *w_row, const void *xq_row);

/* ---- mul_mat: y[m*ldy + n] = sum_k W[n,k] * X[m,k] with ggml CPU semantics ---- */
void or_mul_mat(int wtype, const void *w, int64_t n, int64_t k, const float *x, int64_t ldx, int64_t m,
                float *y, int64_t ldy, int nthreads, int q8_0_variant);
/* mul_mat from already-quantized activations (xq in vec_dot_type rows). */
void or_mul_mat_q(int wtype, const void *w, int64_t n, int64_t k, const void *xq, int64_t m, float *y,
                  int64_t ldy, int nthreads);
/* fp64 product of the quantized operands: integer block sums, fp64 scaling. */
void or_mul_mat_exact(int wtype, const void *w, int64_t n, int64_t k, const void *xq, int64_t m, double *y);

/* ---- CPU baseline (cpu_fast.c): the same mul_mat with AVX2 integer dots and threads ---- */
int or_fast_supported(int wtype);
const char *or_fast_isa(void);
int or_fast_mul_mat(int wtype, const void *w, int64_t n, int64_t k, const float *x, int64_t ldx, int64_t m, float *y,
                    int64_t ldy, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
