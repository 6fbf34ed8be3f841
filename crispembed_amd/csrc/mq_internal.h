// mq_internal.h -- shared definitions for the gfx950 quantized mat-mul library.
//
// GGUF block formats (ggml-common.h in ggml; sizes asserted below):
//   block_q8_0 {fp16 d; int8 qs[32]}                                  34 B / 32
//   block_q4_K {fp16 d; fp16 dmin; u8 scales[12]; u8 qs[128]}         144 B / 256
//   block_q6_K {u8 ql[128]; u8 qh[64]; i8 scales[16]; fp16 d}         210 B / 256
//   block_q8_K {float d; i8 qs[256]; i16 bsums[16]}                   292 B / 256
#pragma once

#include <atomic>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/mq.h"

namespace mq {

// Raises kernel fn's dynamic-LDS limit to `bytes` once per device: flags[dev] is set after a
// successful hipFuncSetAttribute (threads that race on it both set the same value).
constexpr int MQ_MAX_DEVICES = 64;
inline hipError_t dyn_lds_once(const void *fn, int bytes, std::atomic<bool> *flags) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= MQ_MAX_DEVICES) return hipErrorInvalidDevice;
    if (flags[dev].load(std::memory_order_acquire)) return hipSuccess;
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess) flags[dev].store(true, std::memory_order_release);
    return e;
}

constexpr int QK8_0 = 32;
constexpr int QK_K = 256;

#pragma pack(push, 1)
struct block_q8_0 {
    uint16_t d;
    int8_t qs[32];
};
struct block_q4_K {
    uint16_t d;
    uint16_t dmin;
    uint8_t scales[12];
    uint8_t qs[128];
};
struct block_q6_K {
    uint8_t ql[128];
    uint8_t qh[64];
    int8_t scales[16];
    uint16_t d;
};
struct block_q8_K {
    float d;
    int8_t qs[256];
    int16_t bsums[16];
};
#pragma pack(pop)
static_assert(sizeof(block_q8_0) == 34, "block_q8_0");
static_assert(sizeof(block_q4_K) == 144, "block_q4_K");
static_assert(sizeof(block_q6_K) == 210, "block_q6_K");
static_assert(sizeof(block_q8_K) == 292, "block_q8_K");

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// ---------------------------------------------------------------------------
// Tiled ("fragment-major") int8 planes, read by the MFMA GEMM.
// Rows are padded to TILE_ROWS, the K bytes of a row to KSTAGE.  The plane is a
// sequence of 1 KB fragments, one per (32-row tile rt, 32-byte K chunk kc), at
// ((rt * kb_pad/32) + kc) * 1024; inside a fragment lane l's 16 bytes hold row
// rt*32 + l%32, bytes kc*32 + 16*(l/32) .. +16 -- exactly the operand a lane
// feeds to a 32x32x32 int8 (or 32x32x16 fp16) MFMA.  A wave moves one fragment
// with one 16-byte-per-lane load, global -> LDS -> registers, all contiguous.
// ---------------------------------------------------------------------------
constexpr int TILE_ROWS = 256;
// Q4_K GEMV plane: one tile = 16 weight rows x one 256-value superblock
constexpr int GV_ROWS = 16;
constexpr int GV4_QS = 0, GV4_SC = 2048, GV4_MN = 2176, GV4_DD = 2304, GV4_BYTES = 2368;
constexpr int GV6_LO = 0, GV6_HI = 2048, GV6_SC = 3072, GV6_D = 3328, GV6_BYTES = 3360;  // = 16 GGUF blocks
constexpr int KSTAGE = 128;

__host__ __device__ inline int64_t pad_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

__host__ __device__ inline int64_t tiled_off(int64_t r, int64_t kb, int64_t kb_pad) {
    const int64_t rt = r >> 5, lr = r & 31, kc = kb >> 5, w = kb & 31;
    return ((((rt * (kb_pad >> 5) + kc) << 6) + ((w >> 4) << 5) + lr) << 4) + (w & 15);
}

// ---------------------------------------------------------------------------
// Weight image: GGUF bytes, then planes (each 256-byte aligned).
//  GEMV planes (row-major, byte-identical to the GGUF fields):
//   Q8_0: qs  i8 [n][k]            d16  u16 [n][k/32]
//   Q6_K: gv  [ceil(n/16)][k/256] tiles of GV6_BYTES (the GGUF size of 16 rows), the
//         operands of the MFMA GEMV, with v = q ^ 32 = the 6-bit two's complement of q - 32
//         (q the unsigned 6-bit quant) of value 32kk+8p+b (b < 8) of row r (K-step kk,
//         lane group p):
//           lo [kk/4][p][r][kk%4] u32: byte j = (v_j & 15) | (v_{j+4} & 15) << 4
//           hi [p][r][kk/2] u32: byte j holds (v >> 4) of v_j, v_{j+4} of step 2*(kk/2)
//              (bits 0-1, 2-3) and of step 2*(kk/2)+1 (bits 4-5, 6-7)
//           sc [g][r/4][kk][r%4] i8 = scale of 16-group 2kk+g;  d [r] f16 (the GGUF half);
//           rows past n are zero
//   Q4_K: gv  [ceil(n/16)][k/256] tiles of GV4_BYTES (16 rows x one superblock), the
//         operands of the MFMA GEMV: qs [chunk c][half h][row r][16 B] (GGUF qs bytes
//         32c+16h..+16 of row r), sc [g][r/4][c][r%4] (u8 sc_{2c+g}), mn [half][r][4]
//         (u8 m_{4*half+t}), dd [r][2] f16 (d, dmin, the GGUF halves); rows past n are zero
//   (F16 GEMVs read the GGUF rows directly)
//  GEMM planes (tiled, n padded to n_pad = pad(n, 256)):
//   Q8_0: tq  i8 tiled [n_pad][kb_pad]     tdw f32 [kb_pad/32][n_pad]
//   Q4_K: tq (lo limb), thi (hi limb) i8 tiled [n_pad][k]: sc_j*q4 = lo + 128*hi,
//         lo in [0,127], hi in [0,7]
//         tdw, tdmin f32 [k/256][n_pad]
//         tmin f16 fragments [n_pad/32][k/256][64 lanes][8]: lane l holds m_0..m_7
//         of column l%32 (both lane halves), the B operand of the min-term MFMA
//   Q6_K: tq, thi limbs of sc*(q6-32) (lo in [0,127], hi in [-32,32]); tdw
//   F16 : tq  f16 tiled [n_pad][kb_pad bytes]
// ---------------------------------------------------------------------------
struct WeightPlanes {
    size_t gguf = 0;
    size_t qs = 0, d16 = 0, gv = 0;                        // GEMV planes
    size_t tq = 0, thi = 0, tdw = 0, tdmin = 0, tmin = 0;  // GEMM planes
    int64_t n_pad = 0, kb_pad = 0;
    size_t total = 0;
};

inline int64_t blck_size(int type) {
    switch (type) {
        case MQ_TYPE_F32:
        case MQ_TYPE_F16: return 1;
        case MQ_TYPE_Q8_0: return QK8_0;
        case MQ_TYPE_Q4_K:
        case MQ_TYPE_Q6_K:
        case MQ_TYPE_Q8_K: return QK_K;
        default: return 0;
    }
}

inline size_t type_size(int type) {
    switch (type) {
        case MQ_TYPE_F32: return 4;
        case MQ_TYPE_F16: return 2;
        case MQ_TYPE_Q8_0: return sizeof(block_q8_0);
        case MQ_TYPE_Q4_K: return sizeof(block_q4_K);
        case MQ_TYPE_Q6_K: return sizeof(block_q6_K);
        case MQ_TYPE_Q8_K: return sizeof(block_q8_K);
        default: return 0;
    }
}

inline size_t row_size(int type, int64_t k) {
    const int64_t b = blck_size(type);
    return b ? (size_t)(k / b) * type_size(type) : 0;
}

// bytes of K per row in the GEMM operand planes (int8 formats: k; F16: 2k), padded
inline int64_t gemm_kb_pad(int type, int64_t k) {
    return pad_up(type == MQ_TYPE_F16 ? 2 * k : k, KSTAGE);
}

inline WeightPlanes weight_planes(int type, int64_t n, int64_t k) {
    WeightPlanes p;
    p.gguf = row_size(type, k) * (size_t)n;
    p.n_pad = pad_up(n, TILE_ROWS);
    p.kb_pad = gemm_kb_pad(type, k);
    size_t off = align256(p.gguf);
    const size_t nk = (size_t)n * (size_t)k;
    const size_t tiled = (size_t)p.n_pad * (size_t)p.kb_pad;
    const size_t nsb = (size_t)(k / QK_K);
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off = align256(off + bytes);
        return o;
    };
    switch (type) {
        case MQ_TYPE_Q8_0:
            p.qs = take(nk);
            p.d16 = take(nk / QK8_0 * 2);
            p.tq = take(tiled);
            p.tdw = take((size_t)(p.kb_pad / QK8_0) * p.n_pad * 4);
            break;
        case MQ_TYPE_Q4_K:
            p.gv = take((size_t)((n + GV_ROWS - 1) / GV_ROWS) * nsb * GV4_BYTES);
            p.tq = take(tiled);
            p.thi = take(tiled);
            p.tdw = take(nsb * p.n_pad * 4);
            p.tdmin = take(nsb * p.n_pad * 4);
            p.tmin = take((size_t)(p.n_pad / 32) * nsb * 1024);
            break;
        case MQ_TYPE_Q6_K:
            p.gv = take((size_t)((n + GV_ROWS - 1) / GV_ROWS) * nsb * GV6_BYTES);
            p.tq = take(tiled);
            p.thi = take(tiled);
            p.tdw = take(nsb * p.n_pad * 4);
            break;
        case MQ_TYPE_F16: p.tq = take(tiled); break;
        default: break;
    }
    p.total = off;
    return p;
}

// ---------------------------------------------------------------------------
// Activation workspace.
//  Row-major layout (GEMV path, m <= 8):
//   Q8_0: xq i8 [m][k]   xd f32 [m][k/32]      (xd holds the fp16 d widened exactly)
//   Q8_K: xq i8 [m][k]   xd f32 [m][k/256]   xbs i16 [m][k/16]  (ggml's bsums)
//         xgm f16 [k/256][8][16]: for row m < 8, entry e: B_{e%8} & 63 (e < 8) or
//         64*(B_{e%8} >> 6) (e >= 8), B_j = sum of the 32 quants of sub-block j:
//         the B operand of the Q4_K GEMV min-term MFMA
//   F16 : xq f16 [m][k]
//  Tiled layout (GEMM path, m padded to m_pad = pad(m, 256), pad rows zero):
//   Q8_0: xq i8 tiled [m_pad][kb_pad]   xd f32 [kb_pad/32][m_pad]
//   Q8_K: xq i8 tiled [m_pad][k]        xd f32 [k/256][m_pad]
//         xmin f16 fragments [m_pad/32][k/256][64 lanes][8]: lane l, row l%32, holds
//         B_j & 63 (lanes 0-31) or 64*(B_j >> 6) (lanes 32-63) for j = 0..7, where
//         B_j = the sum of the 32 quants of sub-block j: the A operand of the
//         min-term MFMA
//   F16 : xq f16 tiled [m_pad][kb_pad bytes]
// ---------------------------------------------------------------------------
struct ActPlanes {
    size_t xq = 0, xd = 0, xbs = 0, xmin = 0, xgm = 0, total = 0;
    int64_t m_pad = 0, kb_pad = 0;
    bool tiled = false;
};

inline ActPlanes act_planes(int wtype, int64_t m, int64_t k, bool tiled) {
    ActPlanes a;
    a.tiled = tiled;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off = align256(off + bytes);
        return o;
    };
    if (!tiled) {
        const size_t mk = (size_t)m * (size_t)k;
        a.m_pad = m;
        a.kb_pad = (wtype == MQ_TYPE_F16) ? 2 * k : k;
        switch (wtype) {
            case MQ_TYPE_Q8_0:
                a.xq = take(mk);
                a.xd = take(mk / QK8_0 * 4);
                break;
            case MQ_TYPE_Q4_K:
            case MQ_TYPE_Q6_K:
                a.xq = take(mk);
                a.xd = take(mk / QK_K * 4);
                a.xbs = take(mk / 16 * 2);
                a.xgm = take((size_t)(k / QK_K) * 8 * 16 * 2);
                break;
            case MQ_TYPE_F16: a.xq = take(mk * 2); break;
            default: break;
        }
    } else {
        a.m_pad = pad_up(m, TILE_ROWS);
        a.kb_pad = gemm_kb_pad(wtype, k);
        const size_t t = (size_t)a.m_pad * (size_t)a.kb_pad;
        const size_t nsb = (size_t)(k / QK_K);
        switch (wtype) {
            case MQ_TYPE_Q8_0:
                a.xq = take(t);
                a.xd = take((size_t)(a.kb_pad / QK8_0) * a.m_pad * 4);
                break;
            case MQ_TYPE_Q4_K:
            case MQ_TYPE_Q6_K:
                a.xq = take(t);
                a.xd = take(nsb * a.m_pad * 4);
                a.xmin = take((size_t)(a.m_pad / 32) * nsb * 1024);
                break;
            case MQ_TYPE_F16: a.xq = take(t); break;
            default: break;
        }
    }
    a.total = off;
    return a;
}

// The GEMV takes up to GEMV_MAX_M rows in launches of GEMV_CHUNK: its activation layout for m
// rows is ceil(m / 8) independent row layouts (act_planes(type, rows, k, false)) of up to 8
// rows each, chunk c at c * gemv_chunk_bytes.
constexpr int GEMV_CHUNK = 8;
constexpr int GEMV_MAX_M = 32;
inline size_t gemv_chunk_bytes(int wtype, int64_t k) { return act_planes(wtype, GEMV_CHUNK, k, false).total; }
inline size_t gemv_ws_bytes(int wtype, int64_t m, int64_t k) {
    const int64_t full = m / GEMV_CHUNK, rem = m % GEMV_CHUNK;
    return (size_t)full * gemv_chunk_bytes(wtype, k) + (rem ? act_planes(wtype, rem, k, false).total : 0);
}

inline size_t act_workspace_bytes(int wtype, int64_t m, int64_t k) {
    const size_t r = m <= GEMV_MAX_M ? gemv_ws_bytes(wtype, m, k) : 0, t = act_planes(wtype, m, k, true).total;
    return r > t ? r : t;
}

// ---- launchers (defined in the .hip files; return hipError_t) ----
// Quantize m rows of x (stride ldx floats) into the planar workspace layout.
// `pre` / `bias`: the elementwise prologue (MQ_PRE_*, bias row or NULL) applied before quantization;
// x2 (MQ_PRE_SILU_MUL, same row stride): the up projection's rows, NULL when they follow the gate
// projection's k values in each row of x.
hipError_t launch_quantize_act_planar(int wtype, const float *x, int64_t ldx, void *ws, int64_t m, int64_t k,
                                      int q8_0_variant, bool tiled, hipStream_t s, int pre = MQ_PRE_NONE,
                                      const float *bias = nullptr, const float *x2 = nullptr);
hipError_t launch_quantize_q8_0_gguf(const float *x, int64_t ldx, void *y, int64_t m, int64_t k, int variant,
                                     hipStream_t s);
hipError_t launch_quantize_q8_K_gguf(const float *x, int64_t ldx, void *y, int64_t m, int64_t k, hipStream_t s);
hipError_t launch_quantize_f16(const float *x, int64_t ldx, void *y, int64_t m, int64_t k, hipStream_t s,
                               int pre = MQ_PRE_NONE, const float *bias = nullptr, int64_t uoff = 0);
hipError_t launch_dequantize(int type, const void *w, float *y, int64_t nrows, int64_t k, int fused, hipStream_t s);
hipError_t launch_weight_prepare(int type, void *image, int64_t n, int64_t k, int64_t row0, int64_t row1,
                                 hipStream_t s);
// bias: NULL, or n floats added to every output row as it is stored
hipError_t launch_mfma_probe(int iters, int *out, int ncu, hipStream_t s);
hipError_t launch_gemm(int type, const void *image, int64_t n, int64_t k, const void *ws, int64_t m, float *y,
                       int64_t ldy, hipStream_t s, const float *bias = nullptr);
hipError_t launch_gemv(int type, const void *image, int64_t n, int64_t k, const void *ws, int64_t m, float *y,
                       int64_t ldy, hipStream_t s, const float *bias = nullptr);
// the GEMM with its output v = pre(x w^T + bias) quantized into out_ws, the GEMM-layout
// activation workspace of a following mat-mul with k = n whose weights are out_type: Q8_0
// (n a multiple of KSTAGE) or Q4_K / Q6_K (Q8_K activations: n a multiple of 256, this product's
// weights Q4_K or Q6_K, shapes gemm_requant_q8k_fits accepts); pre is MQ_PRE_NONE or
// MQ_PRE_GELU_ERF.  ws must hold x in the tiled (GEMM) layout.
bool gemm_requant_q8k_fits(int type, int64_t m, int64_t n);
// the experts' GEMM of a device-routed MUL_MAT_ID: x (m_rows rows, tiled) sorted by expert in
// segments of whole tile_rows-row tiles; moe[0] = live tiles, moe[1 + t] = expert of tile t;
// expert e's prepared weight image at images + e * stride; y gets m_rows x n floats.
// gemm_moe_tile_rows picks tile_rows (64 or 256) for rows sorted rows over n_used_experts.
int gemm_moe_tile_rows(int64_t rows, int64_t n, int n_used_experts);
hipError_t launch_gemm_moe(int type, const void *images, size_t stride, int64_t n, int64_t k, const void *ws,
                           int64_t m_rows, int tile_rows, const int *moe, float *y, hipStream_t s);
hipError_t launch_gemm_requant(int type, const void *image, int64_t n, int64_t k, const void *ws, int64_t m,
                               const float *bias, int pre, int q8_0_variant, int out_type, void *out_ws, hipStream_t s);
// the GEMM of a gated FFN's gate|up weight (2 n_ff rows: gate, then up) whose store forms
// silu(gate) * up into y (m x n_ff, row stride ldy); only for shapes gemm_swiglu_fits accepts
// (n_ff a multiple of 64, grids of the large-tile configurations)
bool gemm_swiglu_fits(int64_t m, int64_t n_ff);
hipError_t launch_gemm_swiglu(int type, const void *image, int64_t n_ff, int64_t k, const void *ws, int64_t m, float *y,
                              int64_t ldy, hipStream_t s);
// the GEMM of an attention's concatenated q|k|v projection whose K and V columns ([kv_col0,
// kv_col0 + nkv hd), then nkv hd more; n = kv_col0 + 2 nkv hd) leave as the attention's hi/lo
// fp16 operand fragments in kv_frags (the layout launch_attn's K/V pass writes, m = B T rows,
// T a multiple of 32) instead of floats; the columns before kv_col0 go to y as usual
hipError_t launch_gemm_kv(int type, const void *image, int64_t n, int64_t k, const void *ws, int64_t m, float *y,
                          int64_t ldy, const float *bias, int kv_col0, int T, int hd, int nkv, void *kv_frags,
                          hipStream_t s);
// q, k and v projections as one grouped GEMM (images / n / bias of q, k, v): q stores floats to
// yq, k and v (n[1] = n[2] = nkv hd) leave as the attention's fragments (as launch_gemm_kv)
hipError_t launch_gemm_qkv(int type, const void *const *images, const int64_t *n, int64_t k, const void *ws, int64_t m,
                           float *yq, int64_t ldyq, const float *const *bias, int T, int hd, int nkv, void *kv_frags,
                           hipStream_t s);
// xout = y + res (res may be NULL, xout may be NULL or alias), hout (NULL: not written) = rms_norm(xout) * w over
// rows of H floats, and hout quantized to Q8_K in the GEMM activation layout of a K-quant
// weight (act_planes(MQ_TYPE_Q4_K, rows, H, true)) in ws; H a multiple of 256, at most 2048
hipError_t launch_add_rmsnorm_q8_K(const float *y, const float *res, const float *w, float eps, float *xout,
                                   float *hout, int64_t rows, int H, void *ws, hipStream_t s);
// up to 3 weights of the same type and k on one activation on the GEMV path: K-quant weights at
// m <= 8 in one launch of the stream kernel over their concatenated row tiles (bit-identical to
// separate launches), otherwise one launch per weight
hipError_t launch_gemv_group(int type, int ng, const void *const *images, const int64_t *n, int64_t k, const void *ws,
                             int64_t m, float *const *y, const int64_t *ldy, const float *const *bias, hipStream_t s);
// the K-quant GEMV of up to 3 weights on fp32 activation rows (m <= 8, k <= 6144) that it
// quantizes itself -- the bytes mq_quantize_act_ex writes, so the results equal the two-step form
// bit for bit; pre MQ_PRE_NONE, or MQ_PRE_SILU_MUL with x2 the up-projection rows
bool gemv_fused_ok(int type, int ng, int64_t k, int64_t m);
hipError_t launch_gemv_group_f32(int type, int ng, const void *const *images, const int64_t *n, int64_t k,
                                 const float *x, int64_t ldx, const float *x2, int64_t ldx2, int pre, int64_t m,
                                 float *const *y, const int64_t *ldy, const float *const *bias, hipStream_t s);
// up to 4 weights of the same type and k on one activation, one launch (bias may be NULL)
hipError_t launch_gemm_group(int type, int ngroups, const void *const *images, const int64_t *n, int64_t k,
                             const void *ws, int64_t m, float *const *y, const int64_t *ldy, const float *const *bias,
                             hipStream_t s);

// Operands of the fragment attention (mq_decoder.hip).  Element (b, t, h, d) of q is at
// q + b*q_sb + t*q_st + h*q_sh + d (floats; q_sb, q_st, q_sh multiples of 4 and q 16-byte
// aligned), likewise k, v (any float strides) and out; mask element (b, h, query, key) is at
// mask + b*m_sb + h*m_sh + query*m_sq + key (fp16 bits; NULL: no mask).  Query head h reads
// key/value head h / (nq / nkv).  qw / kw: per-head RMS norm weights applied at load (NULL:
// none); cs: RoPE table of max(Tq, Tk) positions (NULL: no rotation); ws: attn_workspace_bytes
// of 16-byte aligned device memory.
struct AttnArgs {
    const float *q = nullptr, *k = nullptr, *v = nullptr;
    float *out = nullptr;
    int64_t q_sb = 0, q_st = 0, q_sh = 0, k_sb = 0, k_st = 0, k_sh = 0, v_sb = 0, v_st = 0, v_sh = 0;
    int64_t o_sb = 0, o_st = 0, o_sh = 0;
    const uint16_t *mask = nullptr;
    int64_t m_sb = 0, m_sh = 0, m_sq = 0;
    bool m_al = false;  // mask pointer 16-byte aligned, m_sb / m_sh / m_sq multiples of 8
    // the mask's block lists (launch_mask_blocks; NULL: the attention classifies the mask's
    // blocks itself): list (mask plane bm, query tile qt) at blist + (bm * bl_nqt + qt) * bl_stride
    const uint32_t *blist = nullptr;
    int bl_nqt = 0, bl_stride = 0;
    int B = 0, Tq = 0, Tk = 0, nq = 0, nkv = 0, hd = 0;
    float scale = 1.0f;
    int causal = 0;
    const float *qw = nullptr, *kw = nullptr;
    float eps = 0.f;
    const float2 *cs = nullptr;
    int64_t cs_sb = 0;  // float2 entries between the angle tables of batch elements (0: shared)
    void *ws = nullptr;
    // q_ws not NULL: the output rows (B * Tq rows of K = nq * hd values; out must hold them as
    // dense rows) also quantized into the GEMM activation workspace q_ws of the projection that
    // reads them, a weight of type q_type: Q8_0 (rounding variant q_var; K a multiple of 128),
    // or Q8_K for a K-quant weight (K a multiple of 256).  launch_attn fills qo, qd, qmin,
    // q_m_pad, q_kch and q_nsb from it.
    void *q_ws = nullptr;
    int q_var = 0;
    int q_type = MQ_TYPE_Q8_0;
    // with q_ws: the 8-wave kernel stores only the quantized rows, not the floats in out (the
    // caller reads the result quantized only; the split-key form still writes out)
    bool q_only = false;
    // the K/V operand fragments are already in ws (written by launch_gemm_kv): no K/V pass
    bool kv_ready = false;
    int8_t *qo = nullptr;
    float *qd = nullptr;
    _Float16 *qmin = nullptr;  // Q8_K: the min-term fragments
    int64_t q_m_pad = 0;
    int q_kch = 0, q_nsb = 0;
};
size_t attn_workspace_bytes(int B, int Tk, int nkv, int hd);
hipError_t launch_attn(const AttnArgs &a, hipStream_t s);
// true when launch_attn takes the split-key kernel for these operands (the form that reads
// mask block lists); a.mask, a.m_sh and the shape fields are what it looks at
bool attn_split_form(const AttnArgs &a);
// Block lists of a mask shared by every head (m_sh = 0) for the split-key attention: for each
// of Bm mask planes (m_sb apart) and each tile of 32 query rows, one list of 1 + nkb words
// (nkb = ceil(Tk / 32)): the count n, then the n key blocks of 32 keys in which some row of the
// tile has a finite mask value, in increasing order, each as kb | 1 << 31 when some value is not
// zero (the block adds the mask; else it runs unmasked).  Rows past Tq repeat row Tq - 1; keys
// past Tk are not read.  The same classification the attention makes when it has no list.
size_t mask_blocks_bytes(int Bm, int Tq, int Tk);
hipError_t launch_mask_blocks(const uint16_t *mask, int64_t m_sq, int64_t m_sb, bool m_al, int Bm, int Tq, int Tk,
                              uint32_t *blocks, hipStream_t s);
// For each of the T rows of a T x T mask (row stride m_sq halves): first[r] = the first key of the
// run of zeros that ends at key r when the row is exactly that (0 on keys first..r, -inf on every
// other key), else -1.
hipError_t launch_mask_rows(const uint16_t *mask, int64_t m_sq, bool m_al, int T, int32_t *first, hipStream_t s);
// *nonzero = 1 when any value of the Tq x Tk region of each (ne2 x ne3) plane of an F16 mask is not
// +-0 (row stride m_sq, plane strides m_s2, m_s3, in halves); *nonzero is left alone otherwise
hipError_t launch_mask_nonzero(const uint16_t *mask, int64_t m_sq, int64_t m_s2, int64_t m_s3, int ne2, int ne3, int Tq,
                               int Tk, int *nonzero, hipStream_t s);

}  // namespace mq
