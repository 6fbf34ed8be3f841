// mq_internal.h -- shared definitions for the gfx950 quantized mat-mul library.
//
// GGUF block formats (ggml-common.h in ggml; sizes asserted below):
//   block_q8_0 {fp16 d; int8 qs[32]}                                  34 B / 32
//   block_q4_K {fp16 d; fp16 dmin; u8 scales[12]; u8 qs[128]}         144 B / 256
//   block_q6_K {u8 ql[128]; u8 qh[64]; i8 scales[16]; fp16 d}         210 B / 256
//   block_q8_K {float d; i8 qs[256]; i16 bsums[16]}                   292 B / 256
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/mq.h"

namespace mq {

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
// Weight image: GGUF bytes, then planes (each 256-byte aligned).
//   Q8_0: qs  i8 [n][k]            d16  u16 [n][k/32]
//   Q4_K: lo  i8 [n][k]  hi i8 [n][k]   (sc_j*q4 = lo + 128*hi, lo in [0,127])
//         dw  f32 [n][k/256]  dmin f32 [n][k/256]  mins f16 [n][k/256][8]
//   Q6_K: lo  i8 [n][k]  hi i8 [n][k]   (sc*(q6-32) = lo + 128*hi)
//         dw  f32 [n][k/256]
//         ql  u8 [n][k/2]  qh u8 [n][k/4]  sc i8 [n][k/16]  d16 u16 [n][k/256]
//   F16 : no planes (the GGUF rows are already k-contiguous fp16)
// ---------------------------------------------------------------------------
struct WeightPlanes {
    size_t gguf = 0;   // bytes of the GGUF part
    size_t qs = 0;     // Q8_0 int8 plane / Q4_K,Q6_K lo limb
    size_t hi = 0;     // hi limb
    size_t dw = 0;     // f32 per-superblock d (K-quants)
    size_t dmin = 0;   // f32 per-superblock dmin (Q4_K)
    size_t mins = 0;   // f16 mins (Q4_K)
    size_t d16 = 0;    // fp16 scale plane (Q8_0 per block, Q6_K per superblock)
    size_t ql = 0, qh = 0, sc = 0;  // Q6_K streaming planes
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

inline WeightPlanes weight_planes(int type, int64_t n, int64_t k) {
    WeightPlanes p;
    p.gguf = row_size(type, k) * (size_t)n;
    size_t off = align256(p.gguf);
    const size_t nk = (size_t)n * (size_t)k;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off = align256(off + bytes);
        return o;
    };
    switch (type) {
        case MQ_TYPE_Q8_0:
            p.qs = take(nk);
            p.d16 = take(nk / QK8_0 * 2);
            break;
        case MQ_TYPE_Q4_K:
            p.qs = take(nk);
            p.hi = take(nk);
            p.dw = take(nk / QK_K * 4);
            p.dmin = take(nk / QK_K * 4);
            p.mins = take(nk / QK_K * 8 * 2);
            break;
        case MQ_TYPE_Q6_K:
            p.qs = take(nk);
            p.hi = take(nk);
            p.dw = take(nk / QK_K * 4);
            p.ql = take(nk / 2);
            p.qh = take(nk / 4);
            p.sc = take(nk / 16);
            p.d16 = take(nk / QK_K * 2);
            break;
        default: break;
    }
    p.total = (type == MQ_TYPE_F16) ? p.gguf : off;
    return p;
}

// ---------------------------------------------------------------------------
// Activation workspace (planar quantized X, m rows):
//   Q8_0: xq i8 [m][k]   xd f32 [m][k/32]      (xd holds the fp16 d widened exactly)
//   Q8_K: xq i8 [m][k]   xd f32 [m][k/256]   xbs i16 [m][k/16]  (ggml's bsums)
//   F16 : xh f16 [m][k]
// ---------------------------------------------------------------------------
struct ActPlanes {
    size_t xq = 0, xd = 0, xbs = 0, total = 0;
};

inline ActPlanes act_planes(int wtype, int64_t m, int64_t k) {
    ActPlanes a;
    const size_t mk = (size_t)m * (size_t)k;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off = align256(off + bytes);
        return o;
    };
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
            break;
        case MQ_TYPE_F16: a.xq = take(mk * 2); break;
        default: break;
    }
    a.total = off;
    return a;
}

// ---- launchers (defined in the .hip files; return hipError_t) ----
// Quantize m rows of x (stride ldx floats) into the planar workspace layout.
hipError_t launch_quantize_act_planar(int wtype, const float *x, int64_t ldx, void *ws, int64_t m, int64_t k,
                                      int q8_0_variant, hipStream_t s);
hipError_t launch_quantize_q8_0_gguf(const float *x, int64_t ldx, void *y, int64_t m, int64_t k, int variant,
                                     hipStream_t s);
hipError_t launch_quantize_q8_K_gguf(const float *x, int64_t ldx, void *y, int64_t m, int64_t k, hipStream_t s);
hipError_t launch_quantize_f16(const float *x, int64_t ldx, void *y, int64_t m, int64_t k, hipStream_t s);
hipError_t launch_dequantize(int type, const void *w, float *y, int64_t nrows, int64_t k, int fused, hipStream_t s);
hipError_t launch_weight_prepare(int type, void *image, int64_t n, int64_t k, int64_t row0, int64_t row1,
                                 hipStream_t s);
hipError_t launch_gemm(int type, const void *image, int64_t n, int64_t k, const void *ws, int64_t m, float *y,
                       int64_t ldy, hipStream_t s);
hipError_t launch_gemv(int type, const void *image, int64_t n, int64_t k, const void *ws, int64_t m, float *y,
                       int64_t ldy, hipStream_t s);

}  // namespace mq
