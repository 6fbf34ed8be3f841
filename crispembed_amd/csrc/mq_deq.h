// mq_deq.h -- one element of a GGUF row as ggml's dequantize_row_* computes it (device code,
// shared by the dequantizer and get_rows).  The translation units that include it are built
// with -ffp-contract=off, so d1 * q - m1 of Q4_K rounds twice unless FUSED asks for the fused
// multiply-add an FMA-contracting host build of ggml performs.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mq_internal.h"

namespace mq {

__device__ __forceinline__ float deq_f16(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }

// 6-bit scale and min j of a Q4_K superblock (ggml's get_scale_min_k4)
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t *q, int &sc, int &mn) {
    if (j < 4) {
        sc = q[j] & 63;
        mn = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

template <int TYPE>
__host__ __device__ constexpr size_t deq_row_bytes(int64_t k) {
    return TYPE == MQ_TYPE_F32    ? (size_t)k * 4
           : TYPE == MQ_TYPE_F16  ? (size_t)k * 2
           : TYPE == MQ_TYPE_Q8_0 ? (size_t)(k / QK8_0) * sizeof(block_q8_0)
           : TYPE == MQ_TYPE_Q4_K ? (size_t)(k / QK_K) * sizeof(block_q4_K)
           : TYPE == MQ_TYPE_Q6_K ? (size_t)(k / QK_K) * sizeof(block_q6_K)
                                  : (size_t)(k / QK_K) * sizeof(block_q8_K);
}

// element col of the row at r
template <int TYPE, bool FUSED = false>
__device__ __forceinline__ float deq_elem(const uint8_t *r, int64_t col) {
    if constexpr (TYPE == MQ_TYPE_F32) {
        return ((const float *)r)[col];
    } else if constexpr (TYPE == MQ_TYPE_F16) {
        return deq_f16(((const uint16_t *)r)[col]);
    } else if constexpr (TYPE == MQ_TYPE_Q8_0) {
        const uint8_t *b = r + (col / QK8_0) * sizeof(block_q8_0);
        const float d = deq_f16(*(const uint16_t *)b);
        return (float)(int8_t)b[2 + col % QK8_0] * d;
    } else if constexpr (TYPE == MQ_TYPE_Q4_K) {
        const uint8_t *b = r + (col / QK_K) * sizeof(block_q4_K);
        const int e = (int)(col % QK_K);
        const int c64 = e >> 6, w64 = e & 63;
        const uint8_t byte = b[16 + 32 * c64 + (w64 & 31)];
        const int qv = (w64 < 32) ? (byte & 0xF) : (byte >> 4);
        int sc, mn;
        scale_min_k4(e >> 5, b + 4, sc, mn);
        const float d = deq_f16(*(const uint16_t *)b);
        const float dmin = deq_f16(*(const uint16_t *)(b + 2));
        const float d1 = d * (float)sc;
        const float m1 = dmin * (float)mn;
        return FUSED ? __builtin_fmaf(d1, (float)qv, -m1) : d1 * (float)qv - m1;
    } else if constexpr (TYPE == MQ_TYPE_Q6_K) {
        const uint8_t *b = r + (col / QK_K) * sizeof(block_q6_K);
        const int e = (int)(col % QK_K);
        const int h = e >> 7, rr = e & 127, g = rr >> 5, l = rr & 31;
        const uint8_t qlb = b[64 * h + l + (g & 1) * 32];
        const int nib = (g < 2) ? (qlb & 0xF) : (qlb >> 4);
        const int hb = (b[128 + 32 * h + l] >> (2 * g)) & 3;
        const int qv = (nib | (hb << 4)) - 32;
        const int8_t sc = (int8_t)b[192 + 8 * h + (l >> 4) + 2 * g];
        const float d = deq_f16(*(const uint16_t *)(b + 208));
        return d * (float)sc * (float)qv;
    } else {  // Q8_K
        const uint8_t *b = r + (col / QK_K) * sizeof(block_q8_K);
        return *(const float *)b * (float)(int8_t)b[4 + col % QK_K];
    }
}

}  // namespace mq
