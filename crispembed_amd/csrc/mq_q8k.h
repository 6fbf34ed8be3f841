// mq_q8k.h -- ggml's Q8_K row quantization (quantize_row_q8_K) of one 256-value superblock by
// one wave, shared by the activation quantizers and the producers that store their output as
// the Q8_K activation of the next mat-mul.  No contraction (the pragma below): the multiplies
// and divisions round on their own, as the quantizers' ISO C restatement does.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mq_wave.h"

namespace mq {

// ggml's nearest_int: (f + 1.5*2^23) keeps round-half-even(f) in the low mantissa bits.
__device__ __forceinline__ int nearest_int(float f) {
#pragma clang fp contract(off)
    const float v = f + 12582912.f;
    return (__float_as_int(v) & 0x007fffff) - 0x00400000;
}

// The four int8 values a, b, c, d (each in [-128, 127]) as one little-endian word (byte selects).
__device__ __forceinline__ uint32_t pack4_i8(int a, int b, int c, int d) {
    const uint32_t ab = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0c0c0400u);  // a.b0, b.b0, 0, 0
    const uint32_t cd = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x04000c0cu);  // 0, 0, c.b0, d.b0
    return ab | cd;
}

// The sum of the four signed bytes of w.
__device__ __forceinline__ int sum4_i8(uint32_t w) { return __builtin_amdgcn_sdot4((int)w, 0x01010101, 0, false); }

// The lane's largest |x| of its 4 values, and the first value (in order) with that magnitude.
__device__ __forceinline__ void first_absmax4(const float (&x)[4], float &la, float &lm) {
    la = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
    lm = fabsf(x[2]) == la ? x[2] : x[3];
    lm = fabsf(x[1]) == la ? x[1] : lm;
    lm = fabsf(x[0]) == la ? x[0] : lm;
}

// nearest_int for the quantizers' |f| <= 127.0001: round half to even, as the magic-number add
// (f + 1.5*2^23 in the default rounding mode) does for every |f| < 2^22.
__device__ __forceinline__ int round_even_i(float f) { return (int)rintf(f); }

// DPP steps inside each 16-lane row (quad_perm [1,0,3,2] = xor 1, quad_perm [2,3,0,1] = xor 2,
// row_half_mirror = i <-> 7-i within 8 lanes): after the three, every lane holds the
// combination over its 8-lane group.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float max8(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    return fmaxf(v, dpp_f<0x141>(v));
}
__device__ __forceinline__ int sum8(int v) {
    v += dpp_i<0xB1>(v);
    v += dpp_i<0x4E>(v);
    return v + dpp_i<0x141>(v);
}

// One 256-value Q8_K block of row r of a 32-row tile, lane l of the wave holding values
// 4l .. 4l + 3 (quantize_row_q8_K).  ggml's max: the FIRST value of largest magnitude -- per
// lane, the first of its 4 values with the lane's largest |x|; then the lowest lane that holds
// the wave's largest |x|.  The lane's 4 quants go to dst (its place in the fragment: LDS
// staging or the workspace itself), the scale 1 / iscale to *dslot (lane 0), and B_j (the sum
// of the 32 quants of sub-block j, split as B_j & 63 and 64 (B_j >> 6)) to the min-term
// fragment msh of the tile.
__device__ __forceinline__ void q8_K_block_row(const float4 v, int lane, int r, int8_t *dst, float *dslot,
                                               _Float16 *msh) {
#pragma clang fp contract(off)
    const float vals[4] = {v.x, v.y, v.z, v.w};
    float la, lm;
    first_absmax4(vals, la, lm);
    const float amax = wave_max_f(la);
    uint32_t packed = 0;
    int s16 = 0;
    float dval = 0.0f;
    if (amax != 0.0f) {
        const unsigned long long hit = __ballot(la == amax);
        const float mx = lane_f(lm, __ffsll((long long)hit) - 1);
        const float iscale = -127.f / mx;
        int qv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) qv[i] = min(round_even_i(iscale * vals[i]), 127);
        packed = pack4_i8(qv[0], qv[1], qv[2], qv[3]);
        s16 = sum4_i8(packed);
        dval = 1.0f / iscale;
    }
    *(uint32_t *)dst = packed;
    if (lane == 0) *dslot = dval;
    // B_j lands in lane 8j
    const int B = sum8(s16);
    if ((lane & 7) == 0) {
        const int j = lane >> 3;
        msh[(r << 3) + j] = (_Float16)(B & 63);
        msh[((32 + r) << 3) + j] = (_Float16)((B >> 6) * 64);
    }
}

// q8_K_block_row's arithmetic for NR rows of a wave at once, without the stores (row i's values
// in v[i], lane l holding values 4l .. 4l + 3): the lane's 4 quants of row i in q[i], B_j (the sum
// of sub-block j's 32 quants) in lane 8j of bs[i], the scale 1 / iscale in d[i] (wave-uniform).
// The NR scales' two divisions (-127 / max and 1 / iscale, wave-uniform values) run once for all
// rows -- row i's operand in lane i -- instead of once per row, which was a quarter of the row's
// instructions.  Bit for bit q8_K_block_row's results.
template <int NR>
__device__ __forceinline__ void q8_K_rows(const float4 *v, int lane, uint32_t *q, int *bs, float *d) {
#pragma clang fp contract(off)
    static_assert(NR >= 1 && NR <= 64, "rows per wave");
    float amax[NR], mx[NR];
#pragma unroll
    for (int i = 0; i < NR; i++) {
        const float vals[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
        float la, lm;
        first_absmax4(vals, la, lm);
        amax[i] = wave_max_f(la);
        const unsigned long long hit = __ballot(la == amax[i]);
        mx[i] = amax[i] != 0.0f ? lane_f(lm, __ffsll((long long)hit) - 1) : 1.0f;
    }
    float m = 1.0f;
#pragma unroll
    for (int i = 0; i < NR; i++) m = lane == i ? mx[i] : m;
    const float is_l = -127.f / m, d_l = 1.0f / is_l;
#pragma unroll
    for (int i = 0; i < NR; i++) {
        const float vals[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
        uint32_t packed = 0;
        int s16 = 0;
        float dval = 0.0f;
        if (amax[i] != 0.0f) {
            const float iscale = lane_f(is_l, i);
            int qv[4];
#pragma unroll
            for (int e = 0; e < 4; e++) qv[e] = min(round_even_i(iscale * vals[e]), 127);
            packed = pack4_i8(qv[0], qv[1], qv[2], qv[3]);
            s16 = sum4_i8(packed);
            dval = lane_f(d_l, i);
        }
        q[i] = packed;
        bs[i] = sum8(s16);
        d[i] = dval;
    }
}

// q8_K_rows with q8_K_block_row's stores: row i's place in the fragment dst[i], its scale slot
// dslot[i], its tile row r[i].
template <int NR>
__device__ __forceinline__ void q8_K_block_rows(const float4 *v, int lane, const int *r, int8_t *const *dst,
                                                float *const *dslot, _Float16 *msh) {
    uint32_t q[NR];
    int bs[NR];
    float d[NR];
    q8_K_rows<NR>(v, lane, q, bs, d);
#pragma unroll
    for (int i = 0; i < NR; i++) {
        *(uint32_t *)dst[i] = q[i];
        if (lane == 0) *dslot[i] = d[i];
        if ((lane & 7) == 0) {
            const int j = lane >> 3;
            msh[(r[i] << 3) + j] = (_Float16)(bs[i] & 63);
            msh[((32 + r[i]) << 3) + j] = (_Float16)((bs[i] >> 6) * 64);
        }
    }
}

}  // namespace mq
