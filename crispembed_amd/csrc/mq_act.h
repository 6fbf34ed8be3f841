// mq_act.h -- device helpers shared by the activation quantizers and the GEMM's quantized
// output: fp16 conversions, ggml's GELU-erf and SiLU.  The arithmetic is written out without
// contraction (the pragma below), so every translation unit that includes it rounds each
// multiply and add on its own, as the quantizers' ISO C restatement does.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mq.h"

namespace mq {

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    const _Float16 h = (_Float16)f;  // v_cvt_f16_f32: round to nearest even, fp16 subnormals kept
    return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }

// ggml_gelu_erf (ggml-cpu vec.h, GGML_GELU_ERF): 0.5 v (1 + erf(v / sqrt 2)) in fp32
__device__ __forceinline__ float gelu_erf_f32(float v) {
#pragma clang fp contract(off)
    return 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
}

// ggml_silu(g) * u (ggml-cpu vec.h ggml_silu_f32, then GGML_OP_MUL) in fp32: g / (1 + exp(-g)), times u
__device__ __forceinline__ float silu_mul_f32(float g, float u) {
#pragma clang fp contract(off)
    return (g / (1.0f + expf(-g))) * u;
}

// Half of one Q8_0 block of a kernel's quantized output: this lane's 16 values, the other 16
// in lane l ^ 32.  The values are op(v) (pre: MQ_PRE_NONE or MQ_PRE_GELU_ERF; rows that are
// not live: zero, as the activation quantizer's pad rows), and the block is quantized as
// k_quantize_tiled<TQ_Q8_0> quantizes a row (ggml's quantize_row_q8_0 variants): the same max,
// scale, reciprocal and rounding, so the bytes equal those of the fp32 values quantized by the
// activation quantizer.  Returns the scale rounded through fp16; q receives the 16 quants.
__device__ __forceinline__ float requant_q8_0(float (&v)[16], bool live, int pre, int variant, uint4 &q) {
#pragma clang fp contract(off)
#pragma unroll
    for (int e = 0; e < 16; e++) {
        float x = v[e];
        if (pre == MQ_PRE_GELU_ERF) x = gelu_erf_f32(x);
        v[e] = live ? x : 0.f;
    }
    float amax = fabsf(v[0]);
#pragma unroll
    for (int e = 1; e < 16; e++) amax = fmaxf(amax, fabsf(v[e]));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    const float d = amax / 127.f;
    float id;
    if (variant == MQ_Q8_0_X86) id = (amax != 0.0f) ? 127.f / amax : 0.0f;
    else id = (d != 0.0f) ? 1.0f / d : 0.0f;
    uint32_t w[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        uint32_t pk = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const float t = v[4 * u + b] * id;
            float r = (variant == MQ_Q8_0_REF) ? roundf(t) : rintf(t);
            r = fminf(fmaxf(r, -128.f), 127.f);
            pk |= ((uint32_t)((int)r & 0xff)) << (8 * b);
        }
        w[u] = pk;
    }
    q = make_uint4(w[0], w[1], w[2], w[3]);
    return f16_bits_to_f32(f32_to_f16_bits(d));
}


typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// hi + lo split of two floats with one explicit rounding (round toward zero) for both
// halves: the remainder is formed from the very hi value the MFMA will read.  (A plain
// (_Float16) cast may be emitted as different conversion instructions for the operand and
// for the remainder; where their roundings disagree the split loses a 2^-11 term.)
__device__ __forceinline__ void split2(float a, float b, v2h &hi, v2h &lo) {
    hi = __builtin_bit_cast(v2h, __builtin_amdgcn_cvt_pkrtz(a, b));
    lo = __builtin_bit_cast(v2h, __builtin_amdgcn_cvt_pkrtz(a - (float)hi[0], b - (float)hi[1]));
}

__device__ __forceinline__ void split8(const float (&x)[8], v8h &hi, v8h &lo) {
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        v2h h, l;
        split2(x[j], x[j + 1], h, l);
        hi[j] = h[0], hi[j + 1] = h[1], lo[j] = l[0], lo[j + 1] = l[1];
    }
}

// fragments per 32-key block: K (NS steps) and V (2 steps x NT column tiles), hi and lo each
template <int HD>
constexpr int kv_frags() { return 2 * (HD / 16) + 4 * (HD / 32); }

}  // namespace mq
