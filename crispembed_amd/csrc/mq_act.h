// mq_act.h -- device helpers shared by the activation quantizers and the GEMM's quantized
// output: fp16 conversions and ggml's GELU-erf.  The arithmetic is written out without
// contraction (the pragma below), so every translation unit that includes it rounds each
// multiply and add on its own, as the quantizers' ISO C restatement does.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

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

}  // namespace mq
