// mq_quant.hip -- activation quantization, dequantization and weight-plane
// preparation kernels for gfx950.
//
// This file is compiled with -ffp-contract=off: every multiply and add below
// rounds on its own, which is what ggml's CPU code computes when its compiler
// does not contract (the restated semantics).  Division is IEEE correctly
// rounded (-fhip-fp32-correctly-rounded-divide-sqrt), like x86 divss.
//
// Layout of work: quantization is HBM-bound byte work, so the kernels are
// plain coalesced streams -- 8 lanes per 32-value Q8_0 block (one float4 each,
// a 3-step xor-shuffle max), one wave per 256-value Q8_K block (a 6-step
// shuffle reduction of the (|x|, index) pair).
#include "mq_internal.h"

namespace mq {

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    const _Float16 h = (_Float16)f;  // v_cvt_f16_f32: round to nearest even, fp16 subnormals kept
    return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }

// ggml's nearest_int: (f + 1.5*2^23) keeps round-half-even(f) in the low mantissa bits.
__device__ __forceinline__ int nearest_int(float f) {
    const float v = f + 12582912.f;
    return (__float_as_int(v) & 0x007fffff) - 0x00400000;
}

template <bool VEC4>
__device__ __forceinline__ float4 load4(const float *p) {
    if (VEC4) return *(const float4 *)p;
    return make_float4(p[0], p[1], p[2], p[3]);
}

// ---------------------------------------------------------------------------
// Q8_0 activations: quantize_row_q8_0 (variant selects the rounding).
// Lanes 8g..8g+7 of a wave own one 32-value block.
// PLANAR: xq int8 [m][k] + xd float [m][k/32]; else GGUF block_q8_0 rows.
// ---------------------------------------------------------------------------
template <int VARIANT, bool PLANAR, bool VEC4>
__global__ __launch_bounds__(256) void k_quantize_q8_0(const float *__restrict__ x, int64_t ldx,
                                                       int8_t *__restrict__ out, float *__restrict__ xd,
                                                       int64_t m, int64_t k) {
    const int64_t nbr = k / QK8_0;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t blk = gid >> 3;
    const int sub = (int)(gid & 7);
    if (blk >= m * nbr) return;  // 8-lane groups leave together
    const int64_t row = blk / nbr, b = blk - row * nbr;
    const float4 v = load4<VEC4>(x + row * ldx + b * QK8_0 + sub * 4);
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 8));
    const float d = amax / 127.f;
    float id;
    if (VARIANT == MQ_Q8_0_X86) id = (amax != 0.0f) ? 127.f / amax : 0.0f;
    else id = (d != 0.0f) ? 1.0f / d : 0.0f;
    auto q = [&](float xv) -> uint32_t {
        const float t = xv * id;
        float r = (VARIANT == MQ_Q8_0_REF) ? roundf(t) : rintf(t);
        r = fminf(fmaxf(r, -128.f), 127.f);
        return (uint32_t)((int)r & 0xff);
    };
    const uint32_t packed = q(v.x) | (q(v.y) << 8) | (q(v.z) << 16) | (q(v.w) << 24);
    const uint16_t dh = f32_to_f16_bits(d);
    if (PLANAR) {
        *(uint32_t *)(out + row * k + b * QK8_0 + sub * 4) = packed;
        if (sub == 0) xd[row * nbr + b] = f16_bits_to_f32(dh);
    } else {
        uint8_t *blkp = (uint8_t *)out + (row * nbr + b) * sizeof(block_q8_0);
        uint16_t *qs16 = (uint16_t *)(blkp + 2 + sub * 4);  // 2-byte aligned in the 34-byte block
        qs16[0] = (uint16_t)(packed & 0xffff);
        qs16[1] = (uint16_t)(packed >> 16);
        if (sub == 0) *(uint16_t *)blkp = dh;
    }
}

// ---------------------------------------------------------------------------
// Q8_K activations: quantize_row_q8_K.  One wave per 256-value block; lane l
// owns values 4l..4l+3.  max is the FIRST value of largest magnitude: the
// reduction orders (|x| descending, index ascending).
// PLANAR: xq int8 [m][k], xd float [m][k/256], xbs int16 [m][k/16].
// ---------------------------------------------------------------------------
template <bool PLANAR, bool VEC4>
__global__ __launch_bounds__(256) void k_quantize_q8_K(const float *__restrict__ x, int64_t ldx,
                                                       int8_t *__restrict__ out, float *__restrict__ xd,
                                                       int16_t *__restrict__ xbs, int64_t m, int64_t k) {
    const int64_t nbr = k / QK_K;
    const int lane = threadIdx.x & 63;
    const int64_t blk = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (blk >= m * nbr) return;  // whole waves leave together
    const int64_t row = blk / nbr, b = blk - row * nbr;
    const float4 v = load4<VEC4>(x + row * ldx + b * QK_K + lane * 4);
    const float vals[4] = {v.x, v.y, v.z, v.w};
    float amax = 0.0f, mx = 0.0f;
    int idx = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float ax = fabsf(vals[i]);
        if (ax > amax) {
            amax = ax;
            mx = vals[i];
            idx = lane * 4 + i;
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float oa = __shfl_xor(amax, off);
        const float om = __shfl_xor(mx, off);
        const int oi = __shfl_xor(idx, off);
        if (oa > amax || (oa == amax && oi < idx)) {
            amax = oa;
            mx = om;
            idx = oi;
        }
    }
    uint32_t packed = 0;
    int s16 = 0;
    float dval = 0.0f;
    if (amax != 0.0f) {
        const float iscale = -127.f / mx;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int qv = nearest_int(iscale * vals[i]);
            qv = qv < 127 ? qv : 127;
            packed |= (uint32_t)(qv & 0xff) << (8 * i);
            s16 += qv;
        }
        dval = 1.0f / iscale;
    }
    s16 += __shfl_xor(s16, 1);
    s16 += __shfl_xor(s16, 2);
    if (PLANAR) {
        *(uint32_t *)(out + row * k + b * QK_K + lane * 4) = packed;
        if ((lane & 3) == 0) xbs[row * (k / 16) + b * 16 + (lane >> 2)] = (int16_t)s16;
        if (lane == 0) xd[row * nbr + b] = dval;
    } else {
        uint8_t *blkp = (uint8_t *)out + (row * nbr + b) * sizeof(block_q8_K);
        *(uint32_t *)(blkp + 4 + lane * 4) = packed;
        if ((lane & 3) == 0) *(int16_t *)(blkp + 260 + 2 * (lane >> 2)) = (int16_t)s16;
        if (lane == 0) *(float *)blkp = dval;
    }
}

// fp32 -> fp16 (round to nearest even), 4 values per lane.
template <bool VEC4>
__global__ __launch_bounds__(256) void k_quantize_f16(const float *__restrict__ x, int64_t ldx,
                                                      uint16_t *__restrict__ y, int64_t m, int64_t k) {
    const int64_t q4 = k / 4;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= m * q4) return;
    const int64_t row = gid / q4, c = gid - row * q4;
    const float4 v = load4<VEC4>(x + row * ldx + c * 4);
    uint16_t *o = y + row * k + c * 4;
    o[0] = f32_to_f16_bits(v.x);
    o[1] = f32_to_f16_bits(v.y);
    o[2] = f32_to_f16_bits(v.z);
    o[3] = f32_to_f16_bits(v.w);
}

// ---------------------------------------------------------------------------
// Dequantization (ggml to_float), one thread per output value.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t *q, int &sc, int &mn) {
    if (j < 4) {
        sc = q[j] & 63;
        mn = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

template <int TYPE, bool FUSED>
__global__ __launch_bounds__(256) void k_dequantize(const uint8_t *__restrict__ w, float *__restrict__ y,
                                                    int64_t nrows, int64_t k) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= nrows * k) return;
    const int64_t row = gid / k, col = gid - row * k;
    const size_t rs = (TYPE == MQ_TYPE_F16) ? (size_t)k * 2
                                             : (size_t)(k / (TYPE == MQ_TYPE_Q8_0 ? QK8_0 : QK_K)) *
                                                   (TYPE == MQ_TYPE_Q8_0   ? sizeof(block_q8_0)
                                                    : TYPE == MQ_TYPE_Q4_K ? sizeof(block_q4_K)
                                                    : TYPE == MQ_TYPE_Q6_K ? sizeof(block_q6_K)
                                                                           : sizeof(block_q8_K));
    const uint8_t *r = w + row * rs;
    float out = 0.0f;
    if (TYPE == MQ_TYPE_F16) {
        out = f16_bits_to_f32(((const uint16_t *)r)[col]);
    } else if (TYPE == MQ_TYPE_Q8_0) {
        const uint8_t *b = r + (col / QK8_0) * sizeof(block_q8_0);
        const float d = f16_bits_to_f32(*(const uint16_t *)b);
        out = (float)(int8_t)b[2 + col % QK8_0] * d;
    } else if (TYPE == MQ_TYPE_Q4_K) {
        const uint8_t *b = r + (col / QK_K) * sizeof(block_q4_K);
        const int e = (int)(col % QK_K);
        const int c64 = e >> 6, w64 = e & 63;
        const uint8_t byte = b[16 + 32 * c64 + (w64 & 31)];
        const int qv = (w64 < 32) ? (byte & 0xF) : (byte >> 4);
        int sc, mn;
        scale_min_k4(e >> 5, b + 4, sc, mn);
        const float d = f16_bits_to_f32(*(const uint16_t *)b);
        const float dmin = f16_bits_to_f32(*(const uint16_t *)(b + 2));
        const float d1 = d * (float)sc;
        const float m1 = dmin * (float)mn;
        out = FUSED ? __builtin_fmaf(d1, (float)qv, -m1) : d1 * (float)qv - m1;
    } else if (TYPE == MQ_TYPE_Q6_K) {
        const uint8_t *b = r + (col / QK_K) * sizeof(block_q6_K);
        const int e = (int)(col % QK_K);
        const int h = e >> 7, rr = e & 127, g = rr >> 5, l = rr & 31;
        const uint8_t qlb = b[64 * h + l + (g & 1) * 32];
        const int nib = (g < 2) ? (qlb & 0xF) : (qlb >> 4);
        const int hb = (b[128 + 32 * h + l] >> (2 * g)) & 3;
        const int qv = (nib | (hb << 4)) - 32;
        const int8_t sc = (int8_t)b[192 + 8 * h + (l >> 4) + 2 * g];
        const float d = f16_bits_to_f32(*(const uint16_t *)(b + 208));
        out = d * (float)sc * (float)qv;
    } else if (TYPE == MQ_TYPE_Q8_K) {
        const uint8_t *b = r + (col / QK_K) * sizeof(block_q8_K);
        out = *(const float *)b * (float)(int8_t)b[4 + col % QK_K];
    }
    y[gid] = out;
}

// ---------------------------------------------------------------------------
// Weight-plane preparation: one thread per (row, GGUF block).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_prepare_q8_0(const uint8_t *__restrict__ gguf, int8_t *__restrict__ qs,
                                                      uint16_t *__restrict__ d16, int64_t row0, int64_t row1,
                                                      int64_t k) {
    const int64_t nbr = k / QK8_0;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (row1 - row0) * nbr) return;
    const int64_t row = row0 + gid / nbr, b = gid % nbr;
    const uint8_t *src = gguf + (row * nbr + b) * sizeof(block_q8_0);
    d16[row * nbr + b] = *(const uint16_t *)src;
    uint32_t *dst = (uint32_t *)(qs + row * k + b * QK8_0);
    const uint16_t *s16 = (const uint16_t *)(src + 2);
#pragma unroll
    for (int i = 0; i < 8; i++) dst[i] = (uint32_t)s16[2 * i] | ((uint32_t)s16[2 * i + 1] << 16);
}

__global__ __launch_bounds__(256) void k_prepare_q4_K(const uint8_t *__restrict__ gguf, int8_t *__restrict__ lo,
                                                      int8_t *__restrict__ hi, float *__restrict__ dw,
                                                      float *__restrict__ dmin, _Float16 *__restrict__ mins,
                                                      int64_t row0, int64_t row1, int64_t k) {
    const int64_t nbr = k / QK_K;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (row1 - row0) * nbr) return;
    const int64_t row = row0 + gid / nbr, b = gid % nbr;
    const uint8_t *src = gguf + (row * nbr + b) * sizeof(block_q4_K);
    const int64_t sbi = row * nbr + b;
    dw[sbi] = f16_bits_to_f32(*(const uint16_t *)src);
    dmin[sbi] = f16_bits_to_f32(*(const uint16_t *)(src + 2));
    int sc[8], mn[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        scale_min_k4(j, src + 4, sc[j], mn[j]);
        mins[sbi * 8 + j] = (_Float16)mn[j];
    }
    int8_t *plo = lo + row * k + b * QK_K;
    int8_t *phi = hi + row * k + b * QK_K;
    for (int c = 0; c < 4; c++) {
        for (int l = 0; l < 32; l++) {
            const uint8_t byte = src[16 + 32 * c + l];
            const int v0 = sc[2 * c] * (byte & 0xF);       // value 64c + l
            const int v1 = sc[2 * c + 1] * (byte >> 4);    // value 64c + 32 + l
            plo[64 * c + l] = (int8_t)(v0 & 127);
            phi[64 * c + l] = (int8_t)(v0 >> 7);
            plo[64 * c + 32 + l] = (int8_t)(v1 & 127);
            phi[64 * c + 32 + l] = (int8_t)(v1 >> 7);
        }
    }
}

__global__ __launch_bounds__(256) void k_prepare_q6_K(const uint8_t *__restrict__ gguf, int8_t *__restrict__ lo,
                                                      int8_t *__restrict__ hi, float *__restrict__ dw,
                                                      uint8_t *__restrict__ ql, uint8_t *__restrict__ qh,
                                                      int8_t *__restrict__ scp, uint16_t *__restrict__ d16,
                                                      int64_t row0, int64_t row1, int64_t k) {
    const int64_t nbr = k / QK_K;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (row1 - row0) * nbr) return;
    const int64_t row = row0 + gid / nbr, b = gid % nbr;
    const uint8_t *src = gguf + (row * nbr + b) * sizeof(block_q6_K);
    const int64_t sbi = row * nbr + b;
    const uint16_t dbits = *(const uint16_t *)(src + 208);
    d16[sbi] = dbits;
    dw[sbi] = f16_bits_to_f32(dbits);
    for (int i = 0; i < 128; i++) ql[sbi * 128 + i] = src[i];
    for (int i = 0; i < 64; i++) qh[sbi * 64 + i] = src[128 + i];
    for (int i = 0; i < 16; i++) scp[sbi * 16 + i] = (int8_t)src[192 + i];
    int8_t *plo = lo + row * k + b * QK_K;
    int8_t *phi = hi + row * k + b * QK_K;
    for (int e = 0; e < QK_K; e++) {
        const int h = e >> 7, rr = e & 127, g = rr >> 5, l = rr & 31;
        const uint8_t qlb = src[64 * h + l + (g & 1) * 32];
        const int nib = (g < 2) ? (qlb & 0xF) : (qlb >> 4);
        const int hb = (src[128 + 32 * h + l] >> (2 * g)) & 3;
        const int qv = (nib | (hb << 4)) - 32;
        const int sc = (int8_t)src[192 + 8 * h + (l >> 4) + 2 * g];
        const int v = sc * qv;  // in [-4064, 4096]
        plo[e] = (int8_t)(v & 127);
        phi[e] = (int8_t)(v >> 7);  // arithmetic shift: v = lo + 128*hi
    }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
static inline bool aligned16(const void *p, int64_t ld_floats) {
    return (((uintptr_t)p) % 16 == 0) && ((ld_floats * 4) % 16 == 0);
}

static inline unsigned grid_for(int64_t threads) { return (unsigned)((threads + 255) / 256); }

template <bool PLANAR>
static hipError_t q8_0_dispatch(const float *x, int64_t ldx, int8_t *out, float *xd, int64_t m, int64_t k, int variant,
                                hipStream_t s) {
    const int64_t threads = m * (k / QK8_0) * 8;
    if (threads == 0) return hipSuccess;
    const bool v4 = aligned16(x, ldx);
    const dim3 g(grid_for(threads)), b(256);
#define MQ_Q80(VAR)                                                                                      \
    if (v4) hipLaunchKernelGGL((k_quantize_q8_0<VAR, PLANAR, true>), g, b, 0, s, x, ldx, out, xd, m, k); \
    else hipLaunchKernelGGL((k_quantize_q8_0<VAR, PLANAR, false>), g, b, 0, s, x, ldx, out, xd, m, k);
    switch (variant) {
        case MQ_Q8_0_X86: MQ_Q80(MQ_Q8_0_X86); break;
        case MQ_Q8_0_NEON: MQ_Q80(MQ_Q8_0_NEON); break;
        case MQ_Q8_0_REF: MQ_Q80(MQ_Q8_0_REF); break;
        default: return hipErrorInvalidValue;
    }
#undef MQ_Q80
    return hipGetLastError();
}

template <bool PLANAR>
static hipError_t q8_K_dispatch(const float *x, int64_t ldx, int8_t *out, float *xd, int16_t *xbs, int64_t m,
                                int64_t k, hipStream_t s) {
    const int64_t threads = m * (k / QK_K) * 64;
    if (threads == 0) return hipSuccess;
    const dim3 g(grid_for(threads)), b(256);
    if (aligned16(x, ldx))
        hipLaunchKernelGGL((k_quantize_q8_K<PLANAR, true>), g, b, 0, s, x, ldx, out, xd, xbs, m, k);
    else
        hipLaunchKernelGGL((k_quantize_q8_K<PLANAR, false>), g, b, 0, s, x, ldx, out, xd, xbs, m, k);
    return hipGetLastError();
}

hipError_t launch_quantize_f16(const float *x, int64_t ldx, void *y, int64_t m, int64_t k, hipStream_t s) {
    const int64_t threads = m * (k / 4);
    if (threads == 0) return hipSuccess;
    const dim3 g(grid_for(threads)), b(256);
    if (aligned16(x, ldx))
        hipLaunchKernelGGL((k_quantize_f16<true>), g, b, 0, s, x, ldx, (uint16_t *)y, m, k);
    else
        hipLaunchKernelGGL((k_quantize_f16<false>), g, b, 0, s, x, ldx, (uint16_t *)y, m, k);
    return hipGetLastError();
}

hipError_t launch_quantize_act_planar(int wtype, const float *x, int64_t ldx, void *ws, int64_t m, int64_t k,
                                      int q8_0_variant, hipStream_t s) {
    const ActPlanes a = act_planes(wtype, m, k);
    uint8_t *base = (uint8_t *)ws;
    switch (wtype) {
        case MQ_TYPE_Q8_0:
            return q8_0_dispatch<true>(x, ldx, (int8_t *)(base + a.xq), (float *)(base + a.xd), m, k, q8_0_variant, s);
        case MQ_TYPE_Q4_K:
        case MQ_TYPE_Q6_K:
            return q8_K_dispatch<true>(x, ldx, (int8_t *)(base + a.xq), (float *)(base + a.xd),
                                       (int16_t *)(base + a.xbs), m, k, s);
        case MQ_TYPE_F16: return launch_quantize_f16(x, ldx, base + a.xq, m, k, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_quantize_q8_0_gguf(const float *x, int64_t ldx, void *y, int64_t m, int64_t k, int variant,
                                     hipStream_t s) {
    return q8_0_dispatch<false>(x, ldx, (int8_t *)y, nullptr, m, k, variant, s);
}

hipError_t launch_quantize_q8_K_gguf(const float *x, int64_t ldx, void *y, int64_t m, int64_t k, hipStream_t s) {
    return q8_K_dispatch<false>(x, ldx, (int8_t *)y, nullptr, nullptr, m, k, s);
}

hipError_t launch_dequantize(int type, const void *w, float *y, int64_t nrows, int64_t k, int fused, hipStream_t s) {
    const int64_t threads = nrows * k;
    if (threads == 0) return hipSuccess;
    const dim3 g(grid_for(threads)), b(256);
    const uint8_t *src = (const uint8_t *)w;
    switch (type) {
        case MQ_TYPE_F16: hipLaunchKernelGGL((k_dequantize<MQ_TYPE_F16, false>), g, b, 0, s, src, y, nrows, k); break;
        case MQ_TYPE_Q8_0: hipLaunchKernelGGL((k_dequantize<MQ_TYPE_Q8_0, false>), g, b, 0, s, src, y, nrows, k); break;
        case MQ_TYPE_Q4_K:
            if (fused) hipLaunchKernelGGL((k_dequantize<MQ_TYPE_Q4_K, true>), g, b, 0, s, src, y, nrows, k);
            else hipLaunchKernelGGL((k_dequantize<MQ_TYPE_Q4_K, false>), g, b, 0, s, src, y, nrows, k);
            break;
        case MQ_TYPE_Q6_K: hipLaunchKernelGGL((k_dequantize<MQ_TYPE_Q6_K, false>), g, b, 0, s, src, y, nrows, k); break;
        case MQ_TYPE_Q8_K: hipLaunchKernelGGL((k_dequantize<MQ_TYPE_Q8_K, false>), g, b, 0, s, src, y, nrows, k); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_weight_prepare(int type, void *image, int64_t n, int64_t k, int64_t row0, int64_t row1,
                                 hipStream_t s) {
    const WeightPlanes p = weight_planes(type, n, k);
    uint8_t *base = (uint8_t *)image;
    if (row1 <= row0) return hipSuccess;
    switch (type) {
        case MQ_TYPE_F16: return hipSuccess;
        case MQ_TYPE_Q8_0: {
            const int64_t threads = (row1 - row0) * (k / QK8_0);
            hipLaunchKernelGGL(k_prepare_q8_0, dim3(grid_for(threads)), dim3(256), 0, s, base,
                               (int8_t *)(base + p.qs), (uint16_t *)(base + p.d16), row0, row1, k);
            break;
        }
        case MQ_TYPE_Q4_K: {
            const int64_t threads = (row1 - row0) * (k / QK_K);
            hipLaunchKernelGGL(k_prepare_q4_K, dim3(grid_for(threads)), dim3(256), 0, s, base,
                               (int8_t *)(base + p.qs), (int8_t *)(base + p.hi), (float *)(base + p.dw),
                               (float *)(base + p.dmin), (_Float16 *)(base + p.mins), row0, row1, k);
            break;
        }
        case MQ_TYPE_Q6_K: {
            const int64_t threads = (row1 - row0) * (k / QK_K);
            hipLaunchKernelGGL(k_prepare_q6_K, dim3(grid_for(threads)), dim3(256), 0, s, base,
                               (int8_t *)(base + p.qs), (int8_t *)(base + p.hi), (float *)(base + p.dw),
                               (uint8_t *)(base + p.ql), (uint8_t *)(base + p.qh), (int8_t *)(base + p.sc),
                               (uint16_t *)(base + p.d16), row0, row1, k);
            break;
        }
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mq
