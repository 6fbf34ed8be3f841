// mq_gemv.hip -- small-M (m <= 8) mul_mat that streams packed weights once.
//
// Decode-shaped MUL_MATs (src/qwen2vl_ocr.cpp:2368-2452: one activation row per
// generated token) touch every weight byte once and do 2*m flops per weight, so
// they are HBM-bound.  Each wave owns one weight row at a time and its 64 lanes
// walk that row's blocks in order, so a wave reads contiguous bytes and every
// byte is read exactly once; activations (m x k int8, a few KB) stay in L1/L2.
// Integer block dots use v_dot4_i32_i8; per-block scales are applied in fp32,
// as ggml's vec_dot does.
//   Q4_K reads the GGUF blocks directly (144-byte blocks stay 16-byte aligned).
//   Q6_K and Q8_0 read the byte-identical split planes of the weight image
//   (their 210- and 34-byte GGUF blocks are only 2-byte aligned).
//   F16 uses v_dot2_f32_f16 on fp16 activations.
#include "mq_internal.h"

namespace mq {

typedef _Float16 v2h __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

template <int MM>
__device__ __forceinline__ void wave_sum_store(float (&part)[MM], float *y, int64_t ldy, int row, int lane) {
#pragma unroll
    for (int m = 0; m < MM; m++) {
        float v = part[m];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
        part[m] = v;
    }
    if (lane < MM) {
        float v = part[0];
#pragma unroll
        for (int m = 1; m < MM; m++)
            if (lane == m) v = part[m];
        y[(int64_t)lane * ldy + row] = v;
    }
}

// ---- Q4_K x Q8_K: lane = 8*sb_slot + (2*c + h); lane covers 16 low + 16 high nibbles ----
template <int MM>
__global__ __launch_bounds__(256) void k_gemv_q4_K(const uint8_t *__restrict__ w, const int8_t *__restrict__ xq,
                                                   const float *__restrict__ xd, const int16_t *__restrict__ xbs,
                                                   float *__restrict__ y, int N, int K, int64_t ldy) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= N) return;
    const int nsb = K / QK_K;
    const uint8_t *wr = w + (int64_t)row * nsb * sizeof(block_q4_K);
    const int t = lane & 7, c = t >> 1, h = t & 1;
    float part[MM];
#pragma unroll
    for (int m = 0; m < MM; m++) part[m] = 0.f;
    for (int sb = lane >> 3; sb < nsb; sb += 8) {
        const uint8_t *blk = wr + sb * sizeof(block_q4_K);
        const uint4 hdr = *(const uint4 *)blk;
        const uint4 qv = *(const uint4 *)(blk + 16 + 32 * c + 16 * h);
        const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(hdr.x & 0xffff));
        const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(hdr.x >> 16));
        uint8_t s[12];
        *(uint32_t *)&s[0] = hdr.y;
        *(uint32_t *)&s[4] = hdr.z;
        *(uint32_t *)&s[8] = hdr.w;
        int sca, ma, scb, mb;
        {
            const int ja = 2 * c, jb = 2 * c + 1;
            if (ja < 4) {
                sca = s[ja] & 63;
                ma = s[ja + 4] & 63;
                scb = s[jb] & 63;
                mb = s[jb + 4] & 63;
            } else {
                sca = (s[ja + 4] & 0xF) | ((s[ja - 4] >> 6) << 4);
                ma = (s[ja + 4] >> 4) | ((s[ja] >> 6) << 4);
                scb = (s[jb + 4] & 0xF) | ((s[jb - 4] >> 6) << 4);
                mb = (s[jb + 4] >> 4) | ((s[jb] >> 6) << 4);
            }
        }
        const uint32_t l0 = qv.x & 0x0F0F0F0F, l1 = qv.y & 0x0F0F0F0F, l2 = qv.z & 0x0F0F0F0F,
                       l3 = qv.w & 0x0F0F0F0F;
        const uint32_t h0 = (qv.x >> 4) & 0x0F0F0F0F, h1 = (qv.y >> 4) & 0x0F0F0F0F,
                       h2 = (qv.z >> 4) & 0x0F0F0F0F, h3 = (qv.w >> 4) & 0x0F0F0F0F;
#pragma unroll
        for (int m = 0; m < MM; m++) {
            const int8_t *xr = xq + (int64_t)m * K + sb * QK_K + 64 * c + 16 * h;
            const uint4 xa = *(const uint4 *)xr;
            const uint4 xb = *(const uint4 *)(xr + 32);
            int sa = dot4(l0, xa.x, 0);
            sa = dot4(l1, xa.y, sa);
            sa = dot4(l2, xa.z, sa);
            sa = dot4(l3, xa.w, sa);
            int sbv = dot4(h0, xb.x, 0);
            sbv = dot4(h1, xb.y, sbv);
            sbv = dot4(h2, xb.z, sbv);
            sbv = dot4(h3, xb.w, sbv);
            const int16_t *bs = xbs + (int64_t)m * (K / 16) + sb * 16 + 4 * c + h;
            const int imain = sca * sa + scb * sbv;
            const int imin = ma * bs[0] + mb * bs[2];
            part[m] += xd[(int64_t)m * nsb + sb] * (d * (float)imain - dmin * (float)imin);
        }
    }
    wave_sum_store<MM>(part, y, ldy, row, lane);
}

// ---- Q6_K x Q8_K on the split planes: lane = 4*sb_slot + (2*h + t), 64 values per lane ----
template <int MM>
__global__ __launch_bounds__(256) void k_gemv_q6_K(const uint8_t *__restrict__ ql, const uint8_t *__restrict__ qh,
                                                   const int8_t *__restrict__ scp, const uint16_t *__restrict__ d16,
                                                   const int8_t *__restrict__ xq, const float *__restrict__ xd,
                                                   const int16_t *__restrict__ xbs, float *__restrict__ y, int N,
                                                   int K, int64_t ldy) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= N) return;
    const int nsb = K / QK_K;
    const int t4 = lane & 3, h = t4 >> 1, t = t4 & 1;
    float part[MM];
#pragma unroll
    for (int m = 0; m < MM; m++) part[m] = 0.f;
    for (int sb = lane >> 2; sb < nsb; sb += 16) {
        const int64_t sbi = (int64_t)row * nsb + sb;
        const uint4 L = *(const uint4 *)(ql + sbi * 128 + 64 * h + 16 * t);
        const uint4 Lh = *(const uint4 *)(ql + sbi * 128 + 64 * h + 32 + 16 * t);
        const uint4 H = *(const uint4 *)(qh + sbi * 64 + 32 * h + 16 * t);
        const uint2 scw = *(const uint2 *)(scp + sbi * 16 + 8 * h);
        const float d = (float)__builtin_bit_cast(_Float16, d16[sbi]);
        int8_t sc8[8];
        *(uint2 *)sc8 = scw;
        const int sc0 = sc8[t], sc1 = sc8[t + 2], sc2 = sc8[t + 4], sc3 = sc8[t + 6];
        const uint32_t Lw[4] = {L.x, L.y, L.z, L.w}, Lhw[4] = {Lh.x, Lh.y, Lh.z, Lh.w}, Hw[4] = {H.x, H.y, H.z, H.w};
        uint32_t g0[4], g1[4], g2[4], g3[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            g0[i] = (Lw[i] & 0x0F0F0F0F) | ((Hw[i] << 4) & 0x30303030);
            g1[i] = (Lhw[i] & 0x0F0F0F0F) | ((Hw[i] << 2) & 0x30303030);
            g2[i] = ((Lw[i] >> 4) & 0x0F0F0F0F) | (Hw[i] & 0x30303030);
            g3[i] = ((Lhw[i] >> 4) & 0x0F0F0F0F) | ((Hw[i] >> 2) & 0x30303030);
        }
#pragma unroll
        for (int m = 0; m < MM; m++) {
            const int8_t *xr = xq + (int64_t)m * K + sb * QK_K + 128 * h + 16 * t;
            const uint4 x0 = *(const uint4 *)(xr + 0);
            const uint4 x1 = *(const uint4 *)(xr + 32);
            const uint4 x2 = *(const uint4 *)(xr + 64);
            const uint4 x3 = *(const uint4 *)(xr + 96);
            int s0 = dot4(g0[0], x0.x, 0), s1 = dot4(g1[0], x1.x, 0), s2 = dot4(g2[0], x2.x, 0),
                s3 = dot4(g3[0], x3.x, 0);
            s0 = dot4(g0[1], x0.y, s0);
            s1 = dot4(g1[1], x1.y, s1);
            s2 = dot4(g2[1], x2.y, s2);
            s3 = dot4(g3[1], x3.y, s3);
            s0 = dot4(g0[2], x0.z, s0);
            s1 = dot4(g1[2], x1.z, s1);
            s2 = dot4(g2[2], x2.z, s2);
            s3 = dot4(g3[2], x3.z, s3);
            s0 = dot4(g0[3], x0.w, s0);
            s1 = dot4(g1[3], x1.w, s1);
            s2 = dot4(g2[3], x2.w, s2);
            s3 = dot4(g3[3], x3.w, s3);
            // (q6 - 32) * q8 summed = q6.q8 - 32 * bsum16 of the same 16 values
            const int16_t *bs = xbs + (int64_t)m * (K / 16) + sb * 16 + 8 * h + t;
            const int isum = sc0 * (s0 - 32 * bs[0]) + sc1 * (s1 - 32 * bs[2]) + sc2 * (s2 - 32 * bs[4]) +
                             sc3 * (s3 - 32 * bs[6]);
            part[m] += (d * xd[(int64_t)m * nsb + sb]) * (float)isum;
        }
    }
    wave_sum_store<MM>(part, y, ldy, row, lane);
}

// ---- Q8_0 x Q8_0 on the split planes: one 32-value block per lane ----
template <int MM>
__global__ __launch_bounds__(256) void k_gemv_q8_0(const int8_t *__restrict__ qs, const uint16_t *__restrict__ d16,
                                                   const int8_t *__restrict__ xq, const float *__restrict__ xd,
                                                   float *__restrict__ y, int N, int K, int64_t ldy) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= N) return;
    const int nb = K / QK8_0;
    float part[MM];
#pragma unroll
    for (int m = 0; m < MM; m++) part[m] = 0.f;
    for (int b = lane; b < nb; b += 64) {
        const int8_t *wp = qs + (int64_t)row * K + b * QK8_0;
        const uint4 w0 = *(const uint4 *)wp;
        const uint4 w1 = *(const uint4 *)(wp + 16);
        const float dw = (float)__builtin_bit_cast(_Float16, d16[(int64_t)row * nb + b]);
#pragma unroll
        for (int m = 0; m < MM; m++) {
            const int8_t *xr = xq + (int64_t)m * K + b * QK8_0;
            const uint4 x0 = *(const uint4 *)xr;
            const uint4 x1 = *(const uint4 *)(xr + 16);
            int s = dot4(w0.x, x0.x, 0);
            s = dot4(w0.y, x0.y, s);
            s = dot4(w0.z, x0.z, s);
            s = dot4(w0.w, x0.w, s);
            s = dot4(w1.x, x1.x, s);
            s = dot4(w1.y, x1.y, s);
            s = dot4(w1.z, x1.z, s);
            s = dot4(w1.w, x1.w, s);
            part[m] += (float)s * (dw * xd[(int64_t)m * nb + b]);
        }
    }
    wave_sum_store<MM>(part, y, ldy, row, lane);
}

// ---- F16 x F16: 8 halves per lane per step ----
template <int MM>
__global__ __launch_bounds__(256) void k_gemv_f16(const uint16_t *__restrict__ w, const uint16_t *__restrict__ xh,
                                                  float *__restrict__ y, int N, int K, int64_t ldy) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= N) return;
    const int nc = K / 8;
    float part[MM];
#pragma unroll
    for (int m = 0; m < MM; m++) part[m] = 0.f;
    for (int c = lane; c < nc; c += 64) {
        const uint4 wv = *(const uint4 *)(w + (int64_t)row * K + c * 8);
        const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
        for (int m = 0; m < MM; m++) {
            const uint4 xv = *(const uint4 *)(xh + (int64_t)m * K + c * 8);
            const uint32_t xx[4] = {xv.x, xv.y, xv.z, xv.w};
            float s = part[m];
#pragma unroll
            for (int i = 0; i < 4; i++)
                s = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2h, ww[i]), __builtin_bit_cast(v2h, xx[i]), s, false);
            part[m] = s;
        }
    }
    wave_sum_store<MM>(part, y, ldy, row, lane);
}

template <int MM>
static void gemv_launch(int type, const uint8_t *wb, const WeightPlanes &p, int64_t n, int64_t k, const uint8_t *xb,
                        const ActPlanes &ap, float *y, int64_t ldy, hipStream_t s) {
    const dim3 grid((unsigned)((n + 3) / 4)), block(256);
    const int8_t *xq = (const int8_t *)(xb + ap.xq);
    const float *xd = (const float *)(xb + ap.xd);
    const int16_t *xbs = (const int16_t *)(xb + ap.xbs);
    switch (type) {
        case MQ_TYPE_Q4_K:
            hipLaunchKernelGGL(k_gemv_q4_K<MM>, grid, block, 0, s, wb, xq, xd, xbs, y, (int)n, (int)k, ldy);
            break;
        case MQ_TYPE_Q6_K:
            hipLaunchKernelGGL(k_gemv_q6_K<MM>, grid, block, 0, s, wb + p.ql, wb + p.qh, (const int8_t *)(wb + p.sc),
                               (const uint16_t *)(wb + p.d16), xq, xd, xbs, y, (int)n, (int)k, ldy);
            break;
        case MQ_TYPE_Q8_0:
            hipLaunchKernelGGL(k_gemv_q8_0<MM>, grid, block, 0, s, (const int8_t *)(wb + p.qs),
                               (const uint16_t *)(wb + p.d16), xq, xd, y, (int)n, (int)k, ldy);
            break;
        case MQ_TYPE_F16:
            hipLaunchKernelGGL(k_gemv_f16<MM>, grid, block, 0, s, (const uint16_t *)wb, (const uint16_t *)xq, y, (int)n,
                               (int)k, ldy);
            break;
        default: break;
    }
}

hipError_t launch_gemv(int type, const void *image, int64_t n, int64_t k, const void *ws, int64_t m, float *y,
                       int64_t ldy, hipStream_t s) {
    if (m <= 0 || n <= 0) return hipSuccess;
    if (m > 8) return hipErrorInvalidValue;
    const WeightPlanes p = weight_planes(type, n, k);
    const ActPlanes ap = act_planes(type, m, k, false);
    const uint8_t *wb = (const uint8_t *)image;
    const uint8_t *xb = (const uint8_t *)ws;
    switch (m) {
        case 1: gemv_launch<1>(type, wb, p, n, k, xb, ap, y, ldy, s); break;
        case 2: gemv_launch<2>(type, wb, p, n, k, xb, ap, y, ldy, s); break;
        case 3: gemv_launch<3>(type, wb, p, n, k, xb, ap, y, ldy, s); break;
        case 4: gemv_launch<4>(type, wb, p, n, k, xb, ap, y, ldy, s); break;
        case 5: gemv_launch<5>(type, wb, p, n, k, xb, ap, y, ldy, s); break;
        case 6: gemv_launch<6>(type, wb, p, n, k, xb, ap, y, ldy, s); break;
        case 7: gemv_launch<7>(type, wb, p, n, k, xb, ap, y, ldy, s); break;
        case 8: gemv_launch<8>(type, wb, p, n, k, xb, ap, y, ldy, s); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mq
