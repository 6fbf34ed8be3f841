// mq_gemv.hip -- small-M (m <= 8) mul_mat that streams packed weights once.
//
// Decode-shaped MUL_MATs (src/qwen2vl_ocr.cpp:2368-2452: one activation row per
// generated token) touch every weight byte once and do 2*m flops per weight, so
// they are HBM-bound.  Each wave owns one weight row at a time and its 64 lanes
// walk that row's blocks in order, so a wave reads contiguous bytes and every
// byte is read exactly once; activations (m x k int8, a few KB) stay in L1/L2.
// Integer block dots use v_dot4_i32_i8; per-block scales are applied in fp32,
// as ggml's vec_dot does.
//   Q4_K runs on the matrix cores (k_gemv_kq_mfma below): at m <= 8 the dot4
//   form is VALU-bound long before HBM is.
//   Q6_K runs on the matrix cores too (same kernel).
//   Q8_0 reads the byte-identical split planes of the weight image (its 34-byte
//   GGUF blocks are only 2-byte aligned).
//   F16 uses v_dot2_f32_f16 on fp16 activations.
#include "mq_internal.h"

#include <climits>

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace mq {

typedef _Float16 v2h __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

template <int MM>
__device__ __forceinline__ void wave_sum_store(float (&part)[MM], float *y, int64_t ldy, int row, int lane,
                                               const float *bias) {
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
        y[(int64_t)lane * ldy + row] = bias ? v + bias[row] : v;
    }
}

// ---- Q8_0 x Q8_0 on the split planes: one 32-value block per lane ----
template <int MM>
__global__ __launch_bounds__(256) void k_gemv_q8_0(const int8_t *__restrict__ qs, const uint16_t *__restrict__ d16,
                                                   const int8_t *__restrict__ xq, const float *__restrict__ xd,
                                                   float *__restrict__ y, int N, int K, int64_t ldy,
                                                   const float *__restrict__ bias) {
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
    wave_sum_store<MM>(part, y, ldy, row, lane, bias);
}

// ---- F16 x F16: 8 halves per lane per step ----
template <int MM>
__global__ __launch_bounds__(256) void k_gemv_f16(const uint16_t *__restrict__ w, const uint16_t *__restrict__ xh,
                                                  float *__restrict__ y, int N, int K, int64_t ldy,
                                                  const float *__restrict__ bias) {
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
    wave_sum_store<MM>(part, y, ldy, row, lane, bias);
}

// ---- K-quants on MFMA (m <= 8) ----
// Q4_K: per 64-value chunk c of a superblock, v_mfma_i32_16x16x64_i8 multiplies the 16
// rows' 4-bit quants (A: row l%16, k 16*(l/16)..+16 of the chunk) by an activation operand
// whose 16 columns are (token m = col%8, sub-block g = col/8): column (m, g) holds the
// token's quants on the k range of sub-block 2c+g and zeros elsewhere.  So output column
// (m, g) is the exact sub-block sum isum_{2c+g}[row][m], and the 6-bit scale is one
// integer multiply-add per output.  The min term sum_j m_j * B_j is one
// v_mfma_f32_16x16x16_f16 (m_j and the two limbs of B_j exact in fp16, products and sums
// below 2^24: exact).  Per superblock, as ggml's vec_dot_q4_K_q8_K:
//   y += d_x * (d * sum_j sc_j isum_j - dmin * sum_j m_j B_j).
// Q6_K: per 32-value K-step, v_mfma_i32_16x16x32_i8 multiplies 4 (q - 32) -- the 6-bit
// two's complement v = q ^ 32 of the plane shifted into the top of each byte, exact in int8
// -- by an activation operand whose columns are (token m, 16-group g) the same way, so each
// output is 4 times one 16-value group sum and its int8 scale is one integer multiply-add.
// Per superblock, as ggml's vec_dot_q6_K_q8_K:
//   y += d_x * d * sum_g sc_g sum_{i in g} (q_i - 32) x_i      (the 4 leaves through d_x / 4)
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v4i_t __attribute__((ext_vector_type(4)));

struct GvLane {
    int lane, wave, col, q, m, g;
    bool xlive;  // this lane carries activation data: its k range lies in the column's sub-block / group
    bool mlive;  // min-term operand column is a real token (cols >= 8 stay zero: M <= 8)
};

__device__ __forceinline__ GvLane gv_lane(int M) {
    GvLane L;
    L.lane = threadIdx.x & 63;
    L.wave = threadIdx.x >> 6;
    L.col = L.lane & 15;
    L.q = L.lane >> 4;
    L.m = L.col & 7;
    L.g = L.col >> 3;
    L.xlive = (L.m < M) && ((L.q >> 1) == L.g);
    L.mlive = L.col < M;
    return L;
}

__device__ __forceinline__ float2 half2_bits(uint32_t u) {
    return make_float2((float)__builtin_bit_cast(_Float16, (uint16_t)(u & 0xffff)),
                       (float)__builtin_bit_cast(_Float16, (uint16_t)(u >> 16)));
}

struct Q4Act {
    v4i_t xa[4];
    v4h bmin;
    float dx;
};
__device__ __forceinline__ Q4Act q4_act(const GvLane &L, const int8_t *xq, const float *xd, const _Float16 *xgm, int K,
                                        int M, int sb) {
    Q4Act A;
    const int8_t *xr = xq + (int64_t)L.m * K + sb * QK_K + 16 * L.q;
#pragma unroll
    for (int c = 0; c < 4; c++) A.xa[c] = L.xlive ? *(const v4i_t *)(xr + 64 * c) : (v4i_t){0, 0, 0, 0};
    A.bmin = (v4h){};
    if (L.mlive) A.bmin = *(const v4h *)(xgm + ((sb * 8 + L.col) << 4) + 4 * L.q);
    A.dx = (L.m < M) ? xd[(int64_t)L.m * (K / QK_K) + sb] : 0.0f;
    return A;
}
struct Q4W {  // one (tile, superblock) of the Q4_K GEMV plane, this lane's share
    v4i_t wq[4], scv, dd;
    uint32_t mnv;
};
__device__ __forceinline__ Q4W q4_load(const GvLane &L, const uint8_t *T) {
    Q4W W;
#pragma unroll
    for (int c = 0; c < 4; c++) W.wq[c] = *(const v4i_t *)(T + GV4_QS + ((c * 2 + (L.q & 1)) * GV_ROWS + L.col) * 16);
    W.scv = *(const v4i_t *)(T + GV4_SC + (L.g * 4 + L.q) * 16);  // sc of rows 4q+i, chunk c: byte 4c+i
    W.mnv = *(const uint32_t *)(T + GV4_MN + ((L.q & 1) * GV_ROWS + L.col) * 4);
    W.dd = *(const v4i_t *)(T + GV4_DD + L.q * 16);  // (d, dmin) halves of rows 4q..4q+3
    return W;
}
__device__ __forceinline__ void q4_compute(const GvLane &L, const Q4W &W, const Q4Act &A, float (&part)[4]) {
    const int sh = 4 * (L.q >> 1);  // low nibbles for k < 32 of the chunk, high for k >= 32
    int acc[4] = {0, 0, 0, 0};
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const v4i_t w = {(W.wq[c].x >> sh) & 0x0F0F0F0F, (W.wq[c].y >> sh) & 0x0F0F0F0F,
                         (W.wq[c].z >> sh) & 0x0F0F0F0F, (W.wq[c].w >> sh) & 0x0F0F0F0F};
        const v4i_t d = __builtin_amdgcn_mfma_i32_16x16x64_i8(w, A.xa[c], (v4i_t){0, 0, 0, 0}, 0, 0, 0);
        const int scw = W.scv[c];
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] += __mul24((scw >> (8 * i)) & 0xff, d[i]);  // |d| < 2^23: v_mad_i32_i24
    }
    const v4h amin = {(_Float16)(float)(W.mnv & 0xff), (_Float16)(float)((W.mnv >> 8) & 0xff),
                      (_Float16)(float)((W.mnv >> 16) & 0xff), (_Float16)(float)(W.mnv >> 24)};
    const v4f fm = __builtin_amdgcn_mfma_f32_16x16x16f16(amin, A.bmin, (v4f){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float2 dm = half2_bits((uint32_t)W.dd[i]);
        // column m + 8 (sub-blocks 2c+1) joins column m: row_ror:8 inside each 16-lane row
        const int isum = acc[i] + __builtin_amdgcn_update_dpp(0, acc[i], 0x128, 0xF, 0xF, false);
        part[i] += A.dx * (dm.x * (float)isum - dm.y * fm[i]);
    }
}

struct Q6Act {
    int64_t xa[8];
    float dx;  // d_x / 4
};
__device__ __forceinline__ Q6Act q6_act(const GvLane &L, const int8_t *xq, const float *xd, const void *, int K,
                                        int M, int sb) {
    Q6Act A;
    const int8_t *xr = xq + (int64_t)L.m * K + sb * QK_K + 8 * L.q;
#pragma unroll
    for (int kk = 0; kk < 8; kk++) A.xa[kk] = L.xlive ? *(const int64_t *)(xr + 32 * kk) : 0;
    A.dx = (L.m < M) ? 0.25f * xd[(int64_t)L.m * (K / QK_K) + sb] : 0.0f;
    return A;
}
struct Q6W {  // one (tile, superblock) of the Q6_K GEMV plane, this lane's share
    v4i_t lo0, lo1, hiv, sc0, sc1;
    uint2 dv;
};
__device__ __forceinline__ Q6W q6_load(const GvLane &L, const uint8_t *T) {
    Q6W W;
    W.lo0 = *(const v4i_t *)(T + GV6_LO + (L.q * GV_ROWS + L.col) * 16);
    W.lo1 = *(const v4i_t *)(T + GV6_LO + 1024 + (L.q * GV_ROWS + L.col) * 16);
    W.hiv = *(const v4i_t *)(T + GV6_HI + (L.q * GV_ROWS + L.col) * 16);
    W.sc0 = *(const v4i_t *)(T + GV6_SC + (L.g * 4 + L.q) * 32);
    W.sc1 = *(const v4i_t *)(T + GV6_SC + (L.g * 4 + L.q) * 32 + 16);
    W.dv = *(const uint2 *)(T + GV6_D + L.q * 8);  // d halves of rows 4q..4q+3
    return W;
}
__device__ __forceinline__ void q6_compute(const GvLane &L, const Q6W &W, const Q6Act &A, float (&part)[4]) {
    const int los[8] = {W.lo0.x, W.lo0.y, W.lo0.z, W.lo0.w, W.lo1.x, W.lo1.y, W.lo1.z, W.lo1.w};
    const int his[4] = {W.hiv.x, W.hiv.y, W.hiv.z, W.hiv.w};
    const int scs[8] = {W.sc0.x, W.sc0.y, W.sc0.z, W.sc0.w, W.sc1.x, W.sc1.y, W.sc1.z, W.sc1.w};
    int acc[4] = {0, 0, 0, 0};
#pragma unroll
    for (int kk = 0; kk < 8; kk++) {
        // bytes 4 v: low nibble of v into bits 2-5, its two high bits into bits 6-7
        const uint32_t h = (uint32_t)his[kk >> 1], lo = (uint32_t)los[kk];
        const uint32_t h0 = (kk & 1) ? (h << 2) : (h << 6), h1 = (kk & 1) ? h : (h << 4);
        const uint32_t w0 = ((lo << 2) & 0x3C3C3C3Cu) | (h0 & 0xC0C0C0C0u);
        const uint32_t w1 = ((lo >> 2) & 0x3C3C3C3Cu) | (h1 & 0xC0C0C0C0u);
        const int64_t w = (int64_t)w0 | ((int64_t)w1 << 32);
        const v4i_t d = __builtin_amdgcn_mfma_i32_16x16x32_i8(w, A.xa[kk], (v4i_t){0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] += __mul24((int)(int8_t)(scs[kk] >> (8 * i)), d[i]);  // |d| < 2^23
    }
    const float2 d01 = half2_bits(W.dv.x), d23 = half2_bits(W.dv.y);
    const float dr[4] = {d01.x, d01.y, d23.x, d23.y};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        // column m + 8 (odd 16-groups) joins column m: row_ror:8 inside each 16-lane row
        const int isum = acc[i] + __builtin_amdgcn_update_dpp(0, acc[i], 0x128, 0xF, 0xF, false);
        part[i] += A.dx * (dr[i] * (float)isum);
    }
}

// Persistent form: a workgroup of 8 waves walks row tiles t = blockIdx.x, + gridDim.x, ...;
// wave w owns superblocks w, w + 8, ... (SBW <= 3 of them, K <= 2048 SBW) and builds their
// activation operands once.  Per tile it issues the weight loads of the NEXT tile before
// computing this one, writes its 16-row partial sums to LDS and, after one barrier, the
// workgroup reduces them (double-buffered, so one barrier per tile) and stores the rows.
// Up to three weights of the same type and K on one activation, their row tiles walked as one
// tile space: group g owns tiles [ts1 or 0 .. next start), tend tiles in all (ts_g = INT_MAX past
// the last group).  Selected per tile with scalar selects.
struct GvGroups {
    const uint8_t *gv0, *gv1, *gv2;
    float *y0, *y1, *y2;
    const float *b0, *b1, *b2;
    int N0, N1, N2;
    int64_t ld0, ld1, ld2;
    int ts1, ts2, tend;
};

// fp32 activation rows the GEMV quantizes itself (FQ = true): x (row stride ldx floats), and for
// MQ_PRE_SILU_MUL the up projection rows x2 (stride ldx2): the value quantized is then
// silu(x) * x2, as the activation quantizer's prologue forms it.
struct GvX {
    const float *x, *x2;
    int64_t ldx, ldx2;
    int pre;
};

// One 256-value superblock sb of rows 0..M-1 of the activation quantized to Q8_K
// (quantize_row_q8_K: the first value of largest magnitude sets iscale = -127 / max,
// q = min(127, nearest_int(iscale x)), d = 1 / iscale, the 16-value sums) by one wave: VPL
// values per lane, 256 / VPL lanes per row, 64 VPL / 256 rows per pass (VPL 4: one row at a
// time over all 64 lanes; 16: four rows), into this wave's LDS slot laid out as one superblock
// of the GEMV activation layout: quants qs[row][256], d ds[row], and the Q4_K min-term operand
// gs[row][16] (B_j & 63, then 64 (B_j >> 6), B_j the sum of the 32 quants of sub-block j).  The
// arithmetic is the activation quantizer's (no contraction), so the bytes are the ones it writes.
template <int VPL>
__device__ __forceinline__ void gv_quantize_sb(const GvX &X, int sb, int M, int lane, int8_t *qs, float *ds,
                                               _Float16 *gs) {
#pragma clang fp contract(off)
    constexpr int LPR = QK_K / VPL, RPP = 64 / LPR;  // lanes per row, rows per pass
    const int r0 = lane / LPR, p = lane % LPR, gbase = lane - p;
    for (int rb = 0; rb < M; rb += RPP) {
        const int m = rb + r0;
        float v[VPL];
        if (m < M) {
            const float *xr = X.x + (int64_t)m * X.ldx + sb * QK_K + VPL * p;
#pragma unroll
            for (int u = 0; u < VPL / 4; u++) {
                const float4 a = *(const float4 *)(xr + 4 * u);
                v[4 * u] = a.x, v[4 * u + 1] = a.y, v[4 * u + 2] = a.z, v[4 * u + 3] = a.w;
            }
            if (X.pre == MQ_PRE_SILU_MUL) {
                const float *ur = X.x2 + (int64_t)m * X.ldx2 + sb * QK_K + VPL * p;
#pragma unroll
                for (int u = 0; u < VPL / 4; u++) {
                    const float4 b = *(const float4 *)(ur + 4 * u);
                    const float w4[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
                    for (int e = 0; e < 4; e++) v[4 * u + e] = (v[4 * u + e] / (1.0f + expf(-v[4 * u + e]))) * w4[e];
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < VPL; e++) v[e] = 0.f;
        }
        // the lane's first value of largest magnitude, then the row's lowest such lane
        float la = 0.f, lm = 0.f;
#pragma unroll
        for (int e = 0; e < VPL; e++)
            if (fabsf(v[e]) > la) la = fabsf(v[e]), lm = v[e];
        float amax = la;
#pragma unroll
        for (int off = LPR / 2; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, LPR));
        const unsigned long long hit = __ballot(la == amax) >> gbase;
        const unsigned long long row_hits = LPR == 64 ? hit : (hit & ((1ull << LPR) - 1));
        const float mx = __shfl(lm, gbase + __ffsll((long long)row_hits) - 1);
        uint32_t w[VPL / 4];
#pragma unroll
        for (int u = 0; u < VPL / 4; u++) w[u] = 0;
        int s = 0;
        float dval = 0.f;
        if (amax != 0.0f) {
            const float iscale = -127.f / mx;
#pragma unroll
            for (int e = 0; e < VPL; e++) {
                const float f = iscale * v[e] + 12582912.f;  // ggml's nearest_int
                int q = (__float_as_int(f) & 0x007fffff) - 0x00400000;
                q = q < 127 ? q : 127;
                w[e >> 2] |= (uint32_t)(q & 0xff) << (8 * (e & 3));
                s += q;
            }
            dval = 1.0f / iscale;
        }
        // the sum of the 32 quants of sub-block (VPL p) / 32, complete in its first lane
#pragma unroll
        for (int off = 1; off < 32 / VPL; off <<= 1) s += __shfl_xor(s, off, LPR);
        if (m < M) {
#pragma unroll
            for (int u = 0; u < VPL / 4; u++) *(uint32_t *)(qs + m * QK_K + VPL * p + 4 * u) = w[u];
            if (p == 0) ds[m] = dval;
            if ((VPL * p) % 32 == 0) {
                const int j = VPL * p / 32;
                gs[m * 16 + j] = (_Float16)(s & 63);
                gs[m * 16 + 8 + j] = (_Float16)((s >> 6) * 64);
            }
        }
    }
}

// gv_quantize_sb with the lane mapping that keeps the most lanes busy for M rows
__device__ __forceinline__ void gv_quantize_rows(const GvX &X, int sb, int M, int lane, int8_t *qs, float *ds,
                                                 _Float16 *gs) {
    if (M == 1) gv_quantize_sb<4>(X, sb, M, lane, qs, ds, gs);
    else if (M == 2) gv_quantize_sb<8>(X, sb, M, lane, qs, ds, gs);
    else gv_quantize_sb<16>(X, sb, M, lane, qs, ds, gs);
}

template <int TYPE, int SBW, int PF, bool FQ = false>
__global__ __launch_bounds__(512) void k_gemv_kq_stream(const GvGroups G, const int8_t *__restrict__ xq,
                                                        const float *__restrict__ xd, const void *__restrict__ xaux,
                                                        int K, int M, const GvX X = GvX{}) {
    constexpr bool Q4 = TYPE == MQ_TYPE_Q4_K;
    constexpr int BYTES = Q4 ? GV4_BYTES : GV6_BYTES;
    using W = typename std::conditional<Q4, Q4W, Q6W>::type;
    using A = typename std::conditional<Q4, Q4Act, Q6Act>::type;
    __shared__ float red[2][8][GV_ROWS][8];
    // FQ: each wave's superblocks of the activation, quantized in the prologue
    __shared__ __attribute__((aligned(16))) int8_t aq[FQ ? 8 * SBW : 1][GEMV_CHUNK * QK_K];
    __shared__ float ad[FQ ? 8 * SBW : 1][GEMV_CHUNK];
    __shared__ __attribute__((aligned(16))) _Float16 ag[FQ ? 8 * SBW : 1][GEMV_CHUNK * 16];
    const GvLane L = gv_lane(M);
    const int nsb = K / QK_K;
    const int ntiles = G.tend;
    bool live[SBW];
    A act[SBW];
    W ring[PF + 1][SBW];
    int t = blockIdx.x;
    auto load = [&](W (&w)[SBW], int t) {
        const int tl = t >= G.ts2 ? t - G.ts2 : t >= G.ts1 ? t - G.ts1 : t;  // tile within its weight
        const uint8_t *gv = t >= G.ts2 ? G.gv2 : t >= G.ts1 ? G.gv1 : G.gv0;
#pragma unroll
        for (int i = 0; i < SBW; i++)
            if (live[i] && t < ntiles) {
                const uint8_t *T = gv + ((int64_t)tl * nsb + L.wave + 8 * i) * BYTES;
                if constexpr (Q4) w[i] = q4_load(L, T);
                else w[i] = q6_load(L, T);
            }
    };
#pragma unroll
    for (int i = 0; i < SBW; i++) live[i] = L.wave + 8 * i < nsb;
    // ring of PF + 1 register sets: the loads of the PF tiles after this one are in flight
    if constexpr (FQ) {
        // the first tiles' weights do not depend on the activation: in flight while it is quantized
#pragma unroll
        for (int f = 0; f < PF; f++) load(ring[f], t + f * (int)gridDim.x);
#pragma unroll
        for (int i = 0; i < SBW; i++)
            if (live[i]) {
                const int slot = L.wave * SBW + i;
                gv_quantize_rows(X, L.wave + 8 * i, M, L.lane, aq[slot], ad[slot], ag[slot]);
            }
        // the wave reads back what its own lanes wrote
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int i = 0; i < SBW; i++)
            if (live[i]) {  // the slot is one superblock of the activation layout (K = 256)
                const int slot = L.wave * SBW + i;
                if constexpr (Q4) act[i] = q4_act(L, aq[slot], ad[slot], ag[slot], QK_K, M, 0);
                else act[i] = q6_act(L, aq[slot], ad[slot], nullptr, QK_K, M, 0);
            }
    } else {
#pragma unroll
        for (int i = 0; i < SBW; i++)
            if (live[i]) {
                const int sb = L.wave + 8 * i;
                if constexpr (Q4) act[i] = q4_act(L, xq, xd, (const _Float16 *)xaux, K, M, sb);
                else act[i] = q6_act(L, xq, xd, xaux, K, M, sb);
            }
#pragma unroll
        for (int f = 0; f < PF; f++) load(ring[f], t + f * (int)gridDim.x);
    }
    for (int it = 0; t < ntiles; it++, t += gridDim.x) {
        // the storing lanes' bias, loaded ahead of the prefetch so that waiting for it at the
        // store does not wait for the next tiles' weights
        const int g = (t >= G.ts1) + (t >= G.ts2);
        const int tl = t - (g == 2 ? G.ts2 : g == 1 ? G.ts1 : 0);
        const float *bias = g == 2 ? G.b2 : g == 1 ? G.b1 : G.b0;
        const int N = g == 2 ? G.N2 : g == 1 ? G.N1 : G.N0;
        float bz = 0.f;
        if (bias && threadIdx.x < GV_ROWS * 8 && (int64_t)tl * GV_ROWS + (threadIdx.x >> 3) < N)
            bz = bias[(int64_t)tl * GV_ROWS + (threadIdx.x >> 3)];
        load(ring[PF], t + PF * (int)gridDim.x);
        W (&cur)[SBW] = ring[0];
        float part[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < SBW; i++)
            if (live[i]) {
                if constexpr (Q4) q4_compute(L, cur[i], act[i], part);
                else q6_compute(L, cur[i], act[i], part);
            }
        const int buf = it & 1;
        if (L.col < 8) {
#pragma unroll
            for (int i = 0; i < 4; i++) red[buf][L.wave][4 * L.q + i][L.col] = part[i];
        }
        __syncthreads();
        if (threadIdx.x < GV_ROWS * 8) {
            const int rr = threadIdx.x >> 3, mm = threadIdx.x & 7;
            float sum = 0.f;
#pragma unroll
            for (int w = 0; w < 8; w++) sum += red[buf][w][rr][mm];
            const int64_t row = (int64_t)tl * GV_ROWS + rr;
            float *y = g == 2 ? G.y2 : g == 1 ? G.y1 : G.y0;
            const int64_t ldy = g == 2 ? G.ld2 : g == 1 ? G.ld1 : G.ld0;
            if (row < N && mm < M) y[(int64_t)mm * ldy + row] = bias ? sum + bz : sum;
        }
#pragma unroll
        for (int f = 0; f < PF; f++)
#pragma unroll
            for (int i = 0; i < SBW; i++) ring[f][i] = ring[f + 1][i];
    }
}

// Any K: per tile, wave w walks superblocks w, w + 8, ... building their activation
// operands as it goes (no operand cache, no prefetch beyond what the waves overlap).
template <int TYPE>
__global__ __launch_bounds__(512) void k_gemv_kq_any(const uint8_t *__restrict__ gv, const int8_t *__restrict__ xq,
                                                     const float *__restrict__ xd, const void *__restrict__ xaux,
                                                     float *__restrict__ y, int N, int K, int M, int64_t ldy,
                                                     const float *__restrict__ bias) {
    constexpr bool Q4 = TYPE == MQ_TYPE_Q4_K;
    constexpr int BYTES = Q4 ? GV4_BYTES : GV6_BYTES;
    __shared__ float red[8][GV_ROWS][8];
    const GvLane L = gv_lane(M);
    const int nsb = K / QK_K;
    const int t = blockIdx.x;
    float part[4] = {0.f, 0.f, 0.f, 0.f};
    for (int sb = L.wave; sb < nsb; sb += 8) {
        const uint8_t *T = gv + ((int64_t)t * nsb + sb) * BYTES;
        if constexpr (Q4) q4_compute(L, q4_load(L, T), q4_act(L, xq, xd, (const _Float16 *)xaux, K, M, sb), part);
        else q6_compute(L, q6_load(L, T), q6_act(L, xq, xd, xaux, K, M, sb), part);
    }
    if (L.col < 8) {
#pragma unroll
        for (int i = 0; i < 4; i++) red[L.wave][4 * L.q + i][L.col] = part[i];
    }
    __syncthreads();
    if (threadIdx.x < GV_ROWS * 8) {
        const int rr = threadIdx.x >> 3, mm = threadIdx.x & 7;
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < 8; w++) sum += red[w][rr][mm];
        const int64_t row = (int64_t)t * GV_ROWS + rr;
        if (row < N && mm < M) y[(int64_t)mm * ldy + row] = bias ? sum + bias[row] : sum;
    }
}

template <int TYPE>
static hipError_t launch_kq_stream_groups(const GvGroups &G, const int8_t *xq, const float *xd, const void *xaux,
                                          int64_t k, int m, hipStream_t s, const GvX *X = nullptr);

template <int TYPE>
static hipError_t launch_kq_stream(const uint8_t *gv, const int8_t *xq, const float *xd, const void *xaux, float *y,
                                   int64_t n, int64_t k, int m, int64_t ldy, const float *bias, hipStream_t s) {
    const int64_t ntiles = (n + GV_ROWS - 1) / GV_ROWS;
    const int nsb = (int)(k / QK_K);
    if ((nsb + 7) / 8 > 3) {  // K > 6144: no operand cache
        hipLaunchKernelGGL((k_gemv_kq_any<TYPE>), dim3((unsigned)ntiles), dim3(512), 0, s, gv, xq, xd, xaux, y, (int)n,
                           (int)k, m, ldy, bias);
        return hipGetLastError();
    }
    GvGroups G{};
    G.gv0 = gv, G.y0 = y, G.b0 = bias, G.N0 = (int)n, G.ld0 = ldy;
    G.ts1 = G.ts2 = INT_MAX;
    G.tend = (int)ntiles;
    return launch_kq_stream_groups<TYPE>(G, xq, xd, xaux, k, m, s);
}

template <int TYPE>
static hipError_t launch_kq_stream_groups(const GvGroups &G, const int8_t *xq, const float *xd, const void *xaux,
                                          int64_t k, int m, hipStream_t s, const GvX *X) {
    const int64_t ntiles = G.tend;
    const int nsb = (int)(k / QK_K);
    const int sbw = (nsb + 7) / 8;
    static std::atomic<int> ncu_cache{0};  // the CU count (the same on every MI355X)
    int ncu = ncu_cache.load(std::memory_order_relaxed);
    if (!ncu) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
            v = 256;
        ncu = v;
        ncu_cache.store(v, std::memory_order_relaxed);
    }
    // workgroups per CU (at most what fits: two at one cached superblock per wave, one
    // beyond, register-bound); MQ_GEMV_WGS overrides for measurements
    int per_cu = sbw == 1 ? 2 : 1;
    if (const char *e = getenv("MQ_GEMV_WGS"))
        if (atoi(e) >= 1 && atoi(e) <= 4) per_cu = atoi(e);
    const unsigned grid = (unsigned)std::min<int64_t>(ntiles, (int64_t)ncu * per_cu);
    const dim3 block(512);
    // tiles in flight ahead of the one computed (MQ_GEMV_PF: 1, 2 or 3 for measurements).  One:
    // MI355X, Q6_K lm_head 151936 x 2048 at m = 1 45.9 -> 44.6 us, m = 8 53.3 -> 52.6 us; the
    // Q4_K layer sweep's separate-quantizer form 41.4 -> 34.8 us per layer (self-quantizing
    // form unchanged) against two.
    const char *pe = getenv("MQ_GEMV_PF");
    const int pf = pe && *pe ? atoi(pe) : 1;
    if (X) {  // the activation quantized inside the kernel
        const GvX x = *X;
        switch (sbw) {
            case 1:
                if (pf == 1)
                    hipLaunchKernelGGL((k_gemv_kq_stream<TYPE, 1, 1, true>), dim3(grid), block, 0, s, G, xq, xd, xaux, (int)k, m, x);
                else
                    hipLaunchKernelGGL((k_gemv_kq_stream<TYPE, 1, 2, true>), dim3(grid), block, 0, s, G, xq, xd, xaux, (int)k, m, x);
                break;
            case 2:
                hipLaunchKernelGGL((k_gemv_kq_stream<TYPE, 2, 1, true>), dim3(grid), block, 0, s, G, xq, xd, xaux, (int)k, m, x);
                break;
            case 3:
                hipLaunchKernelGGL((k_gemv_kq_stream<TYPE, 3, 1, true>), dim3(grid), block, 0, s, G, xq, xd, xaux, (int)k, m, x);
                break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    if (pf == 3 && sbw == 1) {
        hipLaunchKernelGGL((k_gemv_kq_stream<TYPE, 1, 3>), dim3(grid), block, 0, s, G, xq, xd, xaux, (int)k, m);
        return hipGetLastError();
    }
    if (pf == 2 && sbw == 1) {
        hipLaunchKernelGGL((k_gemv_kq_stream<TYPE, 1, 2>), dim3(grid), block, 0, s, G, xq, xd, xaux, (int)k, m);
        return hipGetLastError();
    }
    switch (sbw) {
        case 1: hipLaunchKernelGGL((k_gemv_kq_stream<TYPE, 1, 1>), dim3(grid), block, 0, s, G, xq, xd, xaux, (int)k, m); break;
        case 2: hipLaunchKernelGGL((k_gemv_kq_stream<TYPE, 2, 1>), dim3(grid), block, 0, s, G, xq, xd, xaux, (int)k, m); break;
        case 3: hipLaunchKernelGGL((k_gemv_kq_stream<TYPE, 3, 1>), dim3(grid), block, 0, s, G, xq, xd, xaux, (int)k, m); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int MM>
static hipError_t gemv_launch(int type, const uint8_t *wb, const WeightPlanes &p, int64_t n, int64_t k, const uint8_t *xb,
                        const ActPlanes &ap, float *y, int64_t ldy, const float *bias, hipStream_t s) {
    const dim3 grid((unsigned)((n + 3) / 4)), block(256);
    const int8_t *xq = (const int8_t *)(xb + ap.xq);
    const float *xd = (const float *)(xb + ap.xd);
    const int16_t *xbs = (const int16_t *)(xb + ap.xbs);
    switch (type) {
        case MQ_TYPE_Q4_K: return launch_kq_stream<MQ_TYPE_Q4_K>(wb + p.gv, xq, xd, xb + ap.xgm, y, n, k, MM, ldy, bias, s);
        case MQ_TYPE_Q6_K: return launch_kq_stream<MQ_TYPE_Q6_K>(wb + p.gv, xq, xd, xbs, y, n, k, MM, ldy, bias, s);
        case MQ_TYPE_Q8_0:
            hipLaunchKernelGGL(k_gemv_q8_0<MM>, grid, block, 0, s, (const int8_t *)(wb + p.qs),
                               (const uint16_t *)(wb + p.d16), xq, xd, y, (int)n, (int)k, ldy, bias);
            break;
        case MQ_TYPE_F16:
            hipLaunchKernelGGL(k_gemv_f16<MM>, grid, block, 0, s, (const uint16_t *)wb, (const uint16_t *)xq, y, (int)n,
                               (int)k, ldy, bias);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipSuccess;
}

hipError_t launch_gemv_group(int type, int ng, const void *const *images, const int64_t *n, int64_t k, const void *ws,
                             int64_t m, float *const *y, const int64_t *ldy, const float *const *bias, hipStream_t s) {
    const int nsb = (int)(k / QK_K);
    bool one = (type == MQ_TYPE_Q4_K || type == MQ_TYPE_Q6_K) && ng >= 2 && ng <= 3 && m >= 1 && m <= GEMV_CHUNK &&
               (nsb + 7) / 8 <= 3;
    for (int g = 0; one && g < ng; g++) one = n[g] > 0;
    if (!one) {  // one launch per weight
        for (int g = 0; g < ng; g++) {
            const hipError_t e = launch_gemv(type, images[g], n[g], k, ws, m, y[g], ldy[g], s, bias ? bias[g] : nullptr);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    // the K-quant stream kernel over the concatenated row tiles of the weights
    const ActPlanes ap = act_planes(type, m, k, false);
    const uint8_t *xb = (const uint8_t *)ws;
    GvGroups G{};
    int ts[3] = {0, 0, 0}, t = 0;
    const uint8_t *gv[3] = {nullptr, nullptr, nullptr};
    for (int g = 0; g < ng; g++) {
        gv[g] = (const uint8_t *)images[g] + weight_planes(type, n[g], k).gv;
        ts[g] = t;
        t += (int)((n[g] + GV_ROWS - 1) / GV_ROWS);
    }
    G.gv0 = gv[0], G.gv1 = gv[1], G.gv2 = gv[2];
    G.y0 = y[0], G.y1 = y[1], G.y2 = ng > 2 ? y[2] : nullptr;
    G.b0 = bias ? bias[0] : nullptr, G.b1 = bias ? bias[1] : nullptr, G.b2 = (bias && ng > 2) ? bias[2] : nullptr;
    G.N0 = (int)n[0], G.N1 = (int)n[1], G.N2 = ng > 2 ? (int)n[2] : 0;
    G.ld0 = ldy[0], G.ld1 = ldy[1], G.ld2 = ng > 2 ? ldy[2] : 0;
    G.ts1 = ts[1], G.ts2 = ng > 2 ? ts[2] : INT_MAX, G.tend = t;
    const int8_t *xq = (const int8_t *)(xb + ap.xq);
    const float *xd = (const float *)(xb + ap.xd);
    if (type == MQ_TYPE_Q4_K) return launch_kq_stream_groups<MQ_TYPE_Q4_K>(G, xq, xd, xb + ap.xgm, k, (int)m, s);
    return launch_kq_stream_groups<MQ_TYPE_Q6_K>(G, xq, xd, xb + ap.xbs, k, (int)m, s);
}

bool gemv_fused_ok(int type, int ng, int64_t k, int64_t m) {
    return (type == MQ_TYPE_Q4_K || type == MQ_TYPE_Q6_K) && ng >= 1 && ng <= 3 && m >= 1 && m <= GEMV_CHUNK &&
           k % QK_K == 0 && (k / QK_K + 7) / 8 <= 3;
}

hipError_t launch_gemv_group_f32(int type, int ng, const void *const *images, const int64_t *n, int64_t k,
                                 const float *x, int64_t ldx, const float *x2, int64_t ldx2, int pre, int64_t m,
                                 float *const *y, const int64_t *ldy, const float *const *bias, hipStream_t s) {
    if (!gemv_fused_ok(type, ng, k, m) || (pre != MQ_PRE_NONE && pre != MQ_PRE_SILU_MUL) ||
        (pre == MQ_PRE_SILU_MUL && !x2) || ((uintptr_t)x & 15) || (ldx & 3) || (x2 && (((uintptr_t)x2 & 15) || (ldx2 & 3))))
        return hipErrorInvalidValue;
    GvGroups G{};
    int ts[3] = {0, 0, 0}, t = 0;
    const uint8_t *gv[3] = {nullptr, nullptr, nullptr};
    for (int g = 0; g < ng; g++) {
        if (n[g] <= 0) return hipErrorInvalidValue;
        gv[g] = (const uint8_t *)images[g] + weight_planes(type, n[g], k).gv;
        ts[g] = t;
        t += (int)((n[g] + GV_ROWS - 1) / GV_ROWS);
    }
    G.gv0 = gv[0], G.gv1 = gv[1], G.gv2 = gv[2];
    G.y0 = y[0], G.y1 = ng > 1 ? y[1] : nullptr, G.y2 = ng > 2 ? y[2] : nullptr;
    G.b0 = bias ? bias[0] : nullptr, G.b1 = (bias && ng > 1) ? bias[1] : nullptr, G.b2 = (bias && ng > 2) ? bias[2] : nullptr;
    G.N0 = (int)n[0], G.N1 = ng > 1 ? (int)n[1] : 0, G.N2 = ng > 2 ? (int)n[2] : 0;
    G.ld0 = ldy[0], G.ld1 = ng > 1 ? ldy[1] : 0, G.ld2 = ng > 2 ? ldy[2] : 0;
    G.ts1 = ng > 1 ? ts[1] : INT_MAX, G.ts2 = ng > 2 ? ts[2] : INT_MAX, G.tend = t;
    const GvX X{x, x2, ldx, ldx2, pre};
    if (type == MQ_TYPE_Q4_K) return launch_kq_stream_groups<MQ_TYPE_Q4_K>(G, nullptr, nullptr, nullptr, k, (int)m, s, &X);
    return launch_kq_stream_groups<MQ_TYPE_Q6_K>(G, nullptr, nullptr, nullptr, k, (int)m, s, &X);
}

hipError_t launch_gemv(int type, const void *image, int64_t n, int64_t k, const void *ws, int64_t m, float *y,
                       int64_t ldy, hipStream_t s, const float *bias) {
    if (m <= 0 || n <= 0) return hipSuccess;
    if (m > GEMV_MAX_M) return hipErrorInvalidValue;
    if (m > GEMV_CHUNK) {  // 8 rows per launch, each on its own chunk of the activation layout
        const size_t cb = gemv_chunk_bytes(type, k);
        for (int64_t r0 = 0, c = 0; r0 < m; r0 += GEMV_CHUNK, c++) {
            const hipError_t e = launch_gemv(type, image, n, k, (const uint8_t *)ws + c * cb,
                                             std::min<int64_t>(GEMV_CHUNK, m - r0), y + r0 * ldy, ldy, s, bias);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    const WeightPlanes p = weight_planes(type, n, k);
    const ActPlanes ap = act_planes(type, m, k, false);
    const uint8_t *wb = (const uint8_t *)image;
    const uint8_t *xb = (const uint8_t *)ws;
    hipError_t e = hipErrorInvalidValue;
    switch (m) {
        case 1: e = gemv_launch<1>(type, wb, p, n, k, xb, ap, y, ldy, bias, s); break;
        case 2: e = gemv_launch<2>(type, wb, p, n, k, xb, ap, y, ldy, bias, s); break;
        case 3: e = gemv_launch<3>(type, wb, p, n, k, xb, ap, y, ldy, bias, s); break;
        case 4: e = gemv_launch<4>(type, wb, p, n, k, xb, ap, y, ldy, bias, s); break;
        case 5: e = gemv_launch<5>(type, wb, p, n, k, xb, ap, y, ldy, bias, s); break;
        case 6: e = gemv_launch<6>(type, wb, p, n, k, xb, ap, y, ldy, bias, s); break;
        case 7: e = gemv_launch<7>(type, wb, p, n, k, xb, ap, y, ldy, bias, s); break;
        case 8: e = gemv_launch<8>(type, wb, p, n, k, xb, ap, y, ldy, bias, s); break;
        default: break;
    }
    if (e != hipSuccess) return e;
    return hipGetLastError();
}

}  // namespace mq
