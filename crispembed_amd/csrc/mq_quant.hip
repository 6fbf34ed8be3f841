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
#include <algorithm>

#include "mq_internal.h"
#include "mq_act.h"
#include "mq_deq.h"
#include "mq_q8k.h"

namespace mq {


template <bool VEC4>
__device__ __forceinline__ float4 load4(const float *p) {
    if (VEC4) return *(const float4 *)p;
    return make_float4(p[0], p[1], p[2], p[3]);
}

// Prologue applied to an activation before it is quantized (the graph's elementwise
// producers of the MUL_MAT input, fused): v = x + bias[col] (bias may be NULL), then
//   MQ_PRE_GELU_ERF : v = 0.5 v (1 + erf(v / sqrt 2))            (ggml_gelu_erf)
//   MQ_PRE_SILU_MUL : v = silu(v) * u, u the value uoff floats after v (ggml_silu, ggml_mul:
//                     the gate projection's value and the up projection's; uoff = k when a row
//                     holds the gate projection, then the up projection)
// all in fp32.  `pre` and `bias` are uniform: the branches cost nothing without a prologue.
template <bool VEC4>
__device__ __forceinline__ float4 pre_load(const float *p, int pre, const float *bias, int64_t col, int64_t uoff) {
    const float4 v = load4<VEC4>(p);
    if (pre == MQ_PRE_NONE && bias == nullptr) return v;
    float r[4] = {v.x, v.y, v.z, v.w}, u[4] = {1.f, 1.f, 1.f, 1.f};
    if (pre == MQ_PRE_SILU_MUL) {
        const float4 w = load4<VEC4>(p + uoff);
        u[0] = w.x, u[1] = w.y, u[2] = w.z, u[3] = w.w;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (bias) r[i] = r[i] + bias[col + i];
        if (pre == MQ_PRE_GELU_ERF) r[i] = gelu_erf_f32(r[i]);
        else if (pre == MQ_PRE_SILU_MUL) r[i] = silu_mul_f32(r[i], u[i]);
    }
    return make_float4(r[0], r[1], r[2], r[3]);
}

// Output layouts of the activation quantizers.
enum { OUT_GGUF = 0, OUT_ROWS = 1 };

// ---------------------------------------------------------------------------
// Q8_0 activations: quantize_row_q8_0 (variant selects the rounding).
// Lanes 8g..8g+7 of a wave own one 32-value block.
// OUT_ROWS : xq int8 [m][k] + xd float [m][k/32]
// OUT_GGUF : block_q8_0 rows
// (the tiled GEMM layout is written by k_quantize_tiled below)
// ---------------------------------------------------------------------------
template <int VARIANT, int OUT, bool VEC4>
__global__ __launch_bounds__(256) void k_quantize_q8_0(const float *__restrict__ x, int64_t ldx,
                                                       int8_t *__restrict__ out, float *__restrict__ xd,
                                                       int64_t m, int64_t k, int64_t m_pad, int64_t kb_pad, int pre,
                                                       const float *__restrict__ bias, int64_t uoff) {
    const int64_t nbr = k / QK8_0;
    const int64_t nbx = nbr;
    const int64_t rows = m;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t blk = gid >> 3;
    const int sub = (int)(gid & 7);
    if (blk >= rows * nbx) return;  // 8-lane groups leave together
    const int64_t row = blk / nbx, b = blk - row * nbx;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (row < m && b < nbr) v = pre_load<VEC4>(x + row * ldx + b * QK8_0 + sub * 4, pre, bias, b * QK8_0 + sub * 4, uoff);
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
    if (OUT == OUT_ROWS) {
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
// OUT_ROWS : xq int8 [m][k], xd float [m][k/256], xbs int16 [m][k/16]
// OUT_GGUF : block_q8_K rows
// ---------------------------------------------------------------------------
template <int OUT, bool VEC4>
__global__ __launch_bounds__(256) void k_quantize_q8_K(const float *__restrict__ x, int64_t ldx,
                                                       int8_t *__restrict__ out, float *__restrict__ xd,
                                                       int16_t *__restrict__ xbs, _Float16 *__restrict__ xmin,
                                                       int64_t m, int64_t k, int64_t m_pad, int pre,
                                                       const float *__restrict__ bias, int64_t uoff) {
    const int64_t nbr = k / QK_K;
    const int64_t rows = m;
    const int lane = threadIdx.x & 63;
    const int64_t blk = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (blk >= rows * nbr) return;  // whole waves leave together
    const int64_t row = blk / nbr, b = blk - row * nbr;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (row < m) v = pre_load<VEC4>(x + row * ldx + b * QK_K + lane * 4, pre, bias, b * QK_K + lane * 4, uoff);
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
    if (OUT == OUT_ROWS) {
        *(uint32_t *)(out + row * k + b * QK_K + lane * 4) = packed;
        if ((lane & 3) == 0) xbs[row * (k / 16) + b * 16 + (lane >> 2)] = (int16_t)s16;
        if (lane == 0) xd[row * nbr + b] = dval;
        // GEMV min-term operand (rows < 8): B_j = sum of the 32 quants of sub-block j, in lane 8j
        const int B = s16 + __shfl_xor(s16, 4);
        if (xmin != nullptr && row < 8 && (lane & 7) == 0) {
            const int j = lane >> 3;
            _Float16 *g = xmin + ((b * 8 + row) << 4);
            g[j] = (_Float16)(B & 63);
            g[j + 8] = (_Float16)((B >> 6) * 64);
        }
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
                                                      uint16_t *__restrict__ y, int64_t m, int64_t k, int pre,
                                                      const float *__restrict__ bias, int64_t uoff) {
    const int64_t q4 = k / 4;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= m * q4) return;
    const int64_t row = gid / q4, c = gid - row * q4;
    const float4 v = pre_load<VEC4>(x + row * ldx + c * 4, pre, bias, c * 4, uoff);
    uint16_t *o = y + row * k + c * 4;
    o[0] = f32_to_f16_bits(v.x);
    o[1] = f32_to_f16_bits(v.y);
    o[2] = f32_to_f16_bits(v.z);
    o[3] = f32_to_f16_bits(v.w);
}



// ---------------------------------------------------------------------------
// Activations into the tiled GEMM layout (1 KB fragments: lane L of a fragment
// holds row L%32, bytes 16*(L/32)..+16 of a 32-byte K chunk).  One workgroup
// per (32-row tile, CB bytes of K): it quantizes the 32 rows with the same
// per-block arithmetic as the row kernels above, assembles the CB/32 fragments
// in LDS and writes them as whole 1 KB fragments (16 bytes per lane, fully
// coalesced), then the scales (32 consecutive floats per block) and, for
// Q8_K, the min-term fragment.  Rows past m and K bytes past the row are
// written as zeros (d = 0).
//   Q8_0 (TQ_Q8_0): CB = 128 (4 blocks per row), xd float [kb_pad/32][m_pad]
//   Q8_K (TQ_Q8_K): CB = 256 (one superblock), xd float [k/256][m_pad], and
//        the min-term fragment of (tile, superblock): halves (r, j) = B_j & 63
//        and (32 + r, j) = 64*(B_j >> 6), B_j = sum of the 32 quants of
//        sub-block j (exact in fp16)
//   F16  (TQ_F16) : CB = 128 (64 values per row)
// ---------------------------------------------------------------------------
enum { TQ_Q8_0 = 0, TQ_Q8_K = 1, TQ_F16 = 2 };

// RPW rows per wave: 8 (a workgroup per 32-row tile and CB-byte column block), 2 or 1 (Q8_K:
// 4 or 8 workgroups per tile, the RW = 4 RPW rows RW q .. RW q + RW - 1 in workgroup q, each
// writing only its rows' 16-byte units of the fragments, scales and min-term halves: shorter
// dependency chains per wave and more workgroups to spread).
template <int FMT, int VARIANT, bool VEC4, int RPW = 8>
__global__ __launch_bounds__(256) void k_quantize_tiled(const float *__restrict__ x, int64_t ldx,
                                                        int8_t *__restrict__ xq, float *__restrict__ xd,
                                                        _Float16 *__restrict__ xmin, int64_t m, int64_t k,
                                                        int64_t m_pad, int64_t kb_pad, int pre,
                                                        const float *__restrict__ bias, int64_t uoff) {
    constexpr int CB = (FMT == TQ_Q8_K) ? 256 : 128;   // K bytes per workgroup
    constexpr int BPV = (FMT == TQ_F16) ? 2 : 1;       // bytes per value
    constexpr int NCH = CB / 32;                        // fragments per workgroup
    constexpr int LPR = CB / (4 * BPV);                 // lanes per row (4 values each)
    constexpr int RPI = 64 / LPR;                       // rows per wave pass
    constexpr int FST = 1024 + 16;                      // padded fragment stride (LDS banks)
    constexpr int NSC = (FMT == TQ_Q8_0) ? NCH : (FMT == TQ_Q8_K ? 1 : 0);  // scale rows
    __shared__ __attribute__((aligned(16))) int8_t frag[NCH * FST];
    __shared__ float dsh[NSC > 0 ? NSC : 1][32];
    __shared__ __attribute__((aligned(16))) _Float16 msh[FMT == TQ_Q8_K ? 512 : 8];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int RW = 4 * RPW, WPT = 32 / RW;          // rows per workgroup, workgroups per tile
    const int64_t ncb = kb_pad / CB;
    const int64_t unit = blockIdx.x / WPT;
    const int64_t rt = unit / ncb, cb = unit - rt * ncb;
    const int rbase = RW * (int)(blockIdx.x % WPT);     // the workgroup's first row in the tile
    const int sub = lane % LPR, rsub = lane / LPR;
    const int kbyte = sub * 4 * BPV;                    // byte of this lane's 4 values within CB
    const int c = kbyte >> 5, cbyte = kbyte & 31;       // fragment, byte within the 32-byte chunk
    static_assert(RPW == 8 || RPW == 2 || RPW == 1, "8, 2 or 1 rows per wave");
    static_assert(RPW % RPI == 0, "whole wave passes");
    constexpr int NIT = RPW / RPI;                      // rows per lane
    const int64_t kv = (cb * CB + kbyte) / BPV;         // first value index of this lane
    float4 vin[NIT];                                    // every load in flight before any math
    if (pre == MQ_PRE_NONE && bias == nullptr) {
        // the plain loads on their own (uniform branch): with the prologue's code in the same
        // loop the compiler no longer issues all NIT loads before the first use
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            const int64_t row = rt * 32 + rbase + wave * RPW + it * RPI + rsub;
            vin[it] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (row < m && kv < k) vin[it] = load4<VEC4>(x + row * ldx + kv);
        }
    } else {
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            const int64_t row = rt * 32 + rbase + wave * RPW + it * RPI + rsub;
            vin[it] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (row < m && kv < k) vin[it] = pre_load<VEC4>(x + row * ldx + kv, pre, bias, kv, uoff);
        }
    }
    if constexpr (FMT == TQ_Q8_K) {  // one superblock per row, a row per wave pass (RPI = 1)
        int rr[NIT];
        int8_t *dd[NIT];
        float *ds[NIT];
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            rr[it] = rbase + wave * RPW + it * RPI + rsub;
            dd[it] = frag + c * FST + ((rr[it] + 32 * (cbyte >> 4)) << 4) + (cbyte & 15);
            ds[it] = &dsh[0][rr[it]];
        }
        q8_K_block_rows<NIT>(vin, lane, rr, dd, ds, msh);
    }
#pragma unroll
    for (int it = 0; it < NIT && FMT != TQ_Q8_K; it++) {
        const int r = rbase + wave * RPW + it * RPI + rsub;  // row within the tile
        const float4 v = vin[it];
        int8_t *dst = frag + c * FST + ((r + 32 * (cbyte >> 4)) << 4) + (cbyte & 15);
        if constexpr (FMT == TQ_F16) {
            uint2 o;
            o.x = (uint32_t)f32_to_f16_bits(v.x) | ((uint32_t)f32_to_f16_bits(v.y) << 16);
            o.y = (uint32_t)f32_to_f16_bits(v.z) | ((uint32_t)f32_to_f16_bits(v.w) << 16);
            *(uint2 *)dst = o;
        } else if constexpr (FMT == TQ_Q8_0) {
            const float amax = max8(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
            const float d = amax / 127.f;
            float id;
            if (VARIANT == MQ_Q8_0_X86) id = (amax != 0.0f) ? 127.f / amax : 0.0f;
            else id = (d != 0.0f) ? 1.0f / d : 0.0f;
            auto q = [&](float xv) -> uint32_t {
                const float t = xv * id;
                float rr = (VARIANT == MQ_Q8_0_REF) ? roundf(t) : rintf(t);
                rr = fminf(fmaxf(rr, -128.f), 127.f);
                return (uint32_t)((int)rr & 0xff);
            };
            *(uint32_t *)dst = q(v.x) | (q(v.y) << 8) | (q(v.z) << 16) | (q(v.w) << 24);
            if ((sub & 7) == 0) dsh[c][r] = f16_bits_to_f32(f32_to_f16_bits(d));
        }
    }
    __syncthreads();
    // the 16-byte units of the workgroup's rows rbase .. rbase + RW - 1: lanes rbase + i and
    // 32 + rbase + i of each fragment (all 64 lanes when RW = 32: whole 1 KB fragments)
    const int t = threadIdx.x;
#pragma unroll
    for (int p = t; p < NCH * 2 * RW; p += 256) {
        const int f = p / (2 * RW), u = p % (2 * RW), L = rbase + u % RW + 32 * (u / RW);
        const int4 val = *(const int4 *)(frag + f * FST + L * 16);
        *(int4 *)(xq + ((rt * (kb_pad >> 5) + cb * NCH + f) << 10) + L * 16) = val;
    }
    if constexpr (NSC > 0) {
        if (t < NSC * RW) xd[(cb * NSC + t / RW) * m_pad + rt * 32 + rbase + t % RW] = dsh[t / RW][rbase + t % RW];
    }
    if constexpr (FMT == TQ_Q8_K) {
        if (t < 2 * RW) {
            const int e = rbase + t % RW + 32 * (t / RW);
            ((int4 *)(xmin + ((rt * ncb + cb) << 9)))[e] = ((const int4 *)msh)[e];
        }
    }
}

// ---------------------------------------------------------------------------
// Residual ADD + RMS norm whose normed rows also leave as the Q8_K activation of the mat-mul
// that reads them (the decoder's attn_norm / ffn_norm before the qkv and gate|up products):
//   x = y + res (written to xout), h = x / sqrt(mean(x^2) + eps) * w (written to hout unless NULL),
// and h quantized into the tiled GEMM layout exactly as k_quantize_tiled<TQ_Q8_K> quantizes it.
// Workgroup: 8 rows of a 32-row tile (four workgroups per tile, so a 512-row input still spreads
// over 64 CUs), a wave per row with every load in flight before the first use, lane l holding
// the values 256 p + 4 l .. + 3 of superblock p, which is the tiled quantizer's lane layout; the
// workgroup writes its rows' 16-byte units of each fragment, scales and min-term halves.
// ---------------------------------------------------------------------------
template <int NSB>
__global__ __launch_bounds__(512) void k_add_rmsnorm_q8_K(const float *y, const float *res, const float *__restrict__ w,
                                                          float eps, float *xout, float *hout, int64_t rows,
                                                          int8_t *__restrict__ xq, float *__restrict__ xd,
                                                          _Float16 *__restrict__ xmin, int64_t m_pad) {
    constexpr int H = 256 * NSB, NCH = H / 32, FST = 1024 + 16;
    __shared__ __attribute__((aligned(16))) int8_t frag[NCH * FST];
    __shared__ float dsh[NSB][32];
    __shared__ __attribute__((aligned(16))) _Float16 msh[NSB][512];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t rt = blockIdx.x >> 2;      // 32-row tile
    const int r0 = (int)(blockIdx.x & 3) * 8;  // this workgroup's 8 rows of it, one per wave
    const int r = r0 + wave;
    const int64_t row = rt * 32 + r;
    const bool live = row < rows;
    float4 v[NSB];
#pragma unroll
    for (int p = 0; p < NSB; p++) {  // every load in flight before the first use
        v[p] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (live) {
            const int64_t o = row * H + 256 * p + 4 * lane;
            float4 a = *(const float4 *)(y + o);
            if (res) {
                const float4 c = *(const float4 *)(res + o);
                a.x = a.x + c.x, a.y = a.y + c.y, a.z = a.z + c.z, a.w = a.w + c.w;
            }
            v[p] = a;
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int p = 0; p < NSB; p++) ss += v[p].x * v[p].x + v[p].y * v[p].y + v[p].z * v[p].z + v[p].w * v[p].w;
    ss += __shfl_xor(ss, 32);
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 8);
    ss += __shfl_xor(ss, 4);
    ss += __shfl_xor(ss, 2);
    ss += __shfl_xor(ss, 1);
    const float scale = 1.0f / sqrtf(ss / (float)H + eps);
    const int cbyte = 4 * (lane & 7);
#pragma unroll
    for (int p = 0; p < NSB; p++) {
        const float4 wv = *(const float4 *)(w + 256 * p + 4 * lane);
        float4 h;
        h.x = v[p].x * scale * wv.x, h.y = v[p].y * scale * wv.y;
        h.z = v[p].z * scale * wv.z, h.w = v[p].w * scale * wv.w;
        if (live) {
            const int64_t o = row * H + 256 * p + 4 * lane;
            if (xout) *(float4 *)(xout + o) = v[p];
            if (hout) *(float4 *)(hout + o) = h;
        } else {
            h = make_float4(0.f, 0.f, 0.f, 0.f);  // pad rows of the tile quantize to zero
        }
        int8_t *dst = frag + (8 * p + (lane >> 3)) * FST + ((r + 32 * (cbyte >> 4)) << 4) + (cbyte & 15);
        q8_K_block_row(h, lane, r, dst, &dsh[p][r], msh[p]);
    }
    __syncthreads();
    // this workgroup's lane units of every fragment: rows r0 .. r0 + 7, both 16-byte halves
    const int t = threadIdx.x;
    for (int q = t; q < NCH * 16; q += 512) {
        const int f = q >> 4, u = q & 15, L = r0 + (u & 7) + 32 * (u >> 3);
        *(int4 *)(xq + ((rt * NCH + f) << 10) + L * 16) = *(const int4 *)(frag + f * FST + L * 16);
    }
    for (int q = t; q < NSB * 8; q += 512) xd[(int64_t)(q >> 3) * m_pad + rt * 32 + r0 + (q & 7)] = dsh[q >> 3][r0 + (q & 7)];
    // min-term fragment halves (row, j) and (32 + row, j): two runs of 8 rows x 8 halves = 16 x 8 bytes
    for (int q = t; q < NSB * 16; q += 512) {
        const int p = q >> 4, u = q & 15, hr = r0 + (u & 7) + 32 * (u >> 3);
        *(int4 *)(xmin + ((rt * NSB + p) << 9) + hr * 8) = *(const int4 *)(&msh[p][hr * 8]);
    }
}

hipError_t launch_add_rmsnorm_q8_K(const float *y, const float *res, const float *w, float eps, float *xout,
                                   float *hout, int64_t rows, int H, void *ws, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (H % 256 != 0 || H > 2048 || ((uintptr_t)ws & 255) || ((uintptr_t)y | (uintptr_t)res | (uintptr_t)w |
                                                                (uintptr_t)xout | (uintptr_t)hout) & 15)
        return hipErrorInvalidValue;
    const ActPlanes ap = act_planes(MQ_TYPE_Q4_K, rows, H, true);
    uint8_t *b = (uint8_t *)ws;
    int8_t *xq = (int8_t *)(b + ap.xq);
    float *xd = (float *)(b + ap.xd);
    _Float16 *xm = (_Float16 *)(b + ap.xmin);
    const dim3 g((unsigned)((rows + 31) / 32 * 4)), blk(512);
    switch (H / 256) {
#define MQ_RQ(N)                                                                                                       \
    case N:                                                                                                            \
        hipLaunchKernelGGL((k_add_rmsnorm_q8_K<N>), g, blk, 0, s, y, res, w, eps, xout, hout, rows, xq, xd, xm,         \
                           ap.m_pad);                                                                                  \
        break;
        MQ_RQ(1) MQ_RQ(2) MQ_RQ(3) MQ_RQ(4) MQ_RQ(5) MQ_RQ(6) MQ_RQ(7) MQ_RQ(8)
#undef MQ_RQ
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Dequantization (ggml to_float), one thread per output value.
// ---------------------------------------------------------------------------
template <int TYPE, bool FUSED>
__global__ __launch_bounds__(256) void k_dequantize(const uint8_t *__restrict__ w, float *__restrict__ y,
                                                    int64_t nrows, int64_t k) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= nrows * k) return;
    const int64_t row = gid / k, col = gid - row * k;
    y[gid] = deq_elem<TYPE, FUSED>(w + row * deq_row_bytes<TYPE>(k), col);
}

// ---------------------------------------------------------------------------
// Weight-plane preparation.  GEMV planes: one thread per (row, GGUF block) for
// rows [row0, row1).  GEMM planes: one thread per (row, block) for rows
// [row0, row_end) where row_end extends to n_pad when the range reaches n, so the
// padding rows (and the K padding) are written as zeros.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_prepare_q8_0_rows(const uint8_t *__restrict__ gguf, int8_t *__restrict__ qs,
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

__global__ __launch_bounds__(256) void k_prepare_q8_0_tiled(const uint8_t *__restrict__ gguf, int8_t *__restrict__ tq,
                                                            float *__restrict__ tdw, int64_t n, int64_t row0,
                                                            int64_t row_end, int64_t k, int64_t n_pad,
                                                            int64_t kb_pad) {
    const int64_t nbr = k / QK8_0, nbx = kb_pad / QK8_0;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (row_end - row0) * nbx) return;
    const int64_t row = row0 + gid / nbx, b = gid % nbx;
    uint32_t w[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float d = 0.f;
    if (row < n && b < nbr) {
        const uint8_t *src = gguf + (row * nbr + b) * sizeof(block_q8_0);
        d = f16_bits_to_f32(*(const uint16_t *)src);
        const uint16_t *s16 = (const uint16_t *)(src + 2);
#pragma unroll
        for (int i = 0; i < 8; i++) w[i] = (uint32_t)s16[2 * i] | ((uint32_t)s16[2 * i + 1] << 16);
    }
    *(uint4 *)(tq + tiled_off(row, b * QK8_0, kb_pad)) = make_uint4(w[0], w[1], w[2], w[3]);
    *(uint4 *)(tq + tiled_off(row, b * QK8_0 + 16, kb_pad)) = make_uint4(w[4], w[5], w[6], w[7]);
    tdw[b * n_pad + row] = d;
}

__device__ __forceinline__ uint4 pack16(const int *v) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        w[i] = (uint32_t)(v[4 * i] & 0xff) | ((uint32_t)(v[4 * i + 1] & 0xff) << 8) |
               ((uint32_t)(v[4 * i + 2] & 0xff) << 16) | ((uint32_t)(v[4 * i + 3] & 0xff) << 24);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// The weight-prepare kernels run one thread per (row, superblock); the workgroup's 256
// consecutive GGUF blocks are first copied to LDS with coalesced 2-byte loads (blocks are
// 2-byte aligned), so each thread's many small reads of its block hit LDS, not memory.
// Blocks [b0, b1) exist in the GGUF part (rows < n); the copy is done by every thread.
template <int BB>
__device__ __forceinline__ void stage_blocks(const uint8_t *gguf, int64_t b0, int64_t b1, uint8_t *lds) {
    static_assert(BB % 2 == 0, "2-byte units");
    const int64_t nunits = b1 > b0 ? (b1 - b0) * (BB / 2) : 0;
    const uint16_t *src = (const uint16_t *)(gguf + b0 * BB);
    uint16_t *dst = (uint16_t *)lds;
    for (int64_t i = threadIdx.x; i < nunits; i += blockDim.x) dst[i] = src[i];
    __syncthreads();
}

// Q4_K: limbs of sc_j * q4 (lo = v & 127, hi = v >> 7), per-superblock scales, min fragment.
__global__ __launch_bounds__(256) void k_prepare_q4_K_tiled(const uint8_t *__restrict__ gguf, int8_t *__restrict__ tlo,
                                                            int8_t *__restrict__ thi, float *__restrict__ tdw,
                                                            float *__restrict__ tdmin, _Float16 *__restrict__ tmin,
                                                            int64_t n, int64_t row0, int64_t row_end, int64_t k,
                                                            int64_t n_pad) {
    const int64_t nbr = k / QK_K;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    __shared__ __attribute__((aligned(16))) uint8_t sblk[256 * sizeof(block_q4_K)];
    const int64_t gb0 = row0 * nbr + (int64_t)blockIdx.x * blockDim.x;
    stage_blocks<sizeof(block_q4_K)>(gguf, gb0, min(gb0 + (int64_t)blockDim.x, min(row_end, n) * nbr), sblk);
    if (gid >= (row_end - row0) * nbr) return;
    const int64_t row = row0 + gid / nbr, b = gid % nbr;
    const bool valid = row < n;
    const uint8_t *src = sblk + threadIdx.x * sizeof(block_q4_K);
    int sc[8], mn[8];
    float d = 0.f, dmin = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) sc[j] = mn[j] = 0;
    if (valid) {
        d = f16_bits_to_f32(*(const uint16_t *)src);
        dmin = f16_bits_to_f32(*(const uint16_t *)(src + 2));
#pragma unroll
        for (int j = 0; j < 8; j++) scale_min_k4(j, src + 4, sc[j], mn[j]);
    }
    tdw[b * n_pad + row] = d;
    tdmin[b * n_pad + row] = dmin;
    _Float16 *frag = tmin + (((row >> 5) * nbr + b) << 9);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        frag[((row & 31) << 3) + j] = (_Float16)mn[j];
        frag[((32 + (row & 31)) << 3) + j] = (_Float16)mn[j];
    }
    for (int t = 0; t < 16; t++) {  // 16 chunks of 16 values
        const int c = t >> 2, part = t & 3;
        const int j = 2 * c + (part >> 1);
        int lo[16], hi[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            int q = 0;
            if (valid) {
                const uint8_t byte = src[16 + 32 * c + 16 * (part & 1) + i];
                q = (part < 2) ? (byte & 0xF) : (byte >> 4);
            }
            const int v = sc[j] * q;
            lo[i] = v & 127;
            hi[i] = v >> 7;
        }
        const int64_t off = tiled_off(row, b * QK_K + 16 * t, k);
        *(uint4 *)(tlo + off) = pack16(lo);
        *(uint4 *)(thi + off) = pack16(hi);
    }
}

// Q6_K GEMV plane (layout in mq_internal.h): one thread per (row, superblock).
__device__ __forceinline__ int q6_value(const uint8_t *blk, int e) {  // unsigned 6-bit quant of value e
    const int h = e >> 7, lp = e & 127, s = lp >> 5, l = lp & 31;
    const int qlb = blk[64 * h + (s & 1) * 32 + l];
    const int lo = (s >> 1) ? (qlb >> 4) : (qlb & 15);
    return lo | (((blk[128 + 32 * h + l] >> (2 * s)) & 3) << 4);
}

__global__ __launch_bounds__(256) void k_prepare_q6_K_gv(const uint8_t *__restrict__ gguf, uint8_t *__restrict__ gv,
                                                         int64_t n, int64_t row0, int64_t row1, int64_t k) {
    const int64_t nsb = k / QK_K;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    __shared__ __attribute__((aligned(16))) uint8_t sblk[256 * sizeof(block_q6_K)];
    const int64_t gb0 = row0 * nsb + (int64_t)blockIdx.x * blockDim.x;
    stage_blocks<sizeof(block_q6_K)>(gguf, gb0, min(gb0 + (int64_t)blockDim.x, min(row1, n) * nsb), sblk);
    const int64_t row = row0 + t / nsb, sb = t % nsb;
    if (row >= row1) return;
    const int r = (int)(row % GV_ROWS);
    uint8_t *T = gv + ((row / GV_ROWS) * nsb + sb) * GV6_BYTES;
    const bool live = row < n;
    const uint8_t *blk = sblk + threadIdx.x * sizeof(block_q6_K);
    for (int p = 0; p < 4; p++) {
        uint32_t his[4] = {0, 0, 0, 0};
        for (int kk = 0; kk < 8; kk++) {
            uint32_t lo = 0;
            for (int j = 0; j < 4; j++) {
                const int e = 32 * kk + 8 * p + j;
                const uint32_t qa = live ? (uint32_t)q6_value(blk, e) ^ 32u : 0u;  // 6-bit two's complement of q - 32
                const uint32_t qb = live ? (uint32_t)q6_value(blk, e + 4) ^ 32u : 0u;
                lo |= ((qa & 15) | ((qb & 15) << 4)) << (8 * j);
                const int sh = 8 * j + 4 * (kk & 1);
                his[kk >> 1] |= ((qa >> 4) << sh) | ((qb >> 4) << (sh + 2));
            }
            ((uint32_t *)(T + GV6_LO))[(((kk >> 2) * 4 + p) * GV_ROWS + r) * 4 + (kk & 3)] = lo;
        }
        for (int hp = 0; hp < 4; hp++) ((uint32_t *)(T + GV6_HI))[(p * GV_ROWS + r) * 4 + hp] = his[hp];
    }
    const int8_t *scl = (const int8_t *)(blk + 192);
    for (int grp = 0; grp < 16; grp++) {
        const int8_t sc = live ? scl[grp] : (int8_t)0;
        const int kk = grp >> 1, g = grp & 1;
        ((int8_t *)(T + GV6_SC))[((g * 4 + r / 4) * 8 + kk) * 4 + (r & 3)] = sc;
    }
    ((uint16_t *)(T + GV6_D))[r] = live ? (uint16_t)(blk[208] | (blk[209] << 8)) : (uint16_t)0;
}

// Q6_K: limbs of sc * (q6 - 32) (lo = v & 127, hi = v >> 7 arithmetic), per-superblock d.
__global__ __launch_bounds__(256) void k_prepare_q6_K_tiled(const uint8_t *__restrict__ gguf, int8_t *__restrict__ tlo,
                                                            int8_t *__restrict__ thi, float *__restrict__ tdw,
                                                            int64_t n, int64_t row0, int64_t row_end, int64_t k,
                                                            int64_t n_pad) {
    const int64_t nbr = k / QK_K;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    __shared__ __attribute__((aligned(16))) uint8_t sblk[256 * sizeof(block_q6_K)];
    const int64_t gb0 = row0 * nbr + (int64_t)blockIdx.x * blockDim.x;
    stage_blocks<sizeof(block_q6_K)>(gguf, gb0, min(gb0 + (int64_t)blockDim.x, min(row_end, n) * nbr), sblk);
    if (gid >= (row_end - row0) * nbr) return;
    const int64_t row = row0 + gid / nbr, b = gid % nbr;
    const bool valid = row < n;
    const uint8_t *src = sblk + threadIdx.x * sizeof(block_q6_K);
    tdw[b * n_pad + row] = valid ? f16_bits_to_f32(*(const uint16_t *)(src + 208)) : 0.f;
    for (int t = 0; t < 16; t++) {  // 16 chunks of 16 values
        const int h = t >> 3, g = (t & 7) >> 1, l0 = (t & 1) * 16;
        const int sc = valid ? (int)(int8_t)src[192 + 8 * h + (l0 >> 4) + 2 * g] : 0;
        int lo[16], hi[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            int v = 0;
            if (valid) {
                const int l = l0 + i;
                const uint8_t qlb = src[64 * h + l + (g & 1) * 32];
                const int nib = (g < 2) ? (qlb & 0xF) : (qlb >> 4);
                const int hb = (src[128 + 32 * h + l] >> (2 * g)) & 3;
                v = sc * ((nib | (hb << 4)) - 32);  // in [-4064, 4096]
            }
            lo[i] = v & 127;
            hi[i] = v >> 7;
        }
        const int64_t off = tiled_off(row, b * QK_K + 16 * t, k);
        *(uint4 *)(tlo + off) = pack16(lo);
        *(uint4 *)(thi + off) = pack16(hi);
    }
}

// F16: copy the GGUF rows into the tiled plane, 16 bytes per thread.
__global__ __launch_bounds__(256) void k_prepare_f16_tiled(const uint8_t *__restrict__ gguf, uint8_t *__restrict__ tq,
                                                           int64_t n, int64_t row0, int64_t row_end, int64_t k,
                                                           int64_t kb_pad) {
    const int64_t np = kb_pad / 16;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (row_end - row0) * np) return;
    const int64_t row = row0 + gid / np, c = gid % np;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (row < n && 16 * c < 2 * k) v = *(const uint4 *)(gguf + row * 2 * k + 16 * c);
    *(uint4 *)(tq + tiled_off(row, 16 * c, kb_pad)) = v;
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
static inline bool aligned16(const void *p, int64_t ld_floats) {
    return (((uintptr_t)p) % 16 == 0) && ((ld_floats * 4) % 16 == 0);
}

static inline unsigned grid_for(int64_t threads) { return (unsigned)((threads + 255) / 256); }

template <int OUT>
static hipError_t q8_0_dispatch(const float *x, int64_t ldx, int8_t *out, float *xd, int64_t m, int64_t k, int variant,
                                int64_t m_pad, int64_t kb_pad, hipStream_t s, int pre = MQ_PRE_NONE,
                                const float *bias = nullptr, int64_t uoff = 0) {
    const int64_t rows = m;
    const int64_t nbx = k / QK8_0;
    const int64_t threads = rows * nbx * 8;
    if (threads == 0) return hipSuccess;
    const bool v4 = aligned16(x, ldx) && uoff % 4 == 0;
    const dim3 g(grid_for(threads)), b(256);
#define MQ_Q80(VAR)                                                                                             \
    if (v4) hipLaunchKernelGGL((k_quantize_q8_0<VAR, OUT, true>), g, b, 0, s, x, ldx, out, xd, m, k, m_pad, kb_pad, pre, bias, uoff); \
    else hipLaunchKernelGGL((k_quantize_q8_0<VAR, OUT, false>), g, b, 0, s, x, ldx, out, xd, m, k, m_pad, kb_pad, pre, bias, uoff);
    switch (variant) {
        case MQ_Q8_0_X86: MQ_Q80(MQ_Q8_0_X86); break;
        case MQ_Q8_0_NEON: MQ_Q80(MQ_Q8_0_NEON); break;
        case MQ_Q8_0_REF: MQ_Q80(MQ_Q8_0_REF); break;
        default: return hipErrorInvalidValue;
    }
#undef MQ_Q80
    return hipGetLastError();
}

template <int OUT>
static hipError_t q8_K_dispatch(const float *x, int64_t ldx, int8_t *out, float *xd, int16_t *xbs, _Float16 *xmin,
                                int64_t m, int64_t k, int64_t m_pad, hipStream_t s, int pre = MQ_PRE_NONE,
                                const float *bias = nullptr, int64_t uoff = 0) {
    const int64_t rows = m;
    const int64_t threads = rows * (k / QK_K) * 64;
    if (threads == 0) return hipSuccess;
    const dim3 g(grid_for(threads)), b(256);
    if (aligned16(x, ldx) && uoff % 4 == 0)
        hipLaunchKernelGGL((k_quantize_q8_K<OUT, true>), g, b, 0, s, x, ldx, out, xd, xbs, xmin, m, k, m_pad, pre, bias, uoff);
    else
        hipLaunchKernelGGL((k_quantize_q8_K<OUT, false>), g, b, 0, s, x, ldx, out, xd, xbs, xmin, m, k, m_pad, pre, bias, uoff);
    return hipGetLastError();
}

template <int FMT>
static hipError_t tiled_dispatch(const float *x, int64_t ldx, int8_t *xq, float *xd, _Float16 *xmin, int64_t m,
                                 int64_t k, int variant, int64_t m_pad, int64_t kb_pad, hipStream_t s, int pre,
                                 const float *bias, int64_t uoff) {
    constexpr int CB = (FMT == TQ_Q8_K) ? 256 : 128;
    if (m_pad % 32 != 0 || kb_pad % CB != 0) return hipErrorInvalidValue;
    const int64_t wgs = (m_pad / 32) * (kb_pad / CB);
    if (wgs == 0) return hipSuccess;
    // Rows per wave: Q8_K 2 (four workgroups per tile; measured on MI355X inside the Q4_K FFN
    // step: 8192 x 1024 18.8 -> 14.0 us, 8192 x 4096 43.7 -> 37.3 us against 8); Q8_0 8, or 2
    // under 512 tiles; F16 8 (its lanes cover 4 rows per pass).  MQ_TQ_RPW=8/2/1 (Q8_K) forces one
    // (measurements).
    int rpw = FMT == TQ_Q8_K ? 2 : (FMT == TQ_Q8_0 && wgs < 512 ? 2 : 8);
    if (const char *e = getenv("MQ_TQ_RPW"))
        if (*e && FMT == TQ_Q8_K) rpw = atoi(e) == 8 ? 8 : atoi(e) == 1 ? 1 : 2;
    const dim3 g((unsigned)(wgs * (32 / (4 * rpw)))), b(256);
    const bool v4 = aligned16(x, ldx) && uoff % 4 == 0;
#define MQ_TQ_R(VAR, RPW)                                                                                                    \
    if (v4) hipLaunchKernelGGL((k_quantize_tiled<FMT, VAR, true, RPW>), g, b, 0, s, x, ldx, xq, xd, xmin, m, k, m_pad, kb_pad, pre, bias, uoff); \
    else hipLaunchKernelGGL((k_quantize_tiled<FMT, VAR, false, RPW>), g, b, 0, s, x, ldx, xq, xd, xmin, m, k, m_pad, kb_pad, pre, bias, uoff);
#define MQ_TQ(VAR)                                   \
    if (rpw == 8) {                                  \
        MQ_TQ_R(VAR, 8)                              \
    } else if (FMT != TQ_F16 && rpw == 2) {          \
        MQ_TQ_R(VAR, (FMT == TQ_F16 ? 8 : 2))        \
    } else if (FMT == TQ_Q8_K) {                     \
        MQ_TQ_R(VAR, (FMT == TQ_Q8_K ? 1 : 8))       \
    }
    if (FMT != TQ_Q8_0) {
        MQ_TQ(MQ_Q8_0_X86);
    } else {
        switch (variant) {
            case MQ_Q8_0_X86: MQ_TQ(MQ_Q8_0_X86); break;
            case MQ_Q8_0_NEON: MQ_TQ(MQ_Q8_0_NEON); break;
            case MQ_Q8_0_REF: MQ_TQ(MQ_Q8_0_REF); break;
            default: return hipErrorInvalidValue;
        }
    }
#undef MQ_TQ
#undef MQ_TQ_R
    return hipGetLastError();
}

hipError_t launch_quantize_f16(const float *x, int64_t ldx, void *y, int64_t m, int64_t k, hipStream_t s, int pre,
                               const float *bias, int64_t uoff) {
    const int64_t threads = m * (k / 4);
    if (threads == 0) return hipSuccess;
    const dim3 g(grid_for(threads)), b(256);
    if (aligned16(x, ldx) && uoff % 4 == 0)
        hipLaunchKernelGGL((k_quantize_f16<true>), g, b, 0, s, x, ldx, (uint16_t *)y, m, k, pre, bias, uoff);
    else
        hipLaunchKernelGGL((k_quantize_f16<false>), g, b, 0, s, x, ldx, (uint16_t *)y, m, k, pre, bias, uoff);
    return hipGetLastError();
}

hipError_t launch_quantize_act_planar(int wtype, const float *x, int64_t ldx, void *ws, int64_t m, int64_t k,
                                      int q8_0_variant, bool tiled, hipStream_t s, int pre, const float *bias,
                                      const float *x2) {
    if (!tiled && m > GEMV_CHUNK) {  // the GEMV's chunked layout
        const size_t cb = gemv_chunk_bytes(wtype, k);
        for (int64_t r0 = 0, c = 0; r0 < m; r0 += GEMV_CHUNK, c++) {
            const hipError_t e = launch_quantize_act_planar(wtype, x + r0 * ldx, ldx, (uint8_t *)ws + c * cb,
                                                            std::min<int64_t>(GEMV_CHUNK, m - r0), k, q8_0_variant,
                                                            false, s, pre, bias, x2 ? x2 + r0 * ldx : nullptr);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    // MQ_PRE_SILU_MUL: the up projection's values uoff floats after the gate projection's (the
    // same row stride): in the same row (k) or in x2
    const int64_t uoff = x2 ? (int64_t)(x2 - x) : k;
    const ActPlanes a = act_planes(wtype, m, k, tiled);
    uint8_t *base = (uint8_t *)ws;
    int8_t *xq = (int8_t *)(base + a.xq);
    float *xd = (float *)(base + a.xd);
    switch (wtype) {
        case MQ_TYPE_Q8_0:
            if (tiled)
                return tiled_dispatch<TQ_Q8_0>(x, ldx, xq, xd, nullptr, m, k, q8_0_variant, a.m_pad, a.kb_pad, s, pre,
                                               bias, uoff);
            return q8_0_dispatch<OUT_ROWS>(x, ldx, xq, xd, m, k, q8_0_variant, m, k, s, pre, bias, uoff);
        case MQ_TYPE_Q4_K:
        case MQ_TYPE_Q6_K:
            if (tiled)
                return tiled_dispatch<TQ_Q8_K>(x, ldx, xq, xd, (_Float16 *)(base + a.xmin), m, k, 0, a.m_pad, a.kb_pad, s,
                                               pre, bias, uoff);
            return q8_K_dispatch<OUT_ROWS>(x, ldx, xq, xd, (int16_t *)(base + a.xbs), (_Float16 *)(base + a.xgm), m, k,
                                           m, s, pre, bias, uoff);
        case MQ_TYPE_F16:
            if (tiled)
                return tiled_dispatch<TQ_F16>(x, ldx, xq, nullptr, nullptr, m, k, 0, a.m_pad, a.kb_pad, s, pre, bias,
                                              uoff);
            return launch_quantize_f16(x, ldx, base + a.xq, m, k, s, pre, bias, uoff);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_quantize_q8_0_gguf(const float *x, int64_t ldx, void *y, int64_t m, int64_t k, int variant,
                                     hipStream_t s) {
    return q8_0_dispatch<OUT_GGUF>(x, ldx, (int8_t *)y, nullptr, m, k, variant, m, k, s);
}

hipError_t launch_quantize_q8_K_gguf(const float *x, int64_t ldx, void *y, int64_t m, int64_t k, hipStream_t s) {
    return q8_K_dispatch<OUT_GGUF>(x, ldx, (int8_t *)y, nullptr, nullptr, nullptr, m, k, m, s);
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

// Q4_K GEMV plane (layout in mq_internal.h): one thread per (row, superblock).
__global__ __launch_bounds__(256) void k_prepare_q4_K_gv(const uint8_t *__restrict__ gguf, uint8_t *__restrict__ gv,
                                                         int64_t n, int64_t row0, int64_t row1, int64_t k) {
    const int64_t nsb = k / QK_K;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t row = row0 + t / nsb, sb = t % nsb;
    if (row >= row1) return;
    const int r = (int)(row % GV_ROWS);
    uint8_t *T = gv + ((row / GV_ROWS) * nsb + sb) * GV4_BYTES;
    const bool live = row < n;
    const uint8_t *blk = gguf + (row * nsb + sb) * sizeof(block_q4_K);
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            int4 v = make_int4(0, 0, 0, 0);
            if (live) {
                const uint8_t *src = blk + 16 + 32 * c + 16 * h;  // qs bytes 32c+16h..+16 (16-byte aligned)
                v = *(const int4 *)src;
            }
            *(int4 *)(T + GV4_QS + ((c * 2 + h) * GV_ROWS + r) * 16) = v;
        }
#pragma unroll
    for (int j = 0; j < 8; j++) {
        int sc = 0, mn = 0;
        if (live) scale_min_k4(j, blk + 4, sc, mn);
        T[GV4_SC + (((j & 1) * 4 + r / 4) * 4 + (j >> 1)) * 4 + (r & 3)] = (uint8_t)sc;
        T[GV4_MN + ((j >> 2) * GV_ROWS + r) * 4 + (j & 3)] = (uint8_t)mn;
    }
    ((uint32_t *)(T + GV4_DD))[r] = live ? *(const uint32_t *)blk : 0u;  // d, dmin halves
}

hipError_t launch_weight_prepare(int type, void *image, int64_t n, int64_t k, int64_t row0, int64_t row1,
                                 hipStream_t s) {
    const WeightPlanes p = weight_planes(type, n, k);
    uint8_t *base = (uint8_t *)image;
    if (row1 <= row0) return hipSuccess;
    const int64_t row_end = (row1 >= n) ? p.n_pad : row1;  // tiled planes: zero the padding rows too
    const int64_t nbr = k / (type == MQ_TYPE_Q8_0 ? QK8_0 : QK_K);
    const dim3 b(256);
    switch (type) {
        case MQ_TYPE_F16:
            hipLaunchKernelGGL(k_prepare_f16_tiled, dim3(grid_for((row_end - row0) * (p.kb_pad / 16))), b, 0, s, base,
                               base + p.tq, n, row0, row_end, k, p.kb_pad);
            break;
        case MQ_TYPE_Q8_0:
            hipLaunchKernelGGL(k_prepare_q8_0_rows, dim3(grid_for((row1 - row0) * nbr)), b, 0, s, base,
                               (int8_t *)(base + p.qs), (uint16_t *)(base + p.d16), row0, row1, k);
            hipLaunchKernelGGL(k_prepare_q8_0_tiled, dim3(grid_for((row_end - row0) * (p.kb_pad / QK8_0))), b, 0, s,
                               base, (int8_t *)(base + p.tq), (float *)(base + p.tdw), n, row0, row_end, k, p.n_pad,
                               p.kb_pad);
            break;
        case MQ_TYPE_Q4_K: {
            const int64_t gv_end = (row1 >= n) ? pad_up(n, GV_ROWS) : row1;  // zero the last tile's padding rows
            hipLaunchKernelGGL(k_prepare_q4_K_gv, dim3(grid_for((gv_end - row0) * nbr)), b, 0, s, base, base + p.gv, n,
                               row0, gv_end, k);
        }
            hipLaunchKernelGGL(k_prepare_q4_K_tiled, dim3(grid_for((row_end - row0) * nbr)), b, 0, s, base,
                               (int8_t *)(base + p.tq), (int8_t *)(base + p.thi), (float *)(base + p.tdw),
                               (float *)(base + p.tdmin), (_Float16 *)(base + p.tmin), n, row0, row_end, k, p.n_pad);
            break;
        case MQ_TYPE_Q6_K:
        {
            const int64_t gv_end = (row1 >= n) ? pad_up(n, GV_ROWS) : row1;  // zero the last tile's padding rows
            hipLaunchKernelGGL(k_prepare_q6_K_gv, dim3(grid_for((gv_end - row0) * nbr)), b, 0, s, base, base + p.gv, n,
                               row0, gv_end, k);
        }
            hipLaunchKernelGGL(k_prepare_q6_K_tiled, dim3(grid_for((row_end - row0) * nbr)), b, 0, s, base,
                               (int8_t *)(base + p.tq), (int8_t *)(base + p.thi), (float *)(base + p.tdw), n, row0,
                               row_end, k, p.n_pad);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mq
