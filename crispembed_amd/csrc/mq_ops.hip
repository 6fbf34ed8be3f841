// mq_ops.hip -- the non-matmul ops of CrispEmbed's graphs (mq_ops.h) on strided ggml-style views.
//
// All of them are HBM-bound elementwise or row passes: one read of every input element and one
// write of every output element is the whole cost, so the kernels are built around coalesced
// 16-byte accesses (a float4 per lane when the views allow it), grid-stride loops sized to fill
// the 256 CUs, and one wave per row where a row reduction is needed (norm) or a row is gathered
// (get_rows).  Attention (mq_op_flash_attn) is the fragment-attention kernel pair of
// mq_decoder.hip driven through strided operands.
//
// ggml semantics followed (ggml-cpu ops.cpp of the ggml submodule; the reference calls them from
// src/crispembed.cpp:1043-1468): get_rows dst[:, i10, i11, i12] = src[:, ids[i10, i11, i12], i11,
// i12]; binary ops broadcast src1 by index modulo its extent; norm is two-pass mean / variance with
// scale 1/sqrtf(var + eps); rms_norm scale 1/sqrtf(mean(x^2) + eps); cpy walks both views in
// row-major logical order.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <initializer_list>
#include <vector>

#include "../../include/mq_ops.h"
#include "mq_act.h"
#include "mq_deq.h"
#include "mq_internal.h"
#include "mq_runner.h"
#include "mq_wave.h"

namespace mq {
namespace {

// device-side copy of a view (byte strides)
struct DV {
    char *p;
    int64_t ne[4];
    int64_t nb[4];
};

DV dv(const mq_view *v) {
    DV d;
    d.p = (char *)v->data;
    for (int i = 0; i < 4; i++) d.ne[i] = v->ne[i], d.nb[i] = (int64_t)v->nb[i];
    return d;
}

__device__ __forceinline__ int64_t off3(const DV &v, int64_t i1, int64_t i2, int64_t i3) {
    return i1 * v.nb[1] + i2 * v.nb[2] + i3 * v.nb[3];
}

// unit u of a view walked W elements at a time along ne0 -> (i0, i1, i2, i3)
template <int W>
__device__ __forceinline__ void unflat(int64_t u, const int64_t *ne, int64_t &i0, int64_t &i1, int64_t &i2,
                                       int64_t &i3) {
    const int64_t ne0u = ne[0] / W;
    int64_t r = u / ne0u;
    i0 = (u - r * ne0u) * W;
    i1 = r % ne[1];
    r /= ne[1];
    i2 = r % ne[2];
    i3 = r / ne[2];
}

template <int OP>
__device__ __forceinline__ float bin(float x, float y) {
    if constexpr (OP == MQ_BIN_ADD) return x + y;
    else if constexpr (OP == MQ_BIN_SUB) return x - y;
    else if constexpr (OP == MQ_BIN_MUL) return x * y;
    else return x / y;
}

template <int OP>
__device__ __forceinline__ float una(float x) {
    if constexpr (OP == MQ_UNARY_GELU_ERF) {
        return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f));
    } else if constexpr (OP == MQ_UNARY_GELU) {
        const float c = 0.79788456080286535588f;  // sqrt(2 / pi)
        return 0.5f * x * (1.0f + tanhf(c * x * (1.0f + 0.044715f * x * x)));
    } else if constexpr (OP == MQ_UNARY_SILU) {
        return x / (1.0f + expf(-x));
    } else {
        return x > 0.0f ? x : 0.0f;
    }
}

// dst = a (op) b; W = 4: every view is walked in float4s (b not broadcast along ne0)
template <int OP, int W>
__global__ __launch_bounds__(256) void k_binary(const DV a, const DV b, const DV d, int64_t units) {
    for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < units; u += (int64_t)gridDim.x * 256) {
        int64_t i0, i1, i2, i3;
        unflat<W>(u, a.ne, i0, i1, i2, i3);
        const char *pa = a.p + i0 * 4 + off3(a, i1, i2, i3);
        const char *pb = b.p + off3(b, i1 % b.ne[1], i2 % b.ne[2], i3 % b.ne[3]);
        char *pd = d.p + i0 * 4 + off3(d, i1, i2, i3);
        if constexpr (W == 4) {
            const float4 x = *(const float4 *)pa, y = *(const float4 *)(pb + i0 * 4);
            *(float4 *)pd = make_float4(bin<OP>(x.x, y.x), bin<OP>(x.y, y.y), bin<OP>(x.z, y.z), bin<OP>(x.w, y.w));
        } else {
            const float x = *(const float *)(a.p + i0 * a.nb[0] + off3(a, i1, i2, i3));
            const float y = *(const float *)(pb + (i0 % b.ne[0]) * b.nb[0]);
            *(float *)(d.p + i0 * d.nb[0] + off3(d, i1, i2, i3)) = bin<OP>(x, y);
        }
    }
}

template <int OP, int W>
__global__ __launch_bounds__(256) void k_unary(const DV x, const DV d, int64_t units) {
    for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < units; u += (int64_t)gridDim.x * 256) {
        int64_t i0, i1, i2, i3;
        unflat<W>(u, x.ne, i0, i1, i2, i3);
        if constexpr (W == 4) {
            const float4 v = *(const float4 *)(x.p + i0 * 4 + off3(x, i1, i2, i3));
            *(float4 *)(d.p + i0 * 4 + off3(d, i1, i2, i3)) =
                make_float4(una<OP>(v.x), una<OP>(v.y), una<OP>(v.z), una<OP>(v.w));
        } else {
            const float v = *(const float *)(x.p + i0 * x.nb[0] + off3(x, i1, i2, i3));
            *(float *)(d.p + i0 * d.nb[0] + off3(d, i1, i2, i3)) = una<OP>(v);
        }
    }
}

// One wave per row; V values per lane held in registers (row length <= 64 V), or V = 0: the
// row is read again from memory (L2) for each pass.
template <int KIND, int V>
__global__ __launch_bounds__(256) void k_norm(const DV x, const DV r, const DV d, float eps, const float *__restrict__ w,
                                              const float *__restrict__ bias, int64_t nrows) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + wave;
    if (row >= nrows) return;
    const int n = (int)x.ne[0];
    const int64_t i1 = row % x.ne[1], i2 = (row / x.ne[1]) % x.ne[2], i3 = row / (x.ne[1] * x.ne[2]);
    const float *xr = (const float *)(x.p + off3(x, i1, i2, i3));
    const float *rr = r.p ? (const float *)(r.p + off3(r, i1, i2, i3)) : nullptr;
    float *dr = (float *)(d.p + off3(d, i1, i2, i3));
    const float inv_n = 1.0f / (float)n;
    float mean = 0.f, scale;
    if constexpr (V > 0) {
        float v[V], s = 0.f;
#pragma unroll
        for (int i = 0; i < V; i++) {
            const int c = lane + 64 * i;
            v[i] = c < n ? (rr ? xr[c] + rr[c] : xr[c]) : 0.f;
            s += KIND == MQ_NORM_LAYER ? v[i] : v[i] * v[i];
        }
        if constexpr (KIND == MQ_NORM_LAYER) {
            mean = wave_sum_f(s) * inv_n;
            float s2 = 0.f;
#pragma unroll
            for (int i = 0; i < V; i++) {
                const float t = lane + 64 * i < n ? v[i] - mean : 0.f;
                s2 += t * t;
            }
            scale = 1.0f / sqrtf(wave_sum_f(s2) * inv_n + eps);
        } else {
            scale = 1.0f / sqrtf(wave_sum_f(s) * inv_n + eps);
        }
#pragma unroll
        for (int i = 0; i < V; i++) {
            const int c = lane + 64 * i;
            if (c < n) {
                float y = (v[i] - mean) * scale;
                if (w) y = y * w[c];
                if (bias) y = y + bias[c];
                dr[c] = y;
            }
        }
    } else {
        if (rr) {  // long rows: the sum is formed once, in dst, and normalised in place
            for (int c = lane; c < n; c += 64) dr[c] = xr[c] + rr[c];
            xr = dr;
        }
        float s = 0.f;
        for (int c = lane; c < n; c += 64) s += KIND == MQ_NORM_LAYER ? xr[c] : xr[c] * xr[c];
        if constexpr (KIND == MQ_NORM_LAYER) {
            mean = wave_sum_f(s) * inv_n;
            float s2 = 0.f;
            for (int c = lane; c < n; c += 64) s2 += (xr[c] - mean) * (xr[c] - mean);
            scale = 1.0f / sqrtf(wave_sum_f(s2) * inv_n + eps);
        } else {
            scale = 1.0f / sqrtf(wave_sum_f(s) * inv_n + eps);
        }
        for (int c = lane; c < n; c += 64) {
            float y = (xr[c] - mean) * scale;
            if (w) y = y * w[c];
            if (bias) y = y + bias[c];
            dr[c] = y;
        }
    }
}

// k_norm on dense rows of K = 128 NV floats whose result also leaves as the Q8_0 activation
// of the mat-mul that reads it, in the GEMM layout the tiled activation quantizer writes
// (1 KB fragments per 32-row tile and 32-value chunk: lane l's 16 bytes are row l % 32,
// bytes 16 (l / 32) ..; scales [K / 32][m_pad], pad rows of the tile quantized as zeros).
// Workgroup: RT rows (8: a quarter of a 32-row tile, so a 4096-row input gives every CU two
// workgroups), NW waves; half a wave takes a row, lane s holding values 4 s + 128 p (p < NV) as
// float4, so a Q8_0 block is 8 lanes (a 3-step xor max) and the row sums are 5-step half-wave
// xor sums.  Quants go through LDS and leave as the 16-byte lane units of this workgroup's
// rows in each fragment (lanes r and r + 32 for its rows r): 256-byte contiguous runs.
// Same arithmetic as k_norm (sum, mean, centred sum of squares, 1 / sqrt(var + eps), then
// * w, + b), with the sums taken in this lane order; quantization as quantize_row_q8_0.
template <int KIND, int NV, int NW, int RT>
__global__ __launch_bounds__(64 * NW) void k_norm_q8_0(const float *x, const float *r, float *d, float eps,  // d may be x
                                                       const float *__restrict__ w,
                                                       const float *__restrict__ bias, int64_t nrows,
                                                       int8_t *__restrict__ xq, float *__restrict__ xd, int64_t m_pad,
                                                       int variant) {
    constexpr int K = 128 * NV, NCH = K / 32, FST = 1024 + 16;
    constexpr int RPW = RT / NW, NIT = RPW / 2;  // rows per wave, passes of two rows
    static_assert((RT == 2 || RT == 8 || RT == 16 || RT == 32) && NIT >= 1 && RPW % 2 == 0, "2, 8, 16 or 32 rows, whole passes");
    __shared__ __attribute__((aligned(16))) int8_t frag[NCH * FST];
    __shared__ float dsh[NCH][32];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane & 31, half = lane >> 5;
    const int64_t rt = blockIdx.x / (32 / RT);             // 32-row tile
    const int r0 = (int)(blockIdx.x % (32 / RT)) * RT;     // first row of this workgroup in it
    const float inv_n = 1.0f / (float)K;
    float4 v[NIT][NV];
#pragma unroll
    for (int it = 0; it < NIT; it++) {
        const int64_t row = rt * 32 + r0 + wave * RPW + it * 2 + half;
#pragma unroll
        for (int p = 0; p < NV; p++) {
            v[it][p] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (row < nrows) {
                const int64_t o = row * K + 128 * p + 4 * sub;
                float4 a = *(const float4 *)(x + o);
                if (r) {
                    const float4 c = *(const float4 *)(r + o);
                    a.x = a.x + c.x, a.y = a.y + c.y, a.z = a.z + c.z, a.w = a.w + c.w;
                }
                v[it][p] = a;
            }
        }
    }
    float4 wv[NV], bv[NV];
#pragma unroll
    for (int p = 0; p < NV; p++) {
        wv[p] = w ? *(const float4 *)(w + 128 * p + 4 * sub) : make_float4(1.f, 1.f, 1.f, 1.f);
        bv[p] = bias ? *(const float4 *)(bias + 128 * p + 4 * sub) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    auto hsum = [](float t) {
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) t += __shfl_xor(t, o);
        return t;
    };
#pragma unroll
    for (int it = 0; it < NIT; it++) {
        const int rr = r0 + wave * RPW + it * 2 + half;  // row within the tile
        const int64_t row = rt * 32 + rr;
        float mean = 0.f, s = 0.f;
#pragma unroll
        for (int p = 0; p < NV; p++) {
            const float4 a = v[it][p];
            if (KIND == MQ_NORM_LAYER) s += a.x + a.y + a.z + a.w;
            else s += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
        }
        float scale;
        if (KIND == MQ_NORM_LAYER) {
            mean = hsum(s) * inv_n;
            float s2 = 0.f;
#pragma unroll
            for (int p = 0; p < NV; p++) {
                const float4 a = v[it][p];
                const float t0 = a.x - mean, t1 = a.y - mean, t2 = a.z - mean, t3 = a.w - mean;
                s2 += t0 * t0 + t1 * t1 + t2 * t2 + t3 * t3;
            }
            scale = 1.0f / sqrtf(hsum(s2) * inv_n + eps);
        } else {
            scale = 1.0f / sqrtf(hsum(s) * inv_n + eps);
        }
#pragma unroll
        for (int p = 0; p < NV; p++) {
            const float4 a = v[it][p];
            float y[4] = {a.x, a.y, a.z, a.w};
            const float ww[4] = {wv[p].x, wv[p].y, wv[p].z, wv[p].w}, bb[4] = {bv[p].x, bv[p].y, bv[p].z, bv[p].w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float t = (y[e] - mean) * scale;
                if (w) t = t * ww[e];
                if (bias) t = t + bb[e];
                y[e] = row < nrows ? t : 0.f;  // pad rows of the tile quantize to zero
            }
            if (row < nrows) *(float4 *)(d + row * K + 128 * p + 4 * sub) = make_float4(y[0], y[1], y[2], y[3]);
            float amax = fmaxf(fmaxf(fabsf(y[0]), fabsf(y[1])), fmaxf(fabsf(y[2]), fabsf(y[3])));
            amax = fmaxf(amax, __shfl_xor(amax, 1));
            amax = fmaxf(amax, __shfl_xor(amax, 2));
            amax = fmaxf(amax, __shfl_xor(amax, 4));
            const float dq = amax / 127.f;
            float id;
            if (variant == MQ_Q8_0_X86) id = (amax != 0.0f) ? 127.f / amax : 0.0f;
            else id = (dq != 0.0f) ? 1.0f / dq : 0.0f;
            uint32_t pk = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float t = y[e] * id;
                float q = (variant == MQ_Q8_0_REF) ? roundf(t) : rintf(t);
                q = fminf(fmaxf(q, -128.f), 127.f);
                pk |= ((uint32_t)((int)q & 0xff)) << (8 * e);
            }
            const int c = 4 * p + (sub >> 3), cbyte = 4 * (sub & 7);  // chunk, byte within it
            *(uint32_t *)(frag + c * FST + ((rr + 32 * (cbyte >> 4)) << 4) + (cbyte & 15)) = pk;
            if ((sub & 7) == 0) dsh[c][rr] = f16_bits_to_f32(f32_to_f16_bits(dq));
        }
    }
    __syncthreads();
    const int t = threadIdx.x;
    constexpr int UPF = 2 * RT;  // 16-byte lane units of this workgroup's rows per fragment
    for (int q = t; q < NCH * UPF; q += 64 * NW) {
        const int f = q / UPF, u = q % UPF;
        const int L = r0 + (u % RT) + 32 * (u / RT);  // lane of row r0 + u % RT, half u / RT
        *(int4 *)(xq + ((rt * NCH + f) << 10) + L * 16) = *(const int4 *)(frag + f * FST + L * 16);
    }
    for (int q = t; q < NCH * RT; q += 64 * NW)
        xd[(int64_t)(q / RT) * m_pad + rt * 32 + r0 + (q % RT)] = dsh[q / RT][r0 + (q % RT)];
}

template <typename S>
__device__ __forceinline__ float ld_as_f32(const char *p) {
    if constexpr (sizeof(S) == 4) return *(const float *)p;
    else return (float)*(const _Float16 *)p;
}
template <typename D>
__device__ __forceinline__ void st_from_f32(char *p, float v) {
    if constexpr (sizeof(D) == 4) *(float *)p = v;
    else *(_Float16 *)p = (_Float16)v;  // round to nearest even
}

// same shape both sides; W = 4: float4 rows (F32 -> F32 only)
template <typename S, typename D, int W>
__global__ __launch_bounds__(256) void k_cpy_same(const DV s, const DV d, int64_t units) {
    for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < units; u += (int64_t)gridDim.x * 256) {
        int64_t i0, i1, i2, i3;
        unflat<W>(u, s.ne, i0, i1, i2, i3);
        if constexpr (W == 4) {
            *(float4 *)(d.p + i0 * 4 + off3(d, i1, i2, i3)) = *(const float4 *)(s.p + i0 * 4 + off3(s, i1, i2, i3));
        } else {
            st_from_f32<D>(d.p + i0 * d.nb[0] + off3(d, i1, i2, i3),
                           ld_as_f32<S>(s.p + i0 * s.nb[0] + off3(s, i1, i2, i3)));
        }
    }
}

// element u of src in its row-major order goes to element u of dst in its own
template <typename S, typename D>
__global__ __launch_bounds__(256) void k_cpy_any(const DV s, const DV d, int64_t n) {
    for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < n; u += (int64_t)gridDim.x * 256) {
        int64_t a0, a1, a2, a3, b0, b1, b2, b3;
        unflat<1>(u, s.ne, a0, a1, a2, a3);
        unflat<1>(u, d.ne, b0, b1, b2, b3);
        st_from_f32<D>(d.p + b0 * d.nb[0] + off3(d, b1, b2, b3), ld_as_f32<S>(s.p + a0 * s.nb[0] + off3(s, a1, a2, a3)));
    }
}

// One wave per gathered row.  A row id outside the table yields a zero row.
template <int TYPE>
__global__ __launch_bounds__(256) void k_get_rows(const DV src, const DV ids, const DV d, int64_t nrows) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + wave;
    if (row >= nrows) return;
    const int64_t i10 = row % ids.ne[0], i11 = (row / ids.ne[0]) % ids.ne[1], i12 = row / (ids.ne[0] * ids.ne[1]);
    const int32_t id = *(const int32_t *)(ids.p + i10 * ids.nb[0] + i11 * ids.nb[1] + i12 * ids.nb[2]);
    const bool ok = id >= 0 && id < src.ne[1];
    const uint8_t *sr = (const uint8_t *)src.p + (ok ? (int64_t)id * src.nb[1] : 0) + i11 * src.nb[2] + i12 * src.nb[3];
    float *dr = (float *)(d.p + off3(d, i10, i11, i12));
    const int64_t n = src.ne[0];
    if constexpr (TYPE == MQ_TYPE_F32) {
        if (ok && n % 4 == 0 && ((uintptr_t)sr & 15) == 0 && ((uintptr_t)dr & 15) == 0) {
            for (int64_t c = 4 * lane; c < n; c += 256) *(float4 *)(dr + c) = *(const float4 *)(sr + 4 * c);
            return;
        }
    }
    for (int64_t c = lane; c < n; c += 64) dr[c] = ok ? deq_elem<TYPE>(sr, c) : 0.f;
}

// Sum of 2 or 3 gathered F32 table rows (the embedding ADDs of GET_ROWS results), one wave per
// output row, added in table order as the ADD nodes add them; an id outside its table adds a
// zero row, as k_get_rows gathers one.
struct RowsSumArgs {
    const float *tab[3];
    const int32_t *ids[3];
    int64_t ntab_rows[3], ld[3];
    int n;
};
template <bool V4>
__global__ __launch_bounds__(256) void k_get_rows_sum(const RowsSumArgs a, float *__restrict__ d, int64_t nrows,
                                                      int64_t ne0) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + wave;
    if (row >= nrows) return;
    const float *src[3];
#pragma unroll
    for (int t = 0; t < 3; t++) {
        src[t] = nullptr;
        if (t < a.n) {
            const int32_t id = a.ids[t][row];
            src[t] = (id >= 0 && id < a.ntab_rows[t]) ? a.tab[t] + (int64_t)id * a.ld[t] : nullptr;
        }
    }
    float *dr = d + row * ne0;
    if constexpr (V4) {
        for (int64_t c = 4 * lane; c < ne0; c += 256) {
            float4 acc = src[0] ? *(const float4 *)(src[0] + c) : make_float4(0.f, 0.f, 0.f, 0.f);
            for (int t = 1; t < a.n; t++) {
                const float4 v = src[t] ? *(const float4 *)(src[t] + c) : make_float4(0.f, 0.f, 0.f, 0.f);
                acc.x = acc.x + v.x, acc.y = acc.y + v.y, acc.z = acc.z + v.z, acc.w = acc.w + v.w;
            }
            *(float4 *)(dr + c) = acc;
        }
    } else {
        for (int64_t c = lane; c < ne0; c += 64) {
            float acc = src[0] ? src[0][c] : 0.f;
            for (int t = 1; t < a.n; t++) acc = acc + (src[t] ? src[t][c] : 0.f);
            dr[c] = acc;
        }
    }
}

// Rotary embedding: one thread per (row, pair slot j < ne0/2).  Slots j < n_dims/2 rotate
// their pair; the others copy elements 2j, 2j + 1 (all at or past n_dims).
struct RopeParams {
    int n_dims, mode;
    float theta_scale, freq_scale, ext_factor, attn_factor, corr_lo, corr_hi;
};

template <int MODE>
__global__ __launch_bounds__(256) void k_rope(const DV x, const DV pos, const float *__restrict__ ff, const DV d,
                                              const RopeParams rp, int64_t units) {
    const int64_t half0 = x.ne[0] / 2;
    for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < units; u += (int64_t)gridDim.x * 256) {
        int64_t r = u / half0;
        const int j = (int)(u - r * half0);
        const int64_t i1 = r % x.ne[1];
        r /= x.ne[1];
        const int64_t i2 = r % x.ne[2], i3 = r / x.ne[2];
        const float *xr = (const float *)(x.p + off3(x, i1, i2, i3));
        float *dr = (float *)(d.p + off3(d, i1, i2, i3));
        const int hn = rp.n_dims / 2;
        if (j >= hn) {
            const float a = xr[2 * j], b = xr[2 * j + 1];
            dr[2 * j] = a, dr[2 * j + 1] = b;
            continue;
        }
        // the rope cache's angle chain: theta = p, then one fp32 product per earlier pair
        float theta = (float)*(const int32_t *)(pos.p + i2 * pos.nb[0]);
        for (int k = 0; k < j; k++) theta *= rp.theta_scale;
        const float extrap = ff ? theta / ff[j] : theta;
        float th = rp.freq_scale * extrap, mscale = rp.attn_factor;
        if (rp.ext_factor != 0.0f) {
            const float y = ((float)j - rp.corr_lo) / fmaxf(0.001f, rp.corr_hi - rp.corr_lo);
            const float mix = (1.0f - fminf(1.0f, fmaxf(0.0f, y))) * rp.ext_factor;
            th = th * (1.0f - mix) + extrap * mix;
            mscale *= 1.0f + 0.1f * logf(1.0f / rp.freq_scale);
        }
        const float c = cosf(th) * mscale, sn = sinf(th) * mscale;
        const int e0 = MODE == MQ_ROPE_NEOX ? j : 2 * j, e1 = MODE == MQ_ROPE_NEOX ? j + hn : 2 * j + 1;
        const float a = xr[e0], b = xr[e1];
        dr[e0] = a * c - b * sn;
        dr[e1] = a * sn + b * c;
    }
}

// k_rope for rows with every dimension rotated (ne0 = n_dims <= 128): one workgroup per
// position (i2, i3).  Its n_dims / 2 angles -- the same fp32 chain, freq factors and YaRN mix
// as k_rope, so the same cos / sin -- are formed once into LDS instead of once per row, then a
// wave per row (ne1 rows: the heads), lane j < n_dims / 2 rotating pair j.  NORM: the row is
// first RMS-normed and multiplied by w (ggml_rms_norm, ggml_mul) as k_norm computes it for
// ne0 = 128 (lane j holds elements j and j + 64, the same sum order), so the result equals
// mq_op_norm followed by mq_op_rope bit for bit (NEOX, n_dims 128 only).
// (cos, sin) x mscale of rotation pair j at position p, as the rope cache computes them:
// theta = p * theta_scale^j (j rounded products), / freq_factor[j], YaRN's ramp mix.
__device__ __forceinline__ float2 rope_cs(const RopeParams &rp, int32_t p, int j, const float *__restrict__ ff) {
    float theta = (float)p;
    for (int k = 0; k < j; k++) theta *= rp.theta_scale;
    const float extrap = ff ? theta / ff[j] : theta;
    float th = rp.freq_scale * extrap, mscale = rp.attn_factor;
    if (rp.ext_factor != 0.0f) {
        const float y = ((float)j - rp.corr_lo) / fmaxf(0.001f, rp.corr_hi - rp.corr_lo);
        const float mix = (1.0f - fminf(1.0f, fmaxf(0.0f, y))) * rp.ext_factor;
        th = th * (1.0f - mix) + extrap * mix;
        mscale *= 1.0f + 0.1f * logf(1.0f / rp.freq_scale);
    }
    return make_float2(cosf(th) * mscale, sinf(th) * mscale);
}

// The table of rope_cs for positions pos[0 .. T-1]: cs[t * n_dims / 2 + j], one wave per position.
__global__ __launch_bounds__(64) void k_rope_cache(const DV pos, const float *__restrict__ ff, const RopeParams rp,
                                                   float2 *__restrict__ cs) {
    const int t = blockIdx.x, j = threadIdx.x, hn = rp.n_dims / 2;
    if (j < hn) cs[(int64_t)t * hn + j] = rope_cs(rp, *(const int32_t *)(pos.p + t * pos.nb[0]), j, ff);
}

template <int MODE, bool NORM>
__global__ __launch_bounds__(256) void k_rope_rows(const DV x, const DV pos, const float *__restrict__ ff, const DV d,
                                                   const RopeParams rp, const float *__restrict__ w, float eps) {
    __shared__ float cs[2][64];
    const int64_t i2 = blockIdx.x % x.ne[2], i3 = blockIdx.x / x.ne[2];
    const int hn = rp.n_dims / 2;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const bool on = lane < hn;
    const int e0 = MODE == MQ_ROPE_NEOX ? lane : 2 * lane, e1 = MODE == MQ_ROPE_NEOX ? lane + hn : 2 * lane + 1;
    // the wave's first RU rows are loaded before the angles are computed, so the two overlap
    constexpr int RU = 4;
    float a[RU], b[RU];
#pragma unroll
    for (int u = 0; u < RU; u++) {
        const int64_t i1 = wave + 4 * u;
        a[u] = 0.f, b[u] = 0.f;
        if (on && i1 < x.ne[1]) {
            const float *xr = (const float *)(x.p + off3(x, i1, i2, i3));
            a[u] = xr[e0], b[u] = xr[e1];
        }
    }
    if ((int)threadIdx.x < hn) {
        const float2 r = rope_cs(rp, *(const int32_t *)(pos.p + i2 * pos.nb[0]), threadIdx.x, ff);
        cs[0][threadIdx.x] = r.x;
        cs[1][threadIdx.x] = r.y;
    }
    // LDS only: the row loads above stay in flight across the barrier
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const float c = on ? cs[0][lane] : 0.f, sn = on ? cs[1][lane] : 0.f;
    auto row = [&](int64_t i1, float a, float b) {
        float *dr = (float *)(d.p + off3(d, i1, i2, i3));
        if constexpr (NORM) {
            float s = 0.f;
            s += a * a;
            s += b * b;
            const float inv_n = 1.0f / (float)rp.n_dims;
            const float scale = 1.0f / sqrtf(wave_sum_f(s) * inv_n + eps);
            a = (a - 0.0f) * scale * w[e0];
            b = (b - 0.0f) * scale * w[e1];
        }
        if (on) {
            dr[e0] = a * c - b * sn;
            dr[e1] = a * sn + b * c;
        }
    };
#pragma unroll
    for (int u = 0; u < RU; u++)
        if (wave + 4 * u < x.ne[1]) row(wave + 4 * u, a[u], b[u]);
    for (int64_t i1 = wave + 4 * RU; i1 < x.ne[1]; i1 += 4) {
        const float *xr = (const float *)(x.p + off3(x, i1, i2, i3));
        row(i1, on ? xr[e0] : 0.f, on ? xr[e1] : 0.f);
    }
}

// Row moves of the mixture-of-experts mat-mul: one workgroup per row r, float4 copies
// (rows of k floats, k a multiple of 32 for every weight type), byte offsets per row.
__global__ __launch_bounds__(256) void k_gather_rows(const char *__restrict__ src, const int64_t *__restrict__ off,
                                                     float *__restrict__ dst, int64_t k) {
    const int64_t r = blockIdx.x;
    const float4 *s = (const float4 *)(src + off[r]);
    float4 *d = (float4 *)(dst + r * k);
    for (int64_t c = threadIdx.x; c < k / 4; c += 256) d[c] = s[c];
}

__global__ __launch_bounds__(256) void k_scatter_rows(const float *__restrict__ src, const int64_t *__restrict__ off,
                                                      char *__restrict__ dst, int64_t n) {
    const int64_t r = blockIdx.x;
    const float *s = src + r * n;
    float *d = (float *)(dst + off[r]);
    for (int64_t c = threadIdx.x; c < n; c += 256) d[c] = s[c];
}

// Device-side routing of a mixture-of-experts mat-mul (one workgroup): slot s = (token t, slot i)
// of ids [n_used, T] goes to expert e = ids[i, t].  The experts' rows are laid out by expert in
// segments of whole `tile`-row tiles (segment e starts where segment e - 1's tiles end), so
// that every row tile of the sorted activation belongs to one expert; tiles[0] receives the
// number of live tiles, tiles[1 + j] the expert of tile j.  src_off / dst_off receive each sorted
// row's byte offset in b and dst (-1: a pad row); the order of an expert's rows follows the
// order in which the slots reach the counter (rows are independent).  A slot whose id lies
// outside [0, n_exp) has no sorted row: its dst row is filled with NaN here.
constexpr int MOE_MAX_EXPERTS = 1024;
__global__ __launch_bounds__(1024) void k_moe_route(const char *__restrict__ ids, int64_t ids_nb1, int n_used, int64_t T,
                                                    int n_exp, int64_t b_ne1, int64_t b_nb1, int64_t b_nb2,
                                                    int64_t d_nb1, int64_t d_nb2, int tile, int64_t rmax,
                                                    int64_t *__restrict__ src_off, int64_t *__restrict__ dst_off,
                                                    int *__restrict__ tiles, char *__restrict__ dst, int64_t n) {
    __shared__ int cnt[MOE_MAX_EXPERTS], start[MOE_MAX_EXPERTS], fill[MOE_MAX_EXPERTS];
    const int tid = threadIdx.x;
    const int64_t R = (int64_t)n_used * T;
    for (int e = tid; e < n_exp; e += 1024) cnt[e] = 0, fill[e] = 0;
    for (int64_t r = tid; r < rmax; r += 1024) src_off[r] = -1, dst_off[r] = -1;
    __syncthreads();
    for (int64_t sl = tid; sl < R; sl += 1024) {
        const int64_t t = sl / n_used, i = sl - t * n_used;
        const int e = *(const int *)(ids + t * ids_nb1 + i * 4);
        if (e >= 0 && e < n_exp) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    if (tid == 0) {
        int64_t run = 0;
        for (int e = 0; e < n_exp; e++) {
            start[e] = (int)run;
            const int nt = (cnt[e] + tile - 1) / tile;
            for (int j = 0; j < nt; j++) tiles[1 + run / tile + j] = e;
            run += (int64_t)nt * tile;
        }
        tiles[0] = (int)(run / tile);
    }
    __syncthreads();
    for (int64_t sl = tid; sl < R; sl += 1024) {
        const int64_t t = sl / n_used, i = sl - t * n_used;
        const int e = *(const int *)(ids + t * ids_nb1 + i * 4);
        const int64_t doff = i * d_nb1 + t * d_nb2;
        if (e >= 0 && e < n_exp) {
            const int64_t r = start[e] + atomicAdd(&fill[e], 1);
            src_off[r] = (i % b_ne1) * b_nb1 + t * b_nb2;
            dst_off[r] = doff;
        } else {
            float *d = (float *)(dst + doff);
            for (int64_t c = 0; c < n; c++) d[c] = __builtin_nanf("");
        }
    }
}

// the sorted rows: row r copied from src + off[r] (zeros for a pad row, off[r] < 0)
__global__ __launch_bounds__(256) void k_gather_rows_pad(const char *__restrict__ src, const int64_t *__restrict__ off,
                                                         float *__restrict__ dst, int64_t k) {
    const int64_t r = blockIdx.x;
    const int64_t o = off[r];
    float4 *d = (float4 *)(dst + r * k);
    if (o < 0) {
        for (int64_t c = threadIdx.x; c < k / 4; c += 256) d[c] = make_float4(0.f, 0.f, 0.f, 0.f);
        return;
    }
    const float4 *sp = (const float4 *)(src + o);
    for (int64_t c = threadIdx.x; c < k / 4; c += 256) d[c] = sp[c];
}

// the results back to their slots (pad rows, off[r] < 0, stay)
__global__ __launch_bounds__(256) void k_scatter_rows_pad(const float *__restrict__ src, const int64_t *__restrict__ off,
                                                          char *__restrict__ dst, int64_t n) {
    const int64_t r = blockIdx.x;
    const int64_t o = off[r];
    if (o < 0) return;
    const float *sp = src + r * n;
    float *d = (float *)(dst + o);
    for (int64_t c = threadIdx.x; c < n; c += 256) d[c] = sp[c];
}

// Softmax over ne0, one wave per row (values re-read from memory; rows are short here).
template <int MT>  // mask element type: 0 none, 1 F16, 2 F32
__global__ __launch_bounds__(256) void k_soft_max(const DV x, const DV m, const DV d, float scale, int64_t nrows) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + wave;
    if (row >= nrows) return;
    const int64_t n = x.ne[0];
    const int64_t i1 = row % x.ne[1], i2 = (row / x.ne[1]) % x.ne[2], i3 = row / (x.ne[1] * x.ne[2]);
    const float *xr = (const float *)(x.p + off3(x, i1, i2, i3));
    float *dr = (float *)(d.p + off3(d, i1, i2, i3));
    const char *mr = MT ? m.p + off3(m, i1, i2 % m.ne[2], i3 % m.ne[3]) : nullptr;
    auto val = [&](int64_t c) {
        float v = xr[c] * scale;
        if constexpr (MT == 1) v += (float)((const _Float16 *)mr)[c];
        if constexpr (MT == 2) v += ((const float *)mr)[c];
        return v;
    };
    float mx = -INFINITY;
    for (int64_t c = lane; c < n; c += 64) mx = fmaxf(mx, val(c));
    mx = wave_max_f(mx);
    if (mx == -INFINITY) {  // every entry masked
        for (int64_t c = lane; c < n; c += 64) dr[c] = 0.f;
        return;
    }
    float sum = 0.f;
    for (int64_t c = lane; c < n; c += 64) {
        const float e = expf(val(c) - mx);
        dr[c] = e;
        sum += e;
    }
    const float inv = 1.0f / wave_sum_f(sum);
    for (int64_t c = lane; c < n; c += 64) dr[c] *= inv;
}

// Stable argsort of one row per workgroup: element i's rank is the number of elements that
// come before it (larger, or equal at a lower index, for descending order).
template <bool DESC>
__global__ __launch_bounds__(256) void k_argsort(const DV x, const DV d, int64_t nrows) {
    __shared__ float v[1024];
    const int64_t row = blockIdx.x;
    const int n = (int)x.ne[0];
    const int64_t i1 = row % x.ne[1], i2 = (row / x.ne[1]) % x.ne[2], i3 = row / (x.ne[1] * x.ne[2]);
    const float *xr = (const float *)(x.p + off3(x, i1, i2, i3));
    int32_t *dr = (int32_t *)(d.p + off3(d, i1, i2, i3));
    for (int c = threadIdx.x; c < n; c += 256) v[c] = xr[c];
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += 256) {
        const float vi = v[i];
        int rank = 0;
        for (int j = 0; j < n; j++) {
            const float vj = v[j];
            rank += DESC ? (vj > vi || (vj == vi && j < i)) : (vj < vi || (vj == vi && j < i));
        }
        dr[rank] = i;
    }
}

__global__ __launch_bounds__(256) void k_repeat(const DV s, const DV d, int64_t n) {
    for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < n; u += (int64_t)gridDim.x * 256) {
        int64_t i0, i1, i2, i3;
        unflat<1>(u, d.ne, i0, i1, i2, i3);
        *(float *)(d.p + i0 * d.nb[0] + off3(d, i1, i2, i3)) =
            *(const float *)(s.p + (i0 % s.ne[0]) * s.nb[0] + off3(s, i1 % s.ne[1], i2 % s.ne[2], i3 % s.ne[3]));
    }
}

// One thread per output element, fp32 multiply-adds in k order.
__global__ __launch_bounds__(256) void k_mul_mat_f32(const DV a, const DV b, const DV d, int64_t n) {
    const int64_t r2 = b.ne[2] / a.ne[2], r3 = b.ne[3] / a.ne[3];
    for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < n; u += (int64_t)gridDim.x * 256) {
        int64_t i, j, b2, b3;
        unflat<1>(u, d.ne, i, j, b2, b3);
        const char *ar = a.p + i * a.nb[1] + (b2 / r2) * a.nb[2] + (b3 / r3) * a.nb[3];
        const char *br = b.p + j * b.nb[1] + b2 * b.nb[2] + b3 * b.nb[3];
        float acc = 0.f;
        for (int64_t k = 0; k < a.ne[0]; k++) acc += *(const float *)(ar + k * a.nb[0]) * *(const float *)(br + k * b.nb[0]);
        *(float *)(d.p + i * d.nb[0] + off3(d, j, b2, b3)) = acc;
    }
}

// ------------------------------------------------------------------ checks ----
int64_t nel(const mq_view *v) { return v->ne[0] * v->ne[1] * v->ne[2] * v->ne[3]; }

// Checks read only shapes, types and strides (and the data address's alignment, where data is
// set: mq_op_supported is asked about tensors that are not allocated yet).
bool shape_ok(const mq_view *v) {
    for (int i = 0; i < 4; i++)
        if (v->ne[i] < 1 || v->ne[i] > ((int64_t)1 << 31)) return false;
    return true;
}

bool have_data(std::initializer_list<const mq_view *> vs) {
    for (const mq_view *v : vs)
        if (v && !v->data) return false;
    return true;
}

bool same_shape(const mq_view *a, const mq_view *b) {
    for (int i = 0; i < 4; i++)
        if (a->ne[i] != b->ne[i]) return false;
    return true;
}

// rows of the view are contiguous elements of `esize` bytes
bool rows_dense(const mq_view *v, size_t esize) { return v->nb[0] == esize; }

// every float4 access stays 16-byte aligned
bool vec4_ok(const mq_view *v) {
    if (v->nb[0] != 4 || v->ne[0] % 4 != 0 || ((uintptr_t)v->data & 15) != 0) return false;
    for (int i = 1; i < 4; i++)
        if (v->ne[i] > 1 && v->nb[i] % 16 != 0) return false;
    return true;
}

size_t elem_size(int type) { return type == MQ_TYPE_F16 ? 2 : 4; }

const char *check_get_rows(const mq_view *src, const mq_view *ids, const mq_view *dst) {
    if (!src || !ids || !dst || !shape_ok(src) || !shape_ok(ids) || !shape_ok(dst)) return "missing or empty operand";
    const int t = src->type;
    if (t != MQ_TYPE_F32 && t != MQ_TYPE_F16 && t != MQ_TYPE_Q8_0 && t != MQ_TYPE_Q4_K && t != MQ_TYPE_Q6_K)
        return "get_rows: table type not F32/F16/Q8_0/Q4_K/Q6_K";
    if (ids->type != MQ_TYPE_I32 || dst->type != MQ_TYPE_F32) return "get_rows: ids must be I32 and dst F32";
    if (ids->ne[3] != 1) return "get_rows: ids has 4 dimensions";
    const int64_t bs = blck_size(t);
    if (src->ne[0] % bs != 0) return "get_rows: row length not a multiple of the block";
    if (t == MQ_TYPE_F32 || t == MQ_TYPE_F16) {
        if (src->nb[0] != elem_size(t)) return "get_rows: table rows not contiguous";
    } else if (src->nb[0] != type_size(t)) {
        return "get_rows: table rows not contiguous";
    }
    if (dst->ne[0] != src->ne[0] || dst->ne[1] != ids->ne[0] || dst->ne[2] != ids->ne[1] || dst->ne[3] != ids->ne[2])
        return "get_rows: dst shape";
    if (ids->ne[1] != src->ne[2] || ids->ne[2] != src->ne[3]) return "get_rows: ids / table planes differ";
    if (dst->nb[0] != 4) return "get_rows: dst rows not contiguous";
    return nullptr;
}

const char *check_binary(int op, const mq_view *a, const mq_view *b, const mq_view *d) {
    if (op < MQ_BIN_ADD || op > MQ_BIN_DIV) return "binary: unknown op";
    if (!a || !b || !d || !shape_ok(a) || !shape_ok(b) || !shape_ok(d)) return "missing or empty operand";
    if (a->type != MQ_TYPE_F32 || b->type != MQ_TYPE_F32 || d->type != MQ_TYPE_F32) return "binary: F32 only";
    if (!same_shape(a, d)) return "binary: dst shape differs from src0";
    for (int i = 0; i < 4; i++)
        if (a->ne[i] % b->ne[i] != 0) return "binary: src1 does not broadcast over src0";
    if (a->nb[0] % 4 || b->nb[0] % 4 || d->nb[0] % 4) return "binary: misaligned strides";
    return nullptr;
}

const char *check_unary(int op, const mq_view *x, const mq_view *d) {
    if (op < MQ_UNARY_GELU_ERF || op > MQ_UNARY_RELU) return "unary: unknown op";
    if (!x || !d || !shape_ok(x) || !shape_ok(d)) return "missing or empty operand";
    if (x->type != MQ_TYPE_F32 || d->type != MQ_TYPE_F32) return "unary: F32 only";
    if (!same_shape(x, d)) return "unary: shapes differ";
    return nullptr;
}

const char *check_norm(int kind, const mq_view *x, const mq_view *r, const mq_view *d) {
    if (kind != MQ_NORM_LAYER && kind != MQ_NORM_RMS) return "norm: unknown kind";
    if (!x || !d || !shape_ok(x) || !shape_ok(d)) return "missing or empty operand";
    if (x->type != MQ_TYPE_F32 || d->type != MQ_TYPE_F32) return "norm: F32 only";
    if (!same_shape(x, d)) return "norm: shapes differ";
    if (!rows_dense(x, 4) || !rows_dense(d, 4)) return "norm: rows not contiguous";
    if (r && (!shape_ok(r) || r->type != MQ_TYPE_F32 || !same_shape(x, r) || !rows_dense(r, 4)))
        return "norm: the added tensor must be F32 with x's shape and contiguous rows";
    return nullptr;
}

const char *check_cpy(const mq_view *s, const mq_view *d) {
    if (!s || !d || !shape_ok(s) || !shape_ok(d)) return "missing or empty operand";
    if ((s->type != MQ_TYPE_F32 && s->type != MQ_TYPE_F16) || (d->type != MQ_TYPE_F32 && d->type != MQ_TYPE_F16))
        return "cpy: F32 / F16 only";
    if (nel(s) != nel(d)) return "cpy: element counts differ";
    if (s->nb[0] % elem_size(s->type) || d->nb[0] % elem_size(d->type)) return "cpy: misaligned strides";
    return nullptr;
}

const char *check_flash(const mq_view *q, const mq_view *k, const mq_view *v, const mq_view *m, const mq_view *d) {
    if (!q || !k || !v || !d || !shape_ok(q) || !shape_ok(k) || !shape_ok(v) || !shape_ok(d))
        return "missing or empty operand";
    if (q->type != MQ_TYPE_F32 || k->type != MQ_TYPE_F32 || v->type != MQ_TYPE_F32 || d->type != MQ_TYPE_F32)
        return "flash_attn: q, k, v and dst must be F32";
    const int64_t hd = q->ne[0];
    if (hd != 32 && hd != 64 && hd != 128) return "flash_attn: head_dim not 32, 64 or 128";
    if (k->ne[0] != hd || v->ne[0] != hd) return "flash_attn: k / v head_dim differs from q";
    if (k->ne[1] != v->ne[1] || k->ne[2] != v->ne[2] || k->ne[3] != v->ne[3]) return "flash_attn: k and v shapes differ";
    if (q->ne[2] % k->ne[2] != 0) return "flash_attn: query heads not a multiple of kv heads";
    if (k->ne[3] != q->ne[3] || q->ne[3] > 65535) return "flash_attn: batch";
    if (d->ne[0] != hd || d->ne[1] != q->ne[2] || d->ne[2] != q->ne[1] || d->ne[3] != q->ne[3])
        return "flash_attn: dst must be [hd, n_head, Tq, B]";
    if (q->nb[0] != 4 || k->nb[0] != 4 || v->nb[0] != 4 || d->nb[0] != 4) return "flash_attn: head rows not contiguous";
    if (((uintptr_t)q->data & 15) || q->nb[1] % 16 || q->nb[2] % 16 || q->nb[3] % 16)
        return "flash_attn: q not 16-byte aligned";
    for (const mq_view *t : {k, v, d})
        if (t->nb[1] % 4 || t->nb[2] % 4 || t->nb[3] % 4) return "flash_attn: misaligned strides";
    if (m) {
        if (!shape_ok(m) || m->type != MQ_TYPE_F16 || m->nb[0] != 2) return "flash_attn: mask must be F16 rows";
        if (m->ne[0] < k->ne[1] || m->ne[1] < q->ne[1]) return "flash_attn: mask smaller than [Tk, Tq]";
        if ((m->ne[2] != 1 && m->ne[2] != q->ne[2]) || (m->ne[3] != 1 && m->ne[3] != q->ne[3]))
            return "flash_attn: mask heads / batches do not broadcast";
        if (m->nb[1] % 2 || m->nb[2] % 2 || m->nb[3] % 2) return "flash_attn: misaligned mask strides";
    }
    return nullptr;
}

const char *check_rope(int mode, const mq_view *x, const mq_view *pos, const mq_view *ff, const mq_view *d, int n_dims) {
    if (mode != MQ_ROPE_NORMAL && mode != MQ_ROPE_NEOX) return "rope: mode not 0 (normal) or 2 (NEOX)";
    if (!x || !pos || !d || !shape_ok(x) || !shape_ok(pos) || !shape_ok(d)) return "missing or empty operand";
    if (x->type != MQ_TYPE_F32 || d->type != MQ_TYPE_F32 || pos->type != MQ_TYPE_I32) return "rope: F32 x, I32 pos";
    if (!same_shape(x, d) || !rows_dense(x, 4) || !rows_dense(d, 4)) return "rope: x / dst shapes or rows";
    if (n_dims <= 0 || n_dims % 2 || n_dims > x->ne[0] || x->ne[0] % 2) return "rope: n_dims";
    if (pos->ne[0] != x->ne[2] || pos->ne[1] != 1 || pos->ne[2] != 1 || pos->ne[3] != 1) return "rope: pos must be [T]";
    if (ff && (!shape_ok(ff) || ff->type != MQ_TYPE_F32 || ff->nb[0] != 4 || ff->ne[0] < n_dims / 2))
        return "rope: freq_factors must be F32 [n_dims/2]";
    return nullptr;
}

const char *check_soft_max(const mq_view *x, const mq_view *m, const mq_view *d) {
    if (!x || !d || !shape_ok(x) || !shape_ok(d)) return "missing or empty operand";
    if (x->type != MQ_TYPE_F32 || d->type != MQ_TYPE_F32 || !same_shape(x, d)) return "soft_max: F32 x / dst";
    if (!rows_dense(x, 4) || !rows_dense(d, 4)) return "soft_max: rows not contiguous";
    if (m) {
        if (!shape_ok(m) || (m->type != MQ_TYPE_F16 && m->type != MQ_TYPE_F32) || !rows_dense(m, elem_size(m->type)))
            return "soft_max: mask must be F16 or F32 rows";
        if (m->ne[0] != x->ne[0] || m->ne[1] < x->ne[1]) return "soft_max: mask shape";
        if (x->ne[2] % m->ne[2] || x->ne[3] % m->ne[3]) return "soft_max: mask planes do not broadcast";
    }
    return nullptr;
}

const char *check_argsort(int order, const mq_view *x, const mq_view *d) {
    if (order != MQ_SORT_ASC && order != MQ_SORT_DESC) return "argsort: order";
    if (!x || !d || !shape_ok(x) || !shape_ok(d)) return "missing or empty operand";
    if (x->type != MQ_TYPE_F32 || d->type != MQ_TYPE_I32 || !same_shape(x, d)) return "argsort: F32 x, I32 dst";
    if (x->ne[0] > 1024) return "argsort: rows of at most 1024";
    if (!rows_dense(x, 4) || !rows_dense(d, 4)) return "argsort: rows not contiguous";
    return nullptr;
}

const char *check_repeat(const mq_view *s, const mq_view *d) {
    if (!s || !d || !shape_ok(s) || !shape_ok(d)) return "missing or empty operand";
    if (s->type != MQ_TYPE_F32 || d->type != MQ_TYPE_F32) return "repeat: F32 only";
    for (int i = 0; i < 4; i++)
        if (d->ne[i] % s->ne[i]) return "repeat: src does not tile dst";
    return nullptr;
}

const char *check_mul_mat_f32(const mq_view *a, const mq_view *b, const mq_view *d) {
    if (!a || !b || !d || !shape_ok(a) || !shape_ok(b) || !shape_ok(d)) return "missing or empty operand";
    if (a->type != MQ_TYPE_F32 || b->type != MQ_TYPE_F32 || d->type != MQ_TYPE_F32) return "mul_mat_f32: F32 only";
    if (a->ne[0] != b->ne[0] || b->ne[2] % a->ne[2] || b->ne[3] % a->ne[3]) return "mul_mat_f32: shapes";
    if (d->ne[0] != a->ne[1] || d->ne[1] != b->ne[1] || d->ne[2] != b->ne[2] || d->ne[3] != b->ne[3])
        return "mul_mat_f32: dst shape";
    if (a->nb[0] % 4 || b->nb[0] % 4 || d->nb[0] % 4) return "mul_mat_f32: misaligned strides";
    if ((double)nel(d) * (double)a->ne[0] > (double)(1ll << 26)) return "mul_mat_f32: more than 2^26 multiply-adds";
    return nullptr;
}

unsigned grid_units(int64_t units) {
    const int64_t g = (units + 255) / 256;
    return (unsigned)(g < 8192 ? (g > 0 ? g : 1) : 8192);
}

int fail(const char *msg) { return set_error(strstr(msg, "missing") ? MQ_EINVAL : MQ_EUNSUPPORTED, "%s", msg); }

template <int OP>
void launch_binary_op(const mq_view *a, const mq_view *b, const mq_view *d, hipStream_t s) {
    const bool v4 = vec4_ok(a) && vec4_ok(d) && b->ne[0] == a->ne[0] && vec4_ok(b);
    const int64_t units = nel(a) / (v4 ? 4 : 1);
    if (v4) hipLaunchKernelGGL((k_binary<OP, 4>), dim3(grid_units(units)), dim3(256), 0, s, dv(a), dv(b), dv(d), units);
    else hipLaunchKernelGGL((k_binary<OP, 1>), dim3(grid_units(units)), dim3(256), 0, s, dv(a), dv(b), dv(d), units);
}

template <int OP>
void launch_unary_op(const mq_view *x, const mq_view *d, hipStream_t s) {
    const bool v4 = vec4_ok(x) && vec4_ok(d);
    const int64_t units = nel(x) / (v4 ? 4 : 1);
    if (v4) hipLaunchKernelGGL((k_unary<OP, 4>), dim3(grid_units(units)), dim3(256), 0, s, dv(x), dv(d), units);
    else hipLaunchKernelGGL((k_unary<OP, 1>), dim3(grid_units(units)), dim3(256), 0, s, dv(x), dv(d), units);
}

template <int KIND>
void launch_norm_kind(const mq_view *x, const mq_view *r, const mq_view *d, float eps, const float *w, const float *b,
                      hipStream_t s) {
    const int64_t rows = x->ne[1] * x->ne[2] * x->ne[3];
    const dim3 g((unsigned)((rows + 3) / 4)), blk(256);
    const int64_t need = (x->ne[0] + 63) / 64;
    DV rv{};
    if (r) rv = dv(r);
    if (need <= 4) hipLaunchKernelGGL((k_norm<KIND, 4>), g, blk, 0, s, dv(x), rv, dv(d), eps, w, b, rows);
    else if (need <= 8) hipLaunchKernelGGL((k_norm<KIND, 8>), g, blk, 0, s, dv(x), rv, dv(d), eps, w, b, rows);
    else if (need <= 16) hipLaunchKernelGGL((k_norm<KIND, 16>), g, blk, 0, s, dv(x), rv, dv(d), eps, w, b, rows);
    else hipLaunchKernelGGL((k_norm<KIND, 0>), g, blk, 0, s, dv(x), rv, dv(d), eps, w, b, rows);
}

}  // namespace
}  // namespace mq

using namespace mq;

extern "C" int mq_op_get_rows(const mq_view *src, const mq_view *ids, const mq_view *dst, void *stream) {
    if (const char *e = check_get_rows(src, ids, dst)) return fail(e);
    if (!have_data({src, ids, dst})) return fail("missing data pointer");
    const int64_t rows = ids->ne[0] * ids->ne[1] * ids->ne[2];
    const dim3 g((unsigned)((rows + 3) / 4)), b(256);
    hipStream_t s = (hipStream_t)stream;
    switch (src->type) {
        case MQ_TYPE_F32: hipLaunchKernelGGL((k_get_rows<MQ_TYPE_F32>), g, b, 0, s, dv(src), dv(ids), dv(dst), rows); break;
        case MQ_TYPE_F16: hipLaunchKernelGGL((k_get_rows<MQ_TYPE_F16>), g, b, 0, s, dv(src), dv(ids), dv(dst), rows); break;
        case MQ_TYPE_Q8_0: hipLaunchKernelGGL((k_get_rows<MQ_TYPE_Q8_0>), g, b, 0, s, dv(src), dv(ids), dv(dst), rows); break;
        case MQ_TYPE_Q4_K: hipLaunchKernelGGL((k_get_rows<MQ_TYPE_Q4_K>), g, b, 0, s, dv(src), dv(ids), dv(dst), rows); break;
        default: hipLaunchKernelGGL((k_get_rows<MQ_TYPE_Q6_K>), g, b, 0, s, dv(src), dv(ids), dv(dst), rows); break;
    }
    return hip_rc(hipGetLastError(), "get_rows");
}

extern "C" int mq_op_get_rows_sum(int n, const mq_view *const *srcs, const mq_view *const *ids, const mq_view *dst,
                                  void *stream) {
    if (n < 2 || n > 3 || !srcs || !ids || !dst || !shape_ok(dst)) return fail("get_rows_sum: 2 or 3 tables and a dst");
    if (dst->type != MQ_TYPE_F32 || dst->nb[0] != 4 || dst->nb[1] != (size_t)dst->ne[0] * 4 || dst->ne[2] != 1 ||
        dst->ne[3] != 1)
        return fail("get_rows_sum: dst must be dense F32 rows [ne0, rows]");
    const int64_t ne0 = dst->ne[0], rows = dst->ne[1];
    RowsSumArgs a{};
    a.n = n;
    bool v4 = ne0 % 4 == 0 && ((uintptr_t)dst->data & 15) == 0;
    for (int t = 0; t < n; t++) {
        const mq_view *S = srcs[t], *I = ids[t];
        if (!S || !I || !shape_ok(S) || !shape_ok(I)) return fail("missing or empty operand");
        if (S->type != MQ_TYPE_F32 || S->nb[0] != 4 || S->ne[0] != ne0 || S->ne[2] != 1 || S->ne[3] != 1)
            return fail("get_rows_sum: tables must be F32 [ne0, rows] with contiguous rows");
        if (I->type != MQ_TYPE_I32 || I->nb[0] != 4 || I->ne[0] != rows || I->ne[1] != 1 || I->ne[2] != 1 ||
            I->ne[3] != 1)
            return fail("get_rows_sum: ids must be I32 vectors of dst's row count");
        if (!S->data || !I->data) return fail("missing data pointer");
        a.tab[t] = (const float *)S->data;
        a.ids[t] = (const int32_t *)I->data;
        a.ntab_rows[t] = S->ne[1];
        a.ld[t] = (int64_t)(S->nb[1] / 4);
        v4 = v4 && S->nb[1] % 16 == 0 && ((uintptr_t)S->data & 15) == 0;
    }
    if (!dst->data) return fail("missing data pointer");
    const dim3 g((unsigned)((rows + 3) / 4)), b(256);
    if (v4) hipLaunchKernelGGL((k_get_rows_sum<true>), g, b, 0, (hipStream_t)stream, a, (float *)dst->data, rows, ne0);
    else hipLaunchKernelGGL((k_get_rows_sum<false>), g, b, 0, (hipStream_t)stream, a, (float *)dst->data, rows, ne0);
    return hip_rc(hipGetLastError(), "get_rows_sum");
}

extern "C" int mq_op_binary(int op, const mq_view *a, const mq_view *b, const mq_view *dst, void *stream) {
    if (const char *e = check_binary(op, a, b, dst)) return fail(e);
    if (!have_data({a, b, dst})) return fail("missing data pointer");
    hipStream_t s = (hipStream_t)stream;
    switch (op) {
        case MQ_BIN_ADD: launch_binary_op<MQ_BIN_ADD>(a, b, dst, s); break;
        case MQ_BIN_SUB: launch_binary_op<MQ_BIN_SUB>(a, b, dst, s); break;
        case MQ_BIN_MUL: launch_binary_op<MQ_BIN_MUL>(a, b, dst, s); break;
        default: launch_binary_op<MQ_BIN_DIV>(a, b, dst, s); break;
    }
    return hip_rc(hipGetLastError(), "binary op");
}

extern "C" int mq_op_unary(int op, const mq_view *x, const mq_view *dst, void *stream) {
    if (const char *e = check_unary(op, x, dst)) return fail(e);
    if (!have_data({x, dst})) return fail("missing data pointer");
    hipStream_t s = (hipStream_t)stream;
    switch (op) {
        case MQ_UNARY_GELU_ERF: launch_unary_op<MQ_UNARY_GELU_ERF>(x, dst, s); break;
        case MQ_UNARY_GELU: launch_unary_op<MQ_UNARY_GELU>(x, dst, s); break;
        case MQ_UNARY_SILU: launch_unary_op<MQ_UNARY_SILU>(x, dst, s); break;
        default: launch_unary_op<MQ_UNARY_RELU>(x, dst, s); break;
    }
    return hip_rc(hipGetLastError(), "unary op");
}

extern "C" int mq_op_norm(int kind, const mq_view *x, const mq_view *add, const mq_view *dst, float eps,
                          const float *w, const float *b, void *stream) {
    if (const char *e = check_norm(kind, x, add, dst)) return fail(e);
    if (!have_data({x, add, dst})) return fail("missing data pointer");
    hipStream_t s = (hipStream_t)stream;
    if (kind == MQ_NORM_LAYER) launch_norm_kind<MQ_NORM_LAYER>(x, add, dst, eps, w, b, s);
    else launch_norm_kind<MQ_NORM_RMS>(x, add, dst, eps, w, b, s);
    return hip_rc(hipGetLastError(), "norm");
}

template <int KIND, int NW, int RT>
static void launch_norm_q8_0_rt(int nv, const float *x, const float *r, float *d, float eps, const float *w,
                                const float *b, int64_t rows, int8_t *xq, float *xd, int64_t m_pad, int variant,
                                hipStream_t s) {
    const dim3 grid((unsigned)((rows + 31) / 32 * (32 / RT))), block(64 * NW);
    switch (nv) {
#define MQ_NQ(NV)                                                                                                      \
    case NV:                                                                                                           \
        hipLaunchKernelGGL((k_norm_q8_0<KIND, NV, NW, RT>), grid, block, 0, s, x, r, d, eps, w, b, rows, xq, xd,       \
                           m_pad, variant);                                                                            \
        break;
        MQ_NQ(1) MQ_NQ(2) MQ_NQ(3) MQ_NQ(4) MQ_NQ(5) MQ_NQ(6) MQ_NQ(7) MQ_NQ(8)
#undef MQ_NQ
        default: break;
    }
}

// 8-row workgroups of 4 waves; at most 1024 rows, 2-row workgroups of one wave, so a 384-row
// input spreads over 192 CUs instead of 48.  MQ_NORM_RT=2/8 forces either (measurements).
template <int KIND>
static void launch_norm_q8_0_kind(int nv, const float *x, const float *r, float *d, float eps, const float *w,
                                  const float *b, int64_t rows, int8_t *xq, float *xd, int64_t m_pad, int variant,
                                  hipStream_t s) {
    int rt = rows <= 1024 ? 2 : 8;
    if (const char *e = getenv("MQ_NORM_RT"))
        if (*e) rt = atoi(e) == 2 ? 2 : 8;
    if (rt == 2) launch_norm_q8_0_rt<KIND, 1, 2>(nv, x, r, d, eps, w, b, rows, xq, xd, m_pad, variant, s);
    else launch_norm_q8_0_rt<KIND, 4, 8>(nv, x, r, d, eps, w, b, rows, xq, xd, m_pad, variant, s);
}

extern "C" int mq_op_norm_q8_0(int kind, const mq_view *x, const mq_view *add, const mq_view *dst, float eps,
                               const float *w, const float *b, void *workspace, size_t workspace_bytes, void *stream) {
    if (const char *e = check_norm(kind, x, add, dst)) return fail(e);
    if (!have_data({x, add, dst}) || !workspace) return fail("missing data pointer");
    const int64_t K = x->ne[0], rows = x->ne[1] * x->ne[2] * x->ne[3];
    if (K % 128 != 0 || K > 1024) return fail("norm_q8_0: ne0 must be a multiple of 128, at most 1024");
    for (const mq_view *t : {x, add, dst})
        if (t && (t->nb[1] != (size_t)K * 4 || t->nb[2] != t->nb[1] * (size_t)t->ne[1] ||
                  t->nb[3] != t->nb[2] * (size_t)t->ne[2] || ((uintptr_t)t->data & 15)))
            return fail("norm_q8_0: x, add and dst must be dense, 16-byte aligned rows");
    if (((uintptr_t)w & 15) || ((uintptr_t)b & 15) || ((uintptr_t)workspace & 255))
        return fail("norm_q8_0: w and b 16-byte, the workspace 256-byte aligned");
    if (rows > INT32_MAX) return fail("norm_q8_0: too many rows");
    const ActPlanes ap = act_planes(MQ_TYPE_Q8_0, rows, K, true);
    if (ap.kb_pad != K) return fail("norm_q8_0: K padding");
    if (workspace_bytes < ap.total) return fail("norm_q8_0: workspace too small");
    uint8_t *ws = (uint8_t *)workspace;
    hipStream_t s = (hipStream_t)stream;
    const float *r = add ? (const float *)add->data : nullptr;
    const int var = mq_q8_0_variant();
    if (kind == MQ_NORM_LAYER)
        launch_norm_q8_0_kind<MQ_NORM_LAYER>((int)(K / 128), (const float *)x->data, r, (float *)dst->data, eps, w, b,
                                             rows, (int8_t *)(ws + ap.xq), (float *)(ws + ap.xd), ap.m_pad, var, s);
    else
        launch_norm_q8_0_kind<MQ_NORM_RMS>((int)(K / 128), (const float *)x->data, r, (float *)dst->data, eps, w, b,
                                           rows, (int8_t *)(ws + ap.xq), (float *)(ws + ap.xd), ap.m_pad, var, s);
    return hip_rc(hipGetLastError(), "norm_q8_0");
}

extern "C" int mq_op_norm_q8_K(int kind, const mq_view *x, const mq_view *add, const mq_view *sum, const mq_view *dst,
                               float eps, const float *w, void *workspace, size_t workspace_bytes, void *stream) {
    if (kind != MQ_NORM_RMS) return fail("norm_q8_K: RMS norm only");
    if (const char *e = check_norm(kind, x, add, dst ? dst : x)) return fail(e);
    if (sum && (sum->type != MQ_TYPE_F32 || !shape_ok(sum) || !same_shape(x, sum)))
        return fail("norm_q8_K: sum must be F32 with x's shape");
    if (!have_data({x, add, sum, dst}) || !workspace || !w) return fail("missing data pointer");
    const int64_t K = x->ne[0], rows = x->ne[1] * x->ne[2] * x->ne[3];
    if (K % 256 != 0 || K > 2048) return fail("norm_q8_K: ne0 must be a multiple of 256, at most 2048");
    for (const mq_view *t : {x, add, sum, dst})
        if (t && (t->nb[0] != 4 || t->nb[1] != (size_t)K * 4 || t->nb[2] != t->nb[1] * (size_t)t->ne[1] ||
                  t->nb[3] != t->nb[2] * (size_t)t->ne[2] || ((uintptr_t)t->data & 15)))
            return fail("norm_q8_K: x, add, sum and dst must be dense, 16-byte aligned rows");
    if (((uintptr_t)w & 15) || ((uintptr_t)workspace & 255))
        return fail("norm_q8_K: w 16-byte, the workspace 256-byte aligned");
    if (rows > INT32_MAX) return fail("norm_q8_K: too many rows");
    const ActPlanes ap = act_planes(MQ_TYPE_Q4_K, rows, K, true);
    if (workspace_bytes < ap.total) return fail("norm_q8_K: workspace too small");
    const hipError_t e =
        launch_add_rmsnorm_q8_K((const float *)x->data, add ? (const float *)add->data : nullptr, w, eps,
                                sum ? (float *)sum->data : nullptr, dst ? (float *)dst->data : nullptr, rows, (int)K,
                                workspace, (hipStream_t)stream);
    return hip_rc(e, "norm_q8_K");
}

extern "C" int mq_op_cpy(const mq_view *src, const mq_view *dst, void *stream) {
    if (const char *e = check_cpy(src, dst)) return fail(e);
    if (!have_data({src, dst})) return fail("missing data pointer");
    hipStream_t s = (hipStream_t)stream;
    const int64_t n = nel(src);
    const bool f32s = src->type == MQ_TYPE_F32, f32d = dst->type == MQ_TYPE_F32;
    if (same_shape(src, dst)) {
        if (f32s && f32d && vec4_ok(src) && vec4_ok(dst)) {
            hipLaunchKernelGGL((k_cpy_same<float, float, 4>), dim3(grid_units(n / 4)), dim3(256), 0, s, dv(src), dv(dst),
                               n / 4);
        } else if (f32s && f32d) {
            hipLaunchKernelGGL((k_cpy_same<float, float, 1>), dim3(grid_units(n)), dim3(256), 0, s, dv(src), dv(dst), n);
        } else if (f32s) {
            hipLaunchKernelGGL((k_cpy_same<float, _Float16, 1>), dim3(grid_units(n)), dim3(256), 0, s, dv(src), dv(dst), n);
        } else if (f32d) {
            hipLaunchKernelGGL((k_cpy_same<_Float16, float, 1>), dim3(grid_units(n)), dim3(256), 0, s, dv(src), dv(dst), n);
        } else {
            hipLaunchKernelGGL((k_cpy_same<_Float16, _Float16, 1>), dim3(grid_units(n)), dim3(256), 0, s, dv(src),
                               dv(dst), n);
        }
    } else {
        if (f32s && f32d) hipLaunchKernelGGL((k_cpy_any<float, float>), dim3(grid_units(n)), dim3(256), 0, s, dv(src), dv(dst), n);
        else if (f32s) hipLaunchKernelGGL((k_cpy_any<float, _Float16>), dim3(grid_units(n)), dim3(256), 0, s, dv(src), dv(dst), n);
        else if (f32d) hipLaunchKernelGGL((k_cpy_any<_Float16, float>), dim3(grid_units(n)), dim3(256), 0, s, dv(src), dv(dst), n);
        else hipLaunchKernelGGL((k_cpy_any<_Float16, _Float16>), dim3(grid_units(n)), dim3(256), 0, s, dv(src), dv(dst), n);
    }
    return hip_rc(hipGetLastError(), "cpy");
}

// YaRN correction dimension of rotation count n_rot (ggml_rope_yarn_corr_dim's formula)
static float yarn_corr_dim(int n_dims, int n_ctx_orig, float n_rot, float base) {
    return n_dims * logf((float)n_ctx_orig / (n_rot * 2.0f * 3.14159265358979323846f)) / (2.0f * logf(base));
}

static RopeParams rope_params(int n_dims, int mode, int n_ctx_orig, float freq_base, float freq_scale, float ext_factor,
                              float attn_factor, float beta_fast, float beta_slow) {
    RopeParams rp;
    rp.n_dims = n_dims, rp.mode = mode;
    rp.theta_scale = powf(freq_base, -2.0f / (float)n_dims);
    rp.freq_scale = freq_scale, rp.ext_factor = ext_factor, rp.attn_factor = attn_factor;
    const float lo = floorf(yarn_corr_dim(n_dims, n_ctx_orig, beta_fast, freq_base));
    const float hi = ceilf(yarn_corr_dim(n_dims, n_ctx_orig, beta_slow, freq_base));
    rp.corr_lo = fmaxf(0.0f, lo);
    rp.corr_hi = fminf((float)(n_dims - 1), hi);
    return rp;
}

extern "C" int mq_op_rms_norm_rope(const mq_view *x, float eps, const float *w, const mq_view *pos,
                                   const mq_view *freq_factors, const mq_view *dst, int n_dims, int mode,
                                   int n_ctx_orig, float freq_base, float freq_scale, float ext_factor,
                                   float attn_factor, float beta_fast, float beta_slow, void *stream) {
    if (const char *e = check_rope(mode, x, pos, freq_factors, dst, n_dims)) return fail(e);
    if (!have_data({x, pos, freq_factors, dst}) || !w) return fail("missing data pointer");
    if (mode != MQ_ROPE_NEOX || n_dims != 128 || x->ne[0] != 128)
        return fail("rms_norm_rope: the NEOX rotation of all of ne0 = 128 dimensions only");
    if (x->ne[2] * x->ne[3] > INT32_MAX) return fail("rms_norm_rope: too many positions");
    const RopeParams rp = rope_params(n_dims, mode, n_ctx_orig, freq_base, freq_scale, ext_factor, attn_factor,
                                      beta_fast, beta_slow);
    const float *ff = freq_factors ? (const float *)freq_factors->data : nullptr;
    hipLaunchKernelGGL((k_rope_rows<MQ_ROPE_NEOX, true>), dim3((unsigned)(x->ne[2] * x->ne[3])), dim3(256), 0,
                       (hipStream_t)stream, dv(x), dv(pos), ff, dv(dst), rp, w, eps);
    return hip_rc(hipGetLastError(), "rms_norm_rope");
}

extern "C" int mq_op_rope(const mq_view *x, const mq_view *pos, const mq_view *freq_factors, const mq_view *dst,
                          int n_dims, int mode, int n_ctx_orig, float freq_base, float freq_scale, float ext_factor,
                          float attn_factor, float beta_fast, float beta_slow, void *stream) {
    if (const char *e = check_rope(mode, x, pos, freq_factors, dst, n_dims)) return fail(e);
    if (!have_data({x, pos, freq_factors, dst})) return fail("missing data pointer");
    const RopeParams rp = rope_params(n_dims, mode, n_ctx_orig, freq_base, freq_scale, ext_factor, attn_factor,
                                      beta_fast, beta_slow);
    const int64_t units = nel(x) / 2;
    const float *ff = freq_factors ? (const float *)freq_factors->data : nullptr;
    hipStream_t s = (hipStream_t)stream;
    if (x->ne[0] == n_dims && n_dims <= 128 && x->ne[2] * x->ne[3] <= INT32_MAX) {  // every dimension rotated
        const dim3 g((unsigned)(x->ne[2] * x->ne[3])), b(256);
        if (mode == MQ_ROPE_NEOX)
            hipLaunchKernelGGL((k_rope_rows<MQ_ROPE_NEOX, false>), g, b, 0, s, dv(x), dv(pos), ff, dv(dst), rp, nullptr, 0.f);
        else
            hipLaunchKernelGGL((k_rope_rows<MQ_ROPE_NORMAL, false>), g, b, 0, s, dv(x), dv(pos), ff, dv(dst), rp, nullptr,
                               0.f);
        return hip_rc(hipGetLastError(), "rope");
    }
    if (mode == MQ_ROPE_NEOX)
        hipLaunchKernelGGL((k_rope<MQ_ROPE_NEOX>), dim3(grid_units(units)), dim3(256), 0, s, dv(x), dv(pos), ff, dv(dst), rp,
                           units);
    else
        hipLaunchKernelGGL((k_rope<MQ_ROPE_NORMAL>), dim3(grid_units(units)), dim3(256), 0, s, dv(x), dv(pos), ff, dv(dst),
                           rp, units);
    return hip_rc(hipGetLastError(), "rope");
}

// workspace of the mixture-of-experts mat-mul: gathered rows, their results, the two offset
// lists and the activation quantization of up to `rows` rows
struct MoeWs {
    size_t x, y, src_off, dst_off, q, total;
};
static MoeWs moe_ws(int type, int64_t n, int64_t k, int64_t rows) {
    MoeWs w;
    size_t o = 0;
    auto take = [&](size_t b) {
        const size_t at = o;
        o = align256(o + b);
        return at;
    };
    w.x = take((size_t)rows * k * 4);
    w.y = take((size_t)rows * n * 4);
    w.src_off = take((size_t)rows * 8);
    w.dst_off = take((size_t)rows * 8);
    w.q = take(mq_workspace_bytes(type, rows, k));
    w.total = o;
    return w;
}

extern "C" size_t mq_op_mul_mat_id_workspace_bytes(int type, int64_t n, int64_t k, int64_t rows) {
    if (n <= 0 || k <= 0 || rows <= 0 || mq_row_size(type, k) == 0) return 0;
    return moe_ws(type, n, k, rows).total;
}

extern "C" int mq_op_mul_mat_id(int type, const void *expert_images, size_t expert_stride, int n_exp, int64_t n,
                                int64_t k, const mq_view *b, const mq_view *ids, const mq_view *dst, void *workspace,
                                size_t workspace_bytes, void *stream) {
    if (!expert_images || n_exp <= 0 || !b || !ids || !dst || !b->data || !ids->data || !dst->data || !workspace)
        return set_error(MQ_EINVAL, "mq_op_mul_mat_id: missing operand");
    if (!mq_supports(type, k) || n <= 0 || (expert_stride % 256) != 0 || ((uintptr_t)expert_images & 255) != 0)
        return set_error(MQ_EUNSUPPORTED, "mq_op_mul_mat_id: weight type %d with k %lld", type, (long long)k);
    if (!shape_ok(b) || !shape_ok(ids) || !shape_ok(dst) || b->type != MQ_TYPE_F32 || ids->type != MQ_TYPE_I32 ||
        dst->type != MQ_TYPE_F32)
        return set_error(MQ_EINVAL, "mq_op_mul_mat_id: types (F32 b and dst, I32 ids)");
    const int64_t n_used = ids->ne[0], T = ids->ne[1];
    if (b->ne[0] != k || (b->ne[1] != 1 && b->ne[1] != n_used) || b->ne[2] != T || b->ne[3] != 1 || ids->ne[2] != 1 ||
        ids->ne[3] != 1 || dst->ne[0] != n || dst->ne[1] != n_used || dst->ne[2] != T || dst->ne[3] != 1)
        return set_error(MQ_EINVAL, "mq_op_mul_mat_id: shapes (b [k, 1|n_used, T], ids [n_used, T], dst [n, n_used, T])");
    if (b->nb[0] != 4 || dst->nb[0] != 4 || ids->nb[0] != 4 || b->nb[1] % 16 || b->nb[2] % 16 || dst->nb[1] % 4 ||
        dst->nb[2] % 4 || ((uintptr_t)b->data & 15))
        return set_error(MQ_EINVAL, "mq_op_mul_mat_id: rows must be contiguous (b rows 16-byte aligned)");
    const int64_t R = n_used * T;
    const MoeWs w = moe_ws(type, n, k, R);
    if (((uintptr_t)workspace & 255) || workspace_bytes < w.total)
        return set_error(MQ_EINVAL, "mq_op_mul_mat_id: workspace of %zu bytes (256-byte aligned) needed, %zu given",
                         w.total, workspace_bytes);
    hipStream_t s = (hipStream_t)stream;
    // the routing, read back once
    const size_t span = (size_t)(T - 1) * ids->nb[1] + (size_t)n_used * 4;
    std::vector<char> ih(span);
    if (hipMemcpyAsync(ih.data(), ids->data, span, hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return set_error(MQ_EHIP, "mq_op_mul_mat_id: reading the expert ids failed");
    std::vector<int64_t> cnt(n_exp + 1, 0);
    for (int64_t t = 0; t < T; t++)
        for (int64_t i = 0; i < n_used; i++) {
            const int32_t e = *(const int32_t *)(ih.data() + t * ids->nb[1] + i * 4);
            if (e < 0 || e >= n_exp)
                return set_error(MQ_EINVAL, "mq_op_mul_mat_id: expert id %d of slot %lld, token %lld outside [0, %d)", e,
                                 (long long)i, (long long)t, n_exp);
            cnt[e + 1]++;
        }
    for (int e = 0; e < n_exp; e++) cnt[e + 1] += cnt[e];  // row ranges of the experts
    std::vector<int64_t> offs(2 * R), fill(cnt.begin(), cnt.end() - 1);
    for (int64_t t = 0; t < T; t++)
        for (int64_t i = 0; i < n_used; i++) {
            const int32_t e = *(const int32_t *)(ih.data() + t * ids->nb[1] + i * 4);
            const int64_t r = fill[e]++;
            offs[r] = (int64_t)((i % b->ne[1]) * b->nb[1] + t * b->nb[2]);
            offs[R + r] = (int64_t)(i * dst->nb[1] + t * dst->nb[2]);
        }
    char *ws = (char *)workspace;
    if (hipMemcpyAsync(ws + w.src_off, offs.data(), (size_t)R * 8, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipMemcpyAsync(ws + w.dst_off, offs.data() + R, (size_t)R * 8, hipMemcpyHostToDevice, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)  // the host lists go out of scope on return
        return set_error(MQ_EHIP, "mq_op_mul_mat_id: uploading the row lists failed");
    float *X = (float *)(ws + w.x), *Y = (float *)(ws + w.y);
    hipLaunchKernelGGL(k_gather_rows, dim3((unsigned)R), dim3(256), 0, s, (const char *)b->data,
                       (const int64_t *)(ws + w.src_off), X, k);
    for (int e = 0; e < n_exp; e++) {
        const int64_t r0 = cnt[e], m = cnt[e + 1] - cnt[e];
        if (m == 0) continue;
        const void *img = (const char *)expert_images + (size_t)e * expert_stride;
        const int path = mq_mul_mat_path(type, n, k, m);
        int rc = mq_quantize_act_ex(type, X + r0 * k, k, m, k, nullptr, MQ_PRE_NONE, ws + w.q, workspace_bytes - w.q,
                                    path, stream);
        if (rc == 0) rc = mq_mul_mat_q_ex(type, img, n, k, ws + w.q, m, Y + r0 * n, n, nullptr, path, stream);
        if (rc != 0) return rc;
    }
    hipLaunchKernelGGL(k_scatter_rows, dim3((unsigned)R), dim3(256), 0, s, Y, (const int64_t *)(ws + w.dst_off),
                       (char *)dst->data, n);
    return hip_rc(hipGetLastError(), "mul_mat_id");
}

// workspace of the device-routed mixture-of-experts mat-mul: the sorted rows (rmax: every
// expert's segment padded to whole tiles), their results, the two offset lists, the tile table
// and the activation quantization of the sorted rows (tiled)
struct MoeDevWs {
    int tile;
    int64_t rmax;
    size_t x, y, src_off, dst_off, tiles, q, total;
};
static MoeDevWs moe_dev_ws(int type, int n_exp, int64_t n, int64_t k, int64_t rows) {
    MoeDevWs w;
    w.tile = gemm_moe_tile_rows(rows, n, (int)std::min<int64_t>(n_exp, rows));
    w.rmax = pad_up(rows + std::min<int64_t>(n_exp, rows) * (w.tile - 1), w.tile);
    size_t o = 0;
    auto take = [&](size_t b) {
        const size_t at = o;
        o = align256(o + b);
        return at;
    };
    w.x = take((size_t)w.rmax * k * 4);
    w.y = take((size_t)w.rmax * n * 4);
    w.src_off = take((size_t)w.rmax * 8);
    w.dst_off = take((size_t)w.rmax * 8);
    w.tiles = take((size_t)(1 + w.rmax / w.tile) * 4);
    w.q = take(mq_workspace_bytes(type, w.rmax, k));
    w.total = o;
    return w;
}

extern "C" size_t mq_op_mul_mat_id_device_workspace_bytes(int type, int n_exp, int64_t n, int64_t k, int64_t rows) {
    if (n <= 0 || k <= 0 || rows <= 0 || n_exp <= 0 || mq_row_size(type, k) == 0) return 0;
    return moe_dev_ws(type, n_exp, n, k, rows).total;
}

extern "C" int mq_op_mul_mat_id_device(int type, const void *expert_images, size_t expert_stride, int n_exp, int64_t n,
                                       int64_t k, const mq_view *b, const mq_view *ids, const mq_view *dst,
                                       void *workspace, size_t workspace_bytes, void *stream) {
    if (!expert_images || n_exp <= 0 || !b || !ids || !dst || !b->data || !ids->data || !dst->data || !workspace)
        return set_error(MQ_EINVAL, "mq_op_mul_mat_id_device: missing operand");
    if (!mq_supports(type, k) || n <= 0 || n > INT32_MAX || (expert_stride % 256) != 0 ||
        ((uintptr_t)expert_images & 255) != 0 || n_exp > MOE_MAX_EXPERTS)
        return set_error(MQ_EUNSUPPORTED, "mq_op_mul_mat_id_device: weight type %d with k %lld, %d experts", type,
                         (long long)k, n_exp);
    if (!shape_ok(b) || !shape_ok(ids) || !shape_ok(dst) || b->type != MQ_TYPE_F32 || ids->type != MQ_TYPE_I32 ||
        dst->type != MQ_TYPE_F32)
        return set_error(MQ_EINVAL, "mq_op_mul_mat_id_device: types (F32 b and dst, I32 ids)");
    const int64_t n_used = ids->ne[0], T = ids->ne[1];
    if (b->ne[0] != k || (b->ne[1] != 1 && b->ne[1] != n_used) || b->ne[2] != T || b->ne[3] != 1 || ids->ne[2] != 1 ||
        ids->ne[3] != 1 || dst->ne[0] != n || dst->ne[1] != n_used || dst->ne[2] != T || dst->ne[3] != 1)
        return set_error(MQ_EINVAL,
                         "mq_op_mul_mat_id_device: shapes (b [k, 1|n_used, T], ids [n_used, T], dst [n, n_used, T])");
    if (b->nb[0] != 4 || dst->nb[0] != 4 || ids->nb[0] != 4 || b->nb[1] % 16 || b->nb[2] % 16 || dst->nb[1] % 4 ||
        dst->nb[2] % 4 || ((uintptr_t)b->data & 15) || ids->nb[1] % 4)
        return set_error(MQ_EINVAL, "mq_op_mul_mat_id_device: rows must be contiguous (b rows 16-byte aligned)");
    const int64_t R = n_used * T;
    if (R == 0) return MQ_OK;
    const MoeDevWs w = moe_dev_ws(type, n_exp, n, k, R);
    if (w.rmax > INT32_MAX)
        return set_error(MQ_EUNSUPPORTED, "mq_op_mul_mat_id_device: %lld routed rows", (long long)w.rmax);
    if (((uintptr_t)workspace & 255) || workspace_bytes < w.total)
        return set_error(MQ_EINVAL, "mq_op_mul_mat_id_device: workspace of %zu bytes (256-byte aligned) needed, %zu given",
                         w.total, workspace_bytes);
    hipStream_t s = (hipStream_t)stream;
    char *ws = (char *)workspace;
    int64_t *src_off = (int64_t *)(ws + w.src_off), *dst_off = (int64_t *)(ws + w.dst_off);
    int *tiles = (int *)(ws + w.tiles);
    float *X = (float *)(ws + w.x), *Y = (float *)(ws + w.y);
    hipLaunchKernelGGL(k_moe_route, dim3(1), dim3(1024), 0, s, (const char *)ids->data, (int64_t)ids->nb[1], (int)n_used,
                       T, n_exp, b->ne[1], (int64_t)b->nb[1], (int64_t)b->nb[2], (int64_t)dst->nb[1],
                       (int64_t)dst->nb[2], w.tile, w.rmax, src_off, dst_off, tiles, (char *)dst->data, n);
    hipLaunchKernelGGL(k_gather_rows_pad, dim3((unsigned)w.rmax), dim3(256), 0, s, (const char *)b->data, src_off, X, k);
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return hip_rc(e, "mul_mat_id routing");
    int rc = mq_quantize_act_ex(type, X, k, w.rmax, k, nullptr, MQ_PRE_NONE, ws + w.q, workspace_bytes - w.q,
                                MQ_PATH_GEMM, stream);
    if (rc != 0) return rc;
    if ((rc = hip_rc(launch_gemm_moe(type, expert_images, expert_stride, n, k, ws + w.q, w.rmax, w.tile, tiles, Y, s),
                     "mul_mat_id gemm")))
        return rc;
    hipLaunchKernelGGL(k_scatter_rows_pad, dim3((unsigned)w.rmax), dim3(256), 0, s, Y, dst_off, (char *)dst->data, n);
    return hip_rc(hipGetLastError(), "mul_mat_id");
}

extern "C" int mq_op_soft_max(const mq_view *x, const mq_view *mask, const mq_view *dst, float scale, void *stream) {
    if (const char *e = check_soft_max(x, mask, dst)) return fail(e);
    if (!have_data({x, mask, dst})) return fail("missing data pointer");
    const int64_t rows = x->ne[1] * x->ne[2] * x->ne[3];
    const dim3 g((unsigned)((rows + 3) / 4)), b(256);
    hipStream_t s = (hipStream_t)stream;
    DV mv{};
    if (mask) mv = dv(mask);
    if (!mask) hipLaunchKernelGGL(k_soft_max<0>, g, b, 0, s, dv(x), mv, dv(dst), scale, rows);
    else if (mask->type == MQ_TYPE_F16) hipLaunchKernelGGL(k_soft_max<1>, g, b, 0, s, dv(x), mv, dv(dst), scale, rows);
    else hipLaunchKernelGGL(k_soft_max<2>, g, b, 0, s, dv(x), mv, dv(dst), scale, rows);
    return hip_rc(hipGetLastError(), "soft_max");
}

extern "C" int mq_op_argsort(const mq_view *x, const mq_view *dst, int order, void *stream) {
    if (const char *e = check_argsort(order, x, dst)) return fail(e);
    if (!have_data({x, dst})) return fail("missing data pointer");
    const int64_t rows = x->ne[1] * x->ne[2] * x->ne[3];
    hipStream_t s = (hipStream_t)stream;
    if (order == MQ_SORT_DESC) hipLaunchKernelGGL(k_argsort<true>, dim3((unsigned)rows), dim3(256), 0, s, dv(x), dv(dst), rows);
    else hipLaunchKernelGGL(k_argsort<false>, dim3((unsigned)rows), dim3(256), 0, s, dv(x), dv(dst), rows);
    return hip_rc(hipGetLastError(), "argsort");
}

extern "C" int mq_op_repeat(const mq_view *src, const mq_view *dst, void *stream) {
    if (const char *e = check_repeat(src, dst)) return fail(e);
    if (!have_data({src, dst})) return fail("missing data pointer");
    const int64_t n = nel(dst);
    hipLaunchKernelGGL(k_repeat, dim3(grid_units(n)), dim3(256), 0, (hipStream_t)stream, dv(src), dv(dst), n);
    return hip_rc(hipGetLastError(), "repeat");
}

extern "C" int mq_op_mul_mat_f32(const mq_view *a, const mq_view *b, const mq_view *dst, void *stream) {
    if (const char *e = check_mul_mat_f32(a, b, dst)) return fail(e);
    if (!have_data({a, b, dst})) return fail("missing data pointer");
    const int64_t n = nel(dst);
    hipLaunchKernelGGL(k_mul_mat_f32, dim3(grid_units(n)), dim3(256), 0, (hipStream_t)stream, dv(a), dv(b), dv(dst), n);
    return hip_rc(hipGetLastError(), "mul_mat_f32");
}

extern "C" size_t mq_op_flash_attn_workspace_bytes(const mq_view *k) {
    if (!k || (k->ne[0] != 32 && k->ne[0] != 64 && k->ne[0] != 128) || k->ne[1] < 1 || k->ne[2] < 1 || k->ne[3] < 1)
        return 0;
    return attn_workspace_bytes((int)k->ne[3], (int)k->ne[1], (int)k->ne[2], (int)k->ne[0]);
}

// qk (optional): the per-head RMS norm x weight and NEOX rotation of q and k applied as the
// attention reads them (q_w / k_w: head_dim floats; cs: (cos, sin) x mscale of position t and
// pair j at cs[2 (t head_dim / 2 + j)], t over the Tq = Tk positions).
struct QkNormRope {
    const float *q_w, *k_w, *cs;
    float eps;
};

// The attention's view of operands q / k / mask (shape fields and the mask's addressing only):
// what attn_split_form and the mask block lists look at.
static AttnArgs attn_shape(const mq_view *q, const mq_view *k, const mq_view *mask) {
    AttnArgs a;
    a.B = (int)q->ne[3], a.Tq = (int)q->ne[1], a.Tk = (int)k->ne[1];
    a.nq = (int)q->ne[2], a.nkv = (int)k->ne[2], a.hd = (int)q->ne[0];
    if (mask) {
        a.mask = (const uint16_t *)mask->data;
        a.m_sq = mask->nb[1] / 2;
        a.m_sh = mask->ne[2] == 1 ? 0 : mask->nb[2] / 2;
        a.m_sb = mask->ne[3] == 1 ? 0 : mask->nb[3] / 2;
        a.m_al = (uintptr_t)mask->data % 16 == 0 && a.m_sq % 8 == 0 && a.m_sh % 8 == 0 && a.m_sb % 8 == 0;
        if (!a.mask) a.mask = (const uint16_t *)(uintptr_t)16;  // before allocation: a mask all the same
    }
    return a;
}

// operands whose attention reads mask block lists: the split-key form with a mask shared by
// every head
static bool takes_mask_blocks(const mq_view *q, const mq_view *k, const mq_view *mask) {
    if (!q || !k || !mask || !shape_ok(q) || !shape_ok(k) || !shape_ok(mask) || mask->type != MQ_TYPE_F16 ||
        mask->ne[2] != 1 || mask->ne[1] < q->ne[1] || mask->ne[0] < k->ne[1] || q->ne[1] > INT32_MAX ||
        k->ne[1] > INT32_MAX)
        return false;
    const AttnArgs a = attn_shape(q, k, mask);
    return (a.hd == 32 || a.hd == 64 || a.hd == 128) && attn_split_form(a);
}

extern "C" size_t mq_op_mask_blocks_bytes(const mq_view *q, const mq_view *k, const mq_view *mask) {
    if (!takes_mask_blocks(q, k, mask)) return 0;
    return mask_blocks_bytes(mask->ne[3] == 1 ? 1 : (int)q->ne[3], (int)q->ne[1], (int)k->ne[1]);
}

extern "C" int mq_op_mask_blocks(const mq_view *q, const mq_view *k, const mq_view *mask, void *blocks,
                                 size_t blocks_bytes, void *stream) {
    const size_t need = mq_op_mask_blocks_bytes(q, k, mask);
    if (need == 0) return fail("mask_blocks: these operands' attention takes no block lists");
    if (!have_data({q, k, mask}) || !blocks) return fail("missing data pointer");
    if (((uintptr_t)blocks & 3) || blocks_bytes < need)
        return set_error(MQ_EINVAL, "mq_op_mask_blocks: %zu bytes (4-byte aligned) needed, %zu given", need,
                         blocks_bytes);
    const AttnArgs a = attn_shape(q, k, mask);
    return hip_rc(launch_mask_blocks(a.mask, a.m_sq, a.m_sb, a.m_al, mask->ne[3] == 1 ? 1 : a.B, a.Tq, a.Tk,
                                     (uint32_t *)blocks, (hipStream_t)stream),
                  "mask_blocks");
}

extern "C" size_t mq_op_mask_segments_bytes(const mq_view *q, const mq_view *k, const mq_view *mask) {
    if (!q || !k || !mask || !shape_ok(q) || !shape_ok(k) || !shape_ok(mask) || mask->type != MQ_TYPE_F16 ||
        mask->ne[2] != 1 || mask->ne[3] != 1 || q->ne[3] != 1 || q->ne[1] != k->ne[1] || mask->ne[1] < q->ne[1] ||
        mask->ne[0] < k->ne[1] || q->ne[1] > INT32_MAX || mask->nb[0] != 2 || mask->nb[1] % 2)
        return 0;
    return (size_t)q->ne[1] * sizeof(int32_t);
}

extern "C" int mq_op_mask_segments(const mq_view *q, const mq_view *k, const mq_view *mask, void *scratch,
                                   size_t scratch_bytes, int64_t *seg_len, void *stream) {
    if (!seg_len) return fail("mask_segments: seg_len required");
    *seg_len = 0;
    const size_t need = mq_op_mask_segments_bytes(q, k, mask);
    if (need == 0) return fail("mask_segments: one F16 mask [>= T, >= T] over q and k of T positions and one batch");
    if (!have_data({q, k, mask}) || !scratch) return fail("missing data pointer");
    if (((uintptr_t)scratch & 3) || scratch_bytes < need)
        return set_error(MQ_EINVAL, "mq_op_mask_segments: %zu bytes (4-byte aligned) of scratch needed", need);
    const int T = (int)q->ne[1];
    const int64_t m_sq = mask->nb[1] / 2;
    const bool m_al = (uintptr_t)mask->data % 16 == 0 && m_sq % 8 == 0;
    hipStream_t s = (hipStream_t)stream;
    std::vector<int32_t> first(T);
    int rc = hip_rc(launch_mask_rows((const uint16_t *)mask->data, m_sq, m_al, T, (int32_t *)scratch, s), "mask_rows");
    if (rc != 0) return rc;
    if (hipMemcpyAsync(first.data(), scratch, need, hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return set_error(MQ_EHIP, "mq_op_mask_segments: reading the row summary back failed");
    // segments of S rows: row r's run starts at its segment's first row
    int64_t S = T;
    for (int r = 1; r < T; r++)
        if (first[r] != 0) {
            S = r;
            break;
        }
    if (T % S != 0) return 0;
    for (int r = 0; r < T; r++)
        if (first[r] != (int32_t)(r / S * S)) return 0;
    *seg_len = S;
    return 0;
}

extern "C" int mq_op_mask_is_zero(const mq_view *q, const mq_view *k, const mq_view *mask, void *scratch,
                                  size_t scratch_bytes, int *is_zero, void *stream) {
    if (!is_zero) return fail("mask_is_zero: is_zero required");
    *is_zero = 0;
    if (!q || !k || !mask || !shape_ok(q) || !shape_ok(k) || !shape_ok(mask) || mask->type != MQ_TYPE_F16 ||
        mask->ne[1] < q->ne[1] || mask->ne[0] < k->ne[1] || q->ne[1] > INT32_MAX || k->ne[1] > INT32_MAX ||
        mask->nb[0] != 2 || mask->nb[1] % 2 || mask->nb[2] % 2 || mask->nb[3] % 2 || mask->ne[2] * mask->ne[3] > 65535)
        return fail("mask_is_zero: an F16 mask [>= Tk, >= Tq, ...] over q and k");
    if (!have_data({q, k, mask}) || !scratch) return fail("missing data pointer");
    if (((uintptr_t)scratch & 3) || scratch_bytes < sizeof(int))
        return set_error(MQ_EINVAL, "mq_op_mask_is_zero: 4 bytes (4-byte aligned) of scratch needed");
    hipStream_t s = (hipStream_t)stream;
    int nz = 0;
    if (hipMemsetAsync(scratch, 0, sizeof(int), s) != hipSuccess) return set_error(MQ_EHIP, "mq_op_mask_is_zero: memset");
    int rc = hip_rc(launch_mask_nonzero((const uint16_t *)mask->data, (int64_t)(mask->nb[1] / 2), (int64_t)(mask->nb[2] / 2),
                                        (int64_t)(mask->nb[3] / 2), (int)mask->ne[2], (int)mask->ne[3], (int)q->ne[1],
                                        (int)k->ne[1], (int *)scratch, s),
                    "mask_nonzero");
    if (rc != 0) return rc;
    if (hipMemcpyAsync(&nz, scratch, sizeof(int), hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return set_error(MQ_EHIP, "mq_op_mask_is_zero: reading the flag back failed");
    *is_zero = nz == 0;
    return 0;
}

static int flash_attn(const mq_view *q, const mq_view *k, const mq_view *v, const mq_view *mask, const mq_view *dst,
                      float scale, void *workspace, size_t workspace_bytes, void *act_ws, size_t act_ws_bytes,
                      int flags, void *stream, const QkNormRope *qk = nullptr, const void *blocks = nullptr,
                      int64_t causal_seg = 0, int act_type = MQ_TYPE_Q8_0) {
    if (const char *e = check_flash(q, k, v, mask, dst)) return fail(e);
    if (!have_data({q, k, v, mask, dst})) return fail("missing data pointer");
    if (qk) {
        if (!qk->q_w || !qk->k_w || !qk->cs) return fail("flash_attn_qk_norm_rope: missing data pointer");
        if (flags & MQ_ATTN_KV_READY) return fail("flash_attn_qk_norm_rope: K/V fragments computed elsewhere");
        if (q->ne[1] != k->ne[1]) return fail("flash_attn_qk_norm_rope: q and k must share the positions (Tq = Tk)");
    }
    const size_t need = mq_op_flash_attn_workspace_bytes(k);
    if (!workspace || ((uintptr_t)workspace & 15) != 0 || workspace_bytes < need)
        return set_error(MQ_EINVAL, "mq_op_flash_attn: workspace of %zu bytes (16-byte aligned) needed, %zu given",
                         need, workspace_bytes);
    AttnArgs a;
    a.q = (const float *)q->data, a.k = (const float *)k->data, a.v = (const float *)v->data;
    a.out = (float *)dst->data;
    a.q_st = q->nb[1] / 4, a.q_sh = q->nb[2] / 4, a.q_sb = q->nb[3] / 4;
    a.k_st = k->nb[1] / 4, a.k_sh = k->nb[2] / 4, a.k_sb = k->nb[3] / 4;
    a.v_st = v->nb[1] / 4, a.v_sh = v->nb[2] / 4, a.v_sb = v->nb[3] / 4;
    a.o_sh = dst->nb[1] / 4, a.o_st = dst->nb[2] / 4, a.o_sb = dst->nb[3] / 4;
    if (mask) {
        a.mask = (const uint16_t *)mask->data;
        a.m_sq = mask->nb[1] / 2;
        a.m_sh = mask->ne[2] == 1 ? 0 : mask->nb[2] / 2;
        a.m_sb = mask->ne[3] == 1 ? 0 : mask->nb[3] / 2;
        a.m_al = (uintptr_t)mask->data % 16 == 0 && a.m_sq % 8 == 0 && a.m_sh % 8 == 0 && a.m_sb % 8 == 0;
    }
    a.B = (int)q->ne[3], a.Tq = (int)q->ne[1], a.Tk = (int)k->ne[1];
    a.nq = (int)q->ne[2], a.nkv = (int)k->ne[2], a.hd = (int)q->ne[0];
    if (causal_seg > 0) {  // the mask is block-diagonal causal (mq_op_mask_segments): per-segment causal attention
        const int64_t S = causal_seg, T = q->ne[1];
        if (!mask || k->ne[1] != T || T % S != 0 || S % 32 != 0 || q->ne[3] != 1 || S > INT32_MAX)
            return fail("flash_attn: causal segments need a mask, Tq = Tk = a multiple of the segment (a multiple "
                        "of 32) and one batch");
        a.B = (int)(T / S), a.Tq = a.Tk = (int)S;
        a.q_sb = S * a.q_st, a.k_sb = S * a.k_st, a.v_sb = S * a.v_st, a.o_sb = S * a.o_st;
        a.mask = nullptr, a.m_sq = a.m_sh = a.m_sb = 0, a.m_al = false;
        a.causal = 1;
        blocks = nullptr;
    }
    if (blocks) {  // lists from mq_op_mask_blocks of these operands; ignored by the other forms
        if (!mask || !takes_mask_blocks(q, k, mask)) blocks = nullptr;
        if ((uintptr_t)blocks & 3) return fail("flash_attn: mask block lists not 4-byte aligned");
        a.blist = (const uint32_t *)blocks;
        a.bl_nqt = (a.Tq + 31) / 32;
        a.bl_stride = (a.Tk + 31) / 32 + 1;
    }
    a.scale = scale;
    a.ws = workspace;
    a.kv_ready = (flags & MQ_ATTN_KV_READY) != 0;
    if (qk) a.qw = qk->q_w, a.kw = qk->k_w, a.eps = qk->eps, a.cs = (const float2 *)qk->cs;
    if (qk && causal_seg > 0) a.cs_sb = causal_seg * (q->ne[0] / 2);  // the table holds every row's angles
    if (act_ws) {
        const int64_t K = dst->ne[0] * dst->ne[1], rows = dst->ne[2] * dst->ne[3];
        if (act_type != MQ_TYPE_Q8_0 && act_type != MQ_TYPE_Q4_K && act_type != MQ_TYPE_Q6_K)
            return fail("flash_attn: the quantized output is for a Q8_0, Q4_K or Q6_K projection");
        if (K % (act_type == MQ_TYPE_Q8_0 ? 128 : 256) != 0 || dst->nb[1] != (size_t)dst->ne[0] * 4 ||
            dst->nb[2] != (size_t)K * 4 || dst->nb[3] != dst->nb[2] * (size_t)dst->ne[2])
            return fail("flash_attn: a quantized output needs dst as dense rows of n_head * head_dim floats, a "
                        "multiple of 128 (Q8_0) or 256 (K-quants)");
        if (((uintptr_t)act_ws & 255) || act_ws_bytes < act_planes(act_type, rows, K, true).total)
            return set_error(MQ_EINVAL, "mq_op_flash_attn: activation workspace (256-byte aligned) too small");
        a.q_ws = act_ws;
        a.q_type = act_type;
        a.q_var = mq_q8_0_variant();
    }
    return hip_rc(launch_attn(a, (hipStream_t)stream), "flash_attn");
}

extern "C" int mq_op_flash_attn(const mq_view *q, const mq_view *k, const mq_view *v, const mq_view *mask,
                                const mq_view *dst, float scale, void *workspace, size_t workspace_bytes,
                                void *stream) {
    return flash_attn(q, k, v, mask, dst, scale, workspace, workspace_bytes, nullptr, 0, 0, stream);
}

extern "C" int mq_op_flash_attn_q8_0(const mq_view *q, const mq_view *k, const mq_view *v, const mq_view *mask,
                                     const mq_view *dst, float scale, void *workspace, size_t workspace_bytes,
                                     void *act_workspace, size_t act_workspace_bytes, void *stream) {
    if (!act_workspace) return set_error(MQ_EINVAL, "mq_op_flash_attn_q8_0: no activation workspace");
    return flash_attn(q, k, v, mask, dst, scale, workspace, workspace_bytes, act_workspace, act_workspace_bytes, 0,
                      stream);
}

extern "C" int mq_op_flash_attn_ex(const mq_view *q, const mq_view *k, const mq_view *v, const mq_view *mask,
                                   const mq_view *dst, float scale, void *workspace, size_t workspace_bytes,
                                   void *act_workspace, size_t act_workspace_bytes, int flags, void *stream) {
    if (flags & ~MQ_ATTN_KV_READY) return set_error(MQ_EINVAL, "mq_op_flash_attn_ex: unknown flags");
    return flash_attn(q, k, v, mask, dst, scale, workspace, workspace_bytes, act_workspace, act_workspace_bytes, flags,
                      stream);
}

extern "C" int mq_op_flash_attn_qk_norm_rope(const mq_view *q, const mq_view *k, const mq_view *v,
                                             const mq_view *mask, const mq_view *dst, float scale, const float *q_norm_w,
                                             const float *k_norm_w, float eps, const float *cs, void *workspace,
                                             size_t workspace_bytes, void *act_workspace, size_t act_workspace_bytes,
                                             void *stream) {
    const QkNormRope qk{q_norm_w, k_norm_w, cs, eps};
    return flash_attn(q, k, v, mask, dst, scale, workspace, workspace_bytes, act_workspace, act_workspace_bytes, 0,
                      stream, &qk);
}

extern "C" int mq_op_flash_attn_blocks(const mq_view *q, const mq_view *k, const mq_view *v, const mq_view *mask,
                                       const mq_view *dst, float scale, const float *q_norm_w, const float *k_norm_w,
                                       float eps, const float *cs, const void *mask_blocks, int64_t causal_segment,
                                       void *workspace, size_t workspace_bytes, void *act_workspace,
                                       size_t act_workspace_bytes, int act_type, int flags, void *stream) {
    if (flags & ~MQ_ATTN_KV_READY) return set_error(MQ_EINVAL, "mq_op_flash_attn_blocks: unknown flags");
    const bool norm = q_norm_w || k_norm_w || cs;
    if (norm && !(q_norm_w && k_norm_w && cs))
        return fail("flash_attn_blocks: q_norm_w, k_norm_w and cs go together");
    if (mask_blocks && !mask) return fail("flash_attn_blocks: block lists without a mask");
    if (causal_segment < 0) return fail("flash_attn_blocks: negative causal segment");
    if (norm && (flags & MQ_ATTN_KV_READY)) return fail("flash_attn_blocks: K/V fragments computed elsewhere");
    const QkNormRope qk{q_norm_w, k_norm_w, cs, eps};
    return flash_attn(q, k, v, mask, dst, scale, workspace, workspace_bytes, act_workspace, act_workspace_bytes, flags,
                      stream, norm ? &qk : nullptr, mask_blocks, causal_segment, act_type);
}

extern "C" int mq_op_rope_cache(const mq_view *pos, const mq_view *freq_factors, int n_dims, int n_ctx_orig,
                                float freq_base, float freq_scale, float ext_factor, float attn_factor,
                                float beta_fast, float beta_slow, float *cs, void *stream) {
    if (!pos || !shape_ok(pos) || pos->type != MQ_TYPE_I32 || pos->ne[1] != 1 || pos->ne[2] != 1 || pos->ne[3] != 1)
        return fail("rope_cache: pos must be I32 [T]");
    if (n_dims <= 0 || n_dims % 2 || n_dims > 128) return fail("rope_cache: n_dims must be even, at most 128");
    const mq_view *ff = freq_factors;
    if (ff && (!shape_ok(ff) || ff->type != MQ_TYPE_F32 || ff->nb[0] != 4 || ff->ne[0] < n_dims / 2))
        return fail("rope_cache: freq_factors must be F32 [n_dims/2]");
    if (!have_data({pos, ff}) || !cs) return fail("missing data pointer");
    if (pos->ne[0] > INT32_MAX) return fail("rope_cache: too many positions");
    const RopeParams rp = rope_params(n_dims, MQ_ROPE_NEOX, n_ctx_orig, freq_base, freq_scale, ext_factor,
                                      attn_factor, beta_fast, beta_slow);
    hipLaunchKernelGGL(k_rope_cache, dim3((unsigned)pos->ne[0]), dim3(64), 0, (hipStream_t)stream, dv(pos),
                       ff ? (const float *)ff->data : nullptr, rp, (float2 *)cs);
    return hip_rc(hipGetLastError(), "rope_cache");
}

extern "C" int mq_op_supported(int op, int sub, const mq_view *s0, const mq_view *s1, const mq_view *s2,
                               const mq_view *s3, const mq_view *dst) {
    const char *e = "unknown op";
    switch (op) {
        case MQ_OP_GET_ROWS: e = check_get_rows(s0, s1, dst); break;
        case MQ_OP_BINARY: e = check_binary(sub, s0, s1, dst); break;
        case MQ_OP_UNARY: e = check_unary(sub, s0, dst); break;
        case MQ_OP_NORM: e = check_norm(sub, s0, s1, dst); break;
        case MQ_OP_CPY: e = check_cpy(s0, dst); break;
        case MQ_OP_FLASH_ATTN: e = check_flash(s0, s1, s2, s3, dst); break;
        case MQ_OP_ROPE: e = s0 ? check_rope(sub, s0, s1, s2, dst, (int)s0->ne[0]) : "missing or empty operand"; break;
        case MQ_OP_SOFT_MAX: e = check_soft_max(s0, s1, dst); break;
        case MQ_OP_ARGSORT: e = check_argsort(sub, s0, dst); break;
        case MQ_OP_REPEAT: e = check_repeat(s0, dst); break;
        case MQ_OP_MUL_MAT_F32: e = check_mul_mat_f32(s0, s1, dst); break;
        default: break;
    }
    return e == nullptr;
}
