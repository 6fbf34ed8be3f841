// mq_decoder.hip -- the non-MUL_MAT ops of a decoder-style embedder (Qwen3 family) on gfx950.
//
// CrispEmbed's decoder graph (src/decoder_embed.cpp:565-830) around the mul_mats:
//   embedding   GET_ROWS(token_embd)
//   norms       RMS_NORM(eps) * w before attention and before the FFN; the residual ADD
//               that produces the norm's input is fused in front of it
//   q / k       per-head RMS_NORM * q_norm / k_norm, then ROPE_EXT in NEOX mode (pair
//               (i, i + d/2) rotated by pos * base^(-2i/d), positions 0..T-1 per sequence)
//   attention   FLASH_ATTN_EXT, scale 1/sqrt(head_dim), causal mask (0 / -inf), grouped
//               query heads (head h reads key/value head h / (n_head / n_kv_head))
//   FFN         silu(gate) * up -- applied by the FFN-down activation quantizer
//   pooling     output RMS_NORM of the last token (or of every token, then the mean), L2
//               normalised with sqrtf(max(sum x^2, 1e-12)) (src/decoder_embed.cpp:1044-1100)
// Arithmetic is fp32 throughout; the attention's products run on fp16 MFMAs over split
// (hi + lo) operands, which keeps fp32 accuracy.
#include "mq_internal.h"
#include "mq_wave.h"

namespace mq {

typedef float v16f __attribute__((ext_vector_type(16)));

// One wave per row (V values per lane, rows up to 64*V wide):
//   x = ids ? tok[ids[row]] : y + res      (GET_ROWS, or the residual ADD; res may be NULL)
//   xout = x (if non-NULL; may alias res), hout = x / sqrt(mean(x^2) + eps) * w
template <int V>
__global__ __launch_bounds__(256) void k_add_rmsnorm(const float *y, const float *res, const int32_t *__restrict__ ids,
                                                     const float *__restrict__ tok, const float *__restrict__ w,
                                                     float eps, float *xout, float *__restrict__ hout, int64_t rows,
                                                     int H, int n_vocab) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    // ids outside the table are clamped: a bad id reads a valid row, never out of bounds
    const float *src = ids ? tok + (int64_t)min(max(ids[row], 0), n_vocab - 1) * H : y + row * H;
    float v[V];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int c = lane + 64 * i;
        v[i] = 0.f;
        if (c < H) {
            v[i] = src[c];
            if (!ids && res) v[i] += res[row * H + c];
        }
        ss += v[i] * v[i];
    }
    if (xout) {
#pragma unroll
        for (int i = 0; i < V; i++)
            if (lane + 64 * i < H) xout[row * H + lane + 64 * i] = v[i];
    }
    const float scale = 1.0f / sqrtf(wave_sum_f(ss) / (float)H + eps);
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int c = lane + 64 * i;
        if (c < H) hout[row * H + c] = v[i] * scale * w[c];
    }
}

// RoPE angle table for positions 0..T-1: cs[p][i] = (cos, sin) of p * theta_scale^i, the
// angle built by the same repeated fp32 multiplication as ggml's rope cache.
__global__ __launch_bounds__(256) void k_rope_table(float2 *__restrict__ cs, int T, int half, float theta_scale) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= T * half) return;
    const int p = t / half, i = t - p * half;
    float theta = (float)p;
    for (int j = 0; j < i; j++) theta *= theta_scale;
    cs[t] = make_float2(cosf(theta), sinf(theta));
}

// One wave per (row, head) of Q and K inside the fused projection output qkv[rows][ld]
// (Q heads at columns h*HD for h < nq, K heads right after them).  Lane l < HD/2 holds the
// NEOX pair (l, l + HD/2): per-head RMS norm (when the weight is given), then the rotation
// by the table angle of position row % T.
template <int HD>
__global__ __launch_bounds__(256) void k_qk_norm_rope(float *qkv, int64_t ld, const float *__restrict__ qw,
                                                      const float *__restrict__ kw, float eps, int nq, int nkv, int T,
                                                      const float2 *__restrict__ cs, int64_t rows) {
    constexpr int HALF = HD / 2;
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int nh = nq + nkv;
    if (item >= rows * nh) return;
    const int64_t row = item / nh;
    const int h = (int)(item - row * nh);
    float *x = qkv + row * ld + (int64_t)h * HD;
    const float *w = h < nq ? qw : kw;
    const bool on = lane < HALF;
    float a = on ? x[lane] : 0.f, b = on ? x[lane + HALF] : 0.f;
    if (w) {
        const float scale = 1.0f / sqrtf(wave_sum_f(a * a + b * b) / (float)HD + eps);
        if (on) {
            a = a * scale * w[lane];
            b = b * scale * w[lane + HALF];
        }
    }
    if (on) {
        const float2 r = cs[(row % T) * HALF + lane];
        x[lane] = a * r.x - b * r.y;
        x[lane + HALF] = a * r.y + b * r.x;
    }
}

// Attention with fp32-accurate products on fp16 MFMAs.  Every fp32 operand x is split into
// fp16 x_hi = fp16(x) and x_lo = fp16(x - x_hi) (together ~21 significant bits), and a product
// is accumulated as hi*hi + hi*lo + lo*hi in fp32 (the dropped lo*lo term is 2^-22 relative):
// three v_mfma_f32_32x32x16_f16 per 16-deep step instead of eight fp32 32x32x2 steps.
//
// Workgroup: 4 waves x 32 queries of one (sequence, head); the K and V rows of 32 keys at a
// time are split and staged in LDS (K row-major [key][d], V transposed [d][key]; the row
// strides keep a wave's reads on distinct banks).  Per key block each wave computes
//   S^T[key][query] = sum_d K[key][d] Q[query][d]   A = K (LDS), B = Q^T (registers)
// so each lane owns one query column: 16 scores of its half of the keys, registers i holding
// keys 8(i/4) + 4 half + i%4.  After the online softmax those 16 probabilities are the A
// operands of
//   O[query][d] += sum_key P[query][key] V[key][d]  two 16-deep steps; in step t lane slot j
//                                                   is key 16t + 8(j/4) + 4 half + j%4, i.e.
//                                                   register 8t + j, and B reads those keys'
//                                                   V columns from the transposed tile.
// O's rows are queries 8(r/4) + 4 half + r%4 of register r, so the per-query rescale
// factors pass through a 32-float LDS slot per wave.  Operands below ~2^-4 in magnitude have
// their low part in the fp16 subnormal range (absolute precision 2^-24), so their relative
// precision degrades gracefully; P is scaled by 2^15 before the split to keep it exact.
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

template <int HD>
__global__ __launch_bounds__(256) void k_attn_split(const float *__restrict__ qkv, int64_t ld, float *__restrict__ out,
                                                    int64_t ldo, int T, int nq, int nkv, float scale, int causal) {
    constexpr int NS = HD / 16, NT = HD / 32;
    constexpr int KST = HD + 8;  // K tile row stride (halves): 4 banks apart per row
    constexpr int VST = 36;      // V^T tile row stride (halves): 18 dwords, odd multiple of 2
    __shared__ __attribute__((aligned(16))) _Float16 Kh[32 * KST], Kl[32 * KST];
    __shared__ __attribute__((aligned(16))) _Float16 Vh[HD * VST], Vl[HD * VST];
    __shared__ __attribute__((aligned(16))) float rs[4][32];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l32 = lane & 31, half = lane >> 5;
    const int h = blockIdx.y, hk = h / (nq / nkv);
    const int64_t rbase = (int64_t)blockIdx.z * T;  // first row of the sequence
    const int q0 = blockIdx.x * 128 + wave * 32;    // this wave's first query
    const int qi = q0 + l32;
    const int64_t qcol = (int64_t)h * HD, kcol = (int64_t)nq * HD + (int64_t)hk * HD,
                  vcol = (int64_t)(nq + nkv) * HD + (int64_t)hk * HD;

    // Q^T operand, split: step s holds Q[qi][16s + 8 half + j] * scale, j < 8
    v8h qh[NS], ql[NS];
    {
        const float *qp = qkv + (rbase + min(qi, T - 1)) * ld + qcol + 8 * half;
#pragma unroll
        for (int st = 0; st < NS; st++) {
            const float4 a = *(const float4 *)(qp + 16 * st), b = *(const float4 *)(qp + 16 * st + 4);
            const float x[8] = {a.x * scale, a.y * scale, a.z * scale, a.w * scale,
                                b.x * scale, b.y * scale, b.z * scale, b.w * scale};
            split8(x, qh[st], ql[st]);
        }
    }
    v16f oacc[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) oacc[j] = (v16f){};
    float m_run = -INFINITY, l_run = 0.f;
    const int kend = causal ? min(T, (int)blockIdx.x * 128 + 128) : T;  // keys the workgroup needs
    const int kend_w = q0 >= T ? 0 : causal ? min(T, q0 + 32) : T;      // keys this wave needs

    for (int kb = 0; kb < kend; kb += 32) {
        __syncthreads();  // the previous block's K/V are no longer read
        for (int e = threadIdx.x; e < 32 * HD / 4; e += 256) {
            const int r = e / (HD / 4), c4 = (e % (HD / 4)) * 4;
            float4 kk = make_float4(0.f, 0.f, 0.f, 0.f), vv = kk;
            if (kb + r < T) {
                kk = *(const float4 *)(qkv + (rbase + kb + r) * ld + kcol + c4);
                vv = *(const float4 *)(qkv + (rbase + kb + r) * ld + vcol + c4);
            }
            v2h k01h, k01l, k23h, k23l, v01h, v01l, v23h, v23l;
            split2(kk.x, kk.y, k01h, k01l);
            split2(kk.z, kk.w, k23h, k23l);
            split2(vv.x, vv.y, v01h, v01l);
            split2(vv.z, vv.w, v23h, v23l);
            *(v4h *)&Kh[r * KST + c4] = (v4h){k01h[0], k01h[1], k23h[0], k23h[1]};
            *(v4h *)&Kl[r * KST + c4] = (v4h){k01l[0], k01l[1], k23l[0], k23l[1]};
            Vh[(c4 + 0) * VST + r] = v01h[0], Vl[(c4 + 0) * VST + r] = v01l[0];
            Vh[(c4 + 1) * VST + r] = v01h[1], Vl[(c4 + 1) * VST + r] = v01l[1];
            Vh[(c4 + 2) * VST + r] = v23h[0], Vl[(c4 + 2) * VST + r] = v23l[0];
            Vh[(c4 + 3) * VST + r] = v23h[1], Vl[(c4 + 3) * VST + r] = v23l[1];
        }
        __syncthreads();
        if (kb >= kend_w) continue;  // past this wave's causal range (wave-uniform)

        // three accumulators, so consecutive MFMAs never chain on one accumulator while a
        // later load reuses their operand registers (the chained form gave wrong scores)
        v16f s_hh = (v16f){}, s_hl = (v16f){}, s_lh = (v16f){};
        const _Float16 *kh = &Kh[l32 * KST + 8 * half], *kl = &Kl[l32 * KST + 8 * half];
#pragma unroll
        for (int st = 0; st < NS; st++) {
            const v8h ah = *(const v8h *)(kh + 16 * st), al = *(const v8h *)(kl + 16 * st);
            s_hh = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, qh[st], s_hh, 0, 0, 0);
            s_hl = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, ql[st], s_hl, 0, 0, 0);
            s_lh = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, qh[st], s_lh, 0, 0, 0);
        }
        const v16f sc = s_hh + (s_hl + s_lh);
        float p[16], mblk = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int key = kb + 8 * (i / 4) + 4 * half + (i % 4);
            p[i] = (key >= T || (causal && key > qi)) ? -INFINITY : sc[i];
            mblk = fmaxf(mblk, p[i]);
        }
        mblk = fmaxf(mblk, __shfl_xor(mblk, 32));
        const float m_new = fmaxf(m_run, mblk);
        const float alpha = expf(m_run - m_new);  // 0 on the first block
        float lblk = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            p[i] = expf(p[i] - m_new);
            lblk += p[i];
        }
        lblk += __shfl_xor(lblk, 32);
        l_run = l_run * alpha + lblk;
        m_run = m_new;

        // rescale O's rows (queries 8(r/4) + 4 half + r%4) by their query's alpha
        rs[wave][l32] = alpha;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // one wave writes and reads its slot
        float al[16];
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const float4 t = *(const float4 *)&rs[wave][8 * g + 4 * half];
            al[4 * g] = t.x, al[4 * g + 1] = t.y, al[4 * g + 2] = t.z, al[4 * g + 3] = t.w;
        }
#pragma unroll
        for (int j = 0; j < NT; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) oacc[j][r] *= al[r];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            // P is split as 2^15 p (exact scaling; p <= 1 keeps it below the fp16 maximum) so
            // that the low part of small probabilities stays out of the fp16 subnormal range
            float px[8];
#pragma unroll
            for (int j = 0; j < 8; j++) px[j] = p[8 * t + j] * 32768.0f;
            v8h ph, pl;
            split8(px, ph, pl);
            const int k0 = 16 * t + 4 * half;  // slot j < 4: keys k0 + j; j >= 4: keys k0 + 8 + j - 4
            v8h bh[NT], bl[NT];
#pragma unroll
            for (int j = 0; j < NT; j++) {
                const int d = 32 * j + l32;
                const v4h h0 = *(const v4h *)&Vh[d * VST + k0], h1 = *(const v4h *)&Vh[d * VST + k0 + 8];
                const v4h l0 = *(const v4h *)&Vl[d * VST + k0], l1 = *(const v4h *)&Vl[d * VST + k0 + 8];
                bh[j] = (v8h){h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
                bl[j] = (v8h){l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
            }
            // term-major order: consecutive MFMAs write different accumulators
#pragma unroll
            for (int j = 0; j < NT; j++) oacc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ph, bh[j], oacc[j], 0, 0, 0);
#pragma unroll
            for (int j = 0; j < NT; j++) oacc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ph, bl[j], oacc[j], 0, 0, 0);
#pragma unroll
            for (int j = 0; j < NT; j++) oacc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pl, bh[j], oacc[j], 0, 0, 0);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slot is rewritten next block
    }

    rs[wave][l32] = 1.0f / (l_run * 32768.0f);  // O accumulated 2^15 P V
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    float inv[16];
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const float4 t = *(const float4 *)&rs[wave][8 * g + 4 * half];
        inv[4 * g] = t.x, inv[4 * g + 1] = t.y, inv[4 * g + 2] = t.z, inv[4 * g + 3] = t.w;
    }
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int q = q0 + 8 * (r / 4) + 4 * half + (r % 4);
        if (q >= T) continue;
        float *o = out + (rbase + q) * ldo + qcol + l32;
#pragma unroll
        for (int j = 0; j < NT; j++) o[32 * j] = oacc[j][r] * inv[r];
    }
}

// One wave per sequence: the last token's row, RMS-normed with w, then L2-normalised.
template <int V>
__global__ __launch_bounds__(64) void k_last_rmsnorm_l2(const float *__restrict__ x, const float *__restrict__ w,
                                                        float eps, float *__restrict__ out, int T, int H) {
    const int b = blockIdx.x, lane = threadIdx.x;
    const float *row = x + ((int64_t)b * T + T - 1) * H;
    float v[V], ss = 0.f;
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int c = lane + 64 * i;
        v[i] = c < H ? row[c] : 0.f;
        ss += v[i] * v[i];
    }
    const float scale = 1.0f / sqrtf(wave_sum_f(ss) / (float)H + eps);
    float s2 = 0.f;
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int c = lane + 64 * i;
        v[i] = c < H ? v[i] * scale * w[c] : 0.f;
        s2 += v[i] * v[i];
    }
    const float inv = 1.0f / sqrtf(fmaxf(wave_sum_f(s2), 1e-12f));
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int c = lane + 64 * i;
        if (c < H) out[(int64_t)b * H + c] = v[i] * inv;
    }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
#define MQ_RMS_DISPATCH(KERNEL, GRID, BLOCK, ...)                                           \
    do {                                                                                    \
        const int need = (H + 63) / 64;                                                     \
        if (need <= 4) hipLaunchKernelGGL((KERNEL<4>), GRID, BLOCK, 0, s, __VA_ARGS__);     \
        else if (need <= 8) hipLaunchKernelGGL((KERNEL<8>), GRID, BLOCK, 0, s, __VA_ARGS__); \
        else if (need <= 16) hipLaunchKernelGGL((KERNEL<16>), GRID, BLOCK, 0, s, __VA_ARGS__); \
        else if (need <= 32) hipLaunchKernelGGL((KERNEL<32>), GRID, BLOCK, 0, s, __VA_ARGS__); \
        else if (need <= 64) hipLaunchKernelGGL((KERNEL<64>), GRID, BLOCK, 0, s, __VA_ARGS__); \
        else return hipErrorInvalidValue;                                                   \
    } while (0)

hipError_t launch_add_rmsnorm(const float *y, const float *res, const int32_t *ids, const float *tok, int n_vocab,
                              const float *w, float eps, float *xout, float *hout, int64_t rows, int H, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    MQ_RMS_DISPATCH(k_add_rmsnorm, dim3((unsigned)((rows + 3) / 4)), dim3(256), y, res, ids, tok, w, eps, xout, hout,
                    rows, H, n_vocab);
    return hipGetLastError();
}

// cs: device scratch of T * hd/2 float2 for the angle table
hipError_t launch_qk_norm_rope(float *qkv, int64_t ld, const float *qw, const float *kw, float eps, int nq, int nkv,
                               int hd, int T, float theta_base, int64_t rows, float2 *cs, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (hd != 64 && hd != 128) return hipErrorInvalidValue;
    const float theta_scale = powf(theta_base, -2.0f / (float)hd);
    hipLaunchKernelGGL(k_rope_table, dim3((unsigned)((T * (hd / 2) + 255) / 256)), dim3(256), 0, s, cs, T, hd / 2,
                       theta_scale);
    const dim3 g((unsigned)((rows * (nq + nkv) + 3) / 4)), b(256);
    if (hd == 128) hipLaunchKernelGGL((k_qk_norm_rope<128>), g, b, 0, s, qkv, ld, qw, kw, eps, nq, nkv, T, cs, rows);
    else hipLaunchKernelGGL((k_qk_norm_rope<64>), g, b, 0, s, qkv, ld, qw, kw, eps, nq, nkv, T, cs, rows);
    return hipGetLastError();
}

hipError_t launch_attn_mfma(const float *qkv, int64_t ld, float *out, int64_t ldo, int B, int T, int nq, int nkv, int hd,
                            float scale, int causal, hipStream_t s) {
    if (B <= 0 || T <= 0) return hipSuccess;
    if (nkv <= 0 || nq % nkv != 0 || ld % 4 != 0 || ((uintptr_t)qkv & 15) != 0) return hipErrorInvalidValue;
    const dim3 g((unsigned)((T + 127) / 128), (unsigned)nq, (unsigned)B), b(256);
    if (hd == 128) hipLaunchKernelGGL((k_attn_split<128>), g, b, 0, s, qkv, ld, out, ldo, T, nq, nkv, scale, causal);
    else if (hd == 64) hipLaunchKernelGGL((k_attn_split<64>), g, b, 0, s, qkv, ld, out, ldo, T, nq, nkv, scale, causal);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_last_rmsnorm_l2(const float *x, const float *w, float eps, float *out, int B, int T, int H,
                                  hipStream_t s) {
    if (B <= 0) return hipSuccess;
    MQ_RMS_DISPATCH(k_last_rmsnorm_l2, dim3((unsigned)B), dim3(64), x, w, eps, out, T, H);
    return hipGetLastError();
}
#undef MQ_RMS_DISPATCH

}  // namespace mq
