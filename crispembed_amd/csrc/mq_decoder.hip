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
#include <atomic>
#include <climits>
#include <cstdlib>

#include "mq_internal.h"
#include "mq_act.h"
#include "mq_q8k.h"
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
// Operands below ~2^-4 in magnitude have their low part in the fp16 subnormal range (absolute
// precision 2^-24), so their relative precision degrades gracefully; P is scaled by 2^15
// before its split to keep it exact.
//
// Two kernels:
//  k_kv_frag   per (sequence, key/value head, block of 32 keys): K rows (optionally RMS-normed
//              and rotated, as for Q) and V rows, split and written as MFMA operand fragments
//              of 1 KB each (64 lanes x 8 halves, in lane order), so the attention kernel reads
//              every operand with one coalesced 16-byte load per lane and no LDS staging:
//                K fragment (st, p):    lane l holds K[32 kb + l%32][16 st + 8 (l/32) + j]
//                V fragment (t, n, p):  lane l holds V[32 kb + 16 t + 8 (j/4) + 4 (l/32) + j%4][32 n + l%32]
//              (p = hi / lo; j < 8 the lane's slot).  Each K and V element is split once,
//              instead of once per query block that reads it.
//  k_attn_frag each wave: 32 queries of one head.  Per key block
//                S^T[key][query] = sum_d K[key][d] Q[query][d]   A = K fragments, B = Q^T (registers)
//              so each lane owns one query column: 16 scores of its half of the keys, register
//              i holding key 8(i/4) + 4 half + i%4.  After the online softmax (base 2: Q carries
//              scale * log2 e) those 16 probabilities are the A operands of
//                O[query][d] += sum_key P[query][key] V[key][d]
//              in two 16-deep steps; in step t lane slot j is register 8t + j, the key the V
//              fragment (t, n) holds in that slot.  O's rows are queries 8(r/4) + 4 half + r%4 of
//              register r, so the per-query rescale factors pass through a 32-float LDS slot per
//              wave.  A workgroup is 8 waves, 2 heads x 128 queries (the two heads of a grouped-
//              query pair read the same fragments), two waves per SIMD so that one wave's
//              softmax overlaps the other's matrix work; the longest causal ranges go first.

template <int HD>
__global__ __launch_bounds__(256) void k_kv_frag(const AttnArgs a, int nblk) {
    constexpr int NS = HD / 16, NT = HD / 32, HALF = HD / 2, KS = HD + 4, NFR = kv_frags<HD>();
    __shared__ __attribute__((aligned(16))) float Ks[32 * KS];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l32 = lane & 31, half = lane >> 5;
    const int kb = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
    const float *kp = a.k + (int64_t)b * a.k_sb + (int64_t)hk * a.k_sh;
    const float *vp = a.v + (int64_t)b * a.v_sb + (int64_t)hk * a.v_sh;
    const float *kw = a.kw;
    const float2 *cs = a.cs ? a.cs + (int64_t)b * a.cs_sb : nullptr;
    const bool on = lane < HALF;
    // K rows of the block, normed and rotated (NEOX pair (i, i + HD/2) in one lane), to LDS;
    // rows past Tk are zero.  The wave's 8 rows are loaded first, all in flight at once.
    float k0[8], k1[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int key = kb * 32 + wave + 4 * i;
        const float *x = kp + (int64_t)key * a.k_st;
        k0[i] = (key < a.Tk && on) ? x[lane] : 0.f;
        k1[i] = (key < a.Tk && on) ? x[lane + HALF] : 0.f;
    }
    // and the V values of this wave's fragments (t, n): 2 NT of them, NT / 2 per wave (head_dim 32:
    // one, waves 2 and 3 idle)
    constexpr int VPW = (2 * NT + 3) / 4;
    float vx[VPW][8];
#pragma unroll
    for (int u = 0; u < VPW; u++) {
        const int f = wave + 4 * u, t = f / NT, n = f % NT;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int key = kb * 32 + 16 * t + 8 * (j / 4) + 4 * half + j % 4;
            vx[u][j] = (f < 2 * NT && key < a.Tk) ? vp[(int64_t)key * a.v_st + 32 * n + l32] : 0.f;
        }
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int r = wave + 4 * i, key = kb * 32 + r;
        float x0 = 0.f, x1 = 0.f;
        if (key < a.Tk) {
            x0 = k0[i];
            x1 = k1[i];
            if (kw) {
                const float scale = 1.0f / sqrtf(wave_sum_f(x0 * x0 + x1 * x1) / (float)HD + a.eps);
                if (on) {
                    x0 = x0 * scale * kw[lane];
                    x1 = x1 * scale * kw[lane + HALF];
                }
            }
            if (cs && on) {
                const float2 rot = cs[(int64_t)key * HALF + lane];
                const float n0 = x0 * rot.x - x1 * rot.y, n1 = x0 * rot.y + x1 * rot.x;
                x0 = n0, x1 = n1;
            }
        }
        if (on) Ks[r * KS + lane] = x0, Ks[r * KS + lane + HALF] = x1;
    }
    __syncthreads();
    _Float16 *F = (_Float16 *)a.ws + ((int64_t)(b * a.nkv + hk) * nblk + kb) * NFR * 512 + lane * 8;
    for (int st = wave; st < NS; st += 4) {
        const float4 u = *(const float4 *)&Ks[l32 * KS + 16 * st + 8 * half];
        const float4 w = *(const float4 *)&Ks[l32 * KS + 16 * st + 8 * half + 4];
        const float x[8] = {u.x, u.y, u.z, u.w, w.x, w.y, w.z, w.w};
        v8h h, l;
        split8(x, h, l);
        *(v8h *)(F + (2 * st) * 512) = h;
        *(v8h *)(F + (2 * st + 1) * 512) = l;
    }
#pragma unroll
    for (int u = 0; u < VPW; u++) {
        const int f = wave + 4 * u;
        if (f >= 2 * NT) continue;
        v8h h, l;
        split8(vx[u], h, l);
        *(v8h *)(F + (2 * NS + 2 * f) * 512) = h;
        *(v8h *)(F + (2 * NS + 2 * f + 1) * 512) = l;
    }
}

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) const char lds_cchar;
__device__ __forceinline__ uint32_t lds_addr32(const void *p) { return (uint32_t)(uintptr_t)(lds_cchar *)p; }
// an LDS read the compiler does not track (the data comes from DMA the explicit waits order)
__device__ __forceinline__ v8h ds_read_v8h(uint32_t a) {
    v8h r;
    asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(a));
    return r;
}

// QO: the output also (or, with q_only, only) stored as the projection's quantized activation:
// AQ_Q8_0 (Q8_0 blocks of 32 head dims), AQ_Q8_K (head_dim 128: the workgroup's two heads are
// one 256-value Q8_K superblock of each output row; Tq a multiple of 128)
enum { AQ_NONE = 0, AQ_Q8_0 = 1, AQ_Q8_K = 2 };

template <int HD, bool MASK, int QO = AQ_NONE>
__global__ __launch_bounds__(512) void k_attn_frag(const AttnArgs a, int nblk, float qscale) {
    constexpr int NS = HD / 16, NT = HD / 32, HALF = HD / 2, NFR = kv_frags<HD>();
    constexpr float LOG2E = 1.4426950408889634f;
    __shared__ __attribute__((aligned(16))) float rs[8][32];
    extern __shared__ __attribute__((aligned(16))) char lds[];  // unmasked form: key/value ring, then staging
    // wave-uniform (scalar registers): the wave's head, query tile and ranges
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63, l32 = lane & 31, half = lane >> 5;
    const int h = blockIdx.x * 2 + (wave >> 2);
    const int b = blockIdx.y;
    const int Tq = a.Tq, Tk = a.Tk, causal = a.causal;
    // query tile of the wave: waves w and w + 4 share a SIMD, so they get tiles t and 3 - t
    // (one long and one short causal range each); the longest ranges are dispatched first
    const int qt = wave < 4 ? wave : 7 - wave;
    const int q0 = ((int)gridDim.z - 1 - (int)blockIdx.z) * 128 + qt * 32;
    // The key/value blocks pass through an LDS ring shared by the workgroup in the unmasked
    // head_dim 128 form (measured on MI355X: 97 against 110 us per Qwen3-0.6B layer of 16 x 512
    // tokens; at head_dim 32, MiniLM's 128-token sequences, 10.2 against 9.6 us the other way).
    // That form has workgroup barriers: a wave without queries (q0 >= Tq, or the missing
    // second head of an odd nq) stays and computes nothing.  The others have none.
    constexpr bool RING = !MASK && HD == 128;
    const bool idle = h >= a.nq || q0 >= Tq;
    if (!RING && idle) return;
    const int hq = min(h, a.nq - 1), hk = hq / (a.nq / a.nkv), qi = q0 + l32;
    const int qrow = min(qi, Tq - 1);
    const float2 *cs = a.cs ? a.cs + (int64_t)b * a.cs_sb : nullptr;

    // Q^T operand: step st holds Q[qi][16 st + 8 half + j], normed, rotated, times qscale
    v8h qh[NS], ql[NS];
    {
        const float *qp = a.q + (int64_t)b * a.q_sb + (int64_t)qrow * a.q_st + (int64_t)hq * a.q_sh + 8 * half;
        float x[NS][8];
#pragma unroll
        for (int st = 0; st < NS; st++) {
            const float4 u = *(const float4 *)(qp + 16 * st), w = *(const float4 *)(qp + 16 * st + 4);
            x[st][0] = u.x, x[st][1] = u.y, x[st][2] = u.z, x[st][3] = u.w;
            x[st][4] = w.x, x[st][5] = w.y, x[st][6] = w.z, x[st][7] = w.w;
        }
        if (a.qw) {
            float ss = 0.f;
#pragma unroll
            for (int st = 0; st < NS; st++)
#pragma unroll
                for (int j = 0; j < 8; j++) ss += x[st][j] * x[st][j];
            ss += __shfl_xor(ss, 32);
            const float scale = 1.0f / sqrtf(ss / (float)HD + a.eps);
#pragma unroll
            for (int st = 0; st < NS; st++)
#pragma unroll
                for (int j = 0; j < 8; j++) x[st][j] = x[st][j] * scale * a.qw[16 * st + 8 * half + j];
        }
        if (cs) {
            // pair (d, d + HD/2) sits in steps st and st + NS/2 of the same lane and slot
#pragma unroll
            for (int st = 0; st < NS / 2; st++)
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float2 rot = cs[(int64_t)qrow * HALF + 16 * st + 8 * half + j];
                    const float x0 = x[st][j], x1 = x[st + NS / 2][j];
                    x[st][j] = x0 * rot.x - x1 * rot.y;
                    x[st + NS / 2][j] = x0 * rot.y + x1 * rot.x;
                }
        }
#pragma unroll
        for (int st = 0; st < NS; st++) {
#pragma unroll
            for (int j = 0; j < 8; j++) x[st][j] *= qscale;
            split8(x[st], qh[st], ql[st]);
        }
    }
    // the lane's mask row (its query column of S^T)
    const _Float16 *mrow = nullptr;
    if constexpr (MASK)
        mrow = (const _Float16 *)a.mask + (int64_t)b * a.m_sb + (int64_t)h * a.m_sh + (int64_t)qrow * a.m_sq;
    v16f oacc[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) oacc[n] = (v16f){};
    float m_run = -INFINITY, l_run = 0.f;
    const int kend = causal ? min(Tk, q0 + 32) : Tk;
    // One key block kb: S^T = K Q^T, the online softmax, O += P V.  load(fr, f0) fills fr with
    // the block's fragments f0 .. f0 + NFR/2 - 1 (K: hi, lo per 16-deep step; V from 2 NS: hi,
    // lo per (step, column tile)), complete on return.
    auto block = [&](int kb, auto &&load) __attribute__((always_inline)) {
        // three accumulators, so consecutive MFMAs never chain on one accumulator
        v16f s_hh = (v16f){}, s_hl = (v16f){}, s_lh = (v16f){};
        v8h fr[NFR / 2];
        load(fr, 0);  // K: hi, lo of each 16-deep step
#pragma unroll
        for (int st = 0; st < NS; st++) {
            const v8h ah = fr[2 * st], al = fr[2 * st + 1];
            s_hh = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, qh[st], s_hh, 0, 0, 0);
            s_hl = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, ql[st], s_hl, 0, 0, 0);
            s_lh = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, qh[st], s_lh, 0, 0, 0);
        }
        load(fr, 2 * NS);  // V: hi, lo of each (step t, column tile n)
        const v16f sc = s_hh + (s_hl + s_lh);
        float p[16], mblk = -INFINITY;
        // a block inside every query's range (below the causal diagonal of the wave's first
        // query, before Tk, no mask) needs no per-key test (a wave-uniform branch)
        const bool full = !MASK && kb * 32 + 32 <= Tk && (!causal || kb * 32 + 31 <= q0);
        if (full) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                p[i] = sc[i];
                mblk = fmaxf(mblk, p[i]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int key = kb * 32 + 8 * (i / 4) + 4 * half + (i % 4);
                if (key >= Tk || (causal && key > qi)) {
                    p[i] = -INFINITY;
                } else {
                    p[i] = sc[i];
                    if constexpr (MASK) p[i] += LOG2E * (float)mrow[key];
                }
                mblk = fmaxf(mblk, p[i]);
            }
        }
        mblk = fmaxf(mblk, __shfl_xor(mblk, 32));
        const float m_new = fmaxf(m_run, mblk);
        // -inf while every key so far is masked: then alpha and p are 0 (without a mask key
        // 32 kb <= every query of the wave keeps m_new finite)
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        // 2^x by v_exp_f32 itself: the arguments are <= 0 and results below 2^-126 (flushed by
        // the instruction, which exp2f's denormal path would keep) are nothing beside the
        // block's largest probability, 1.  P carries a factor 2^15 (folded into the exponent)
        // so that its hi / lo fp16 split is exact.
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);  // 0 on the first block
        const float m_off = m_use - 15.0f;
        float lblk = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            p[i] = __builtin_amdgcn_exp2f(p[i] - m_off);
            lblk += p[i];
        }
        lblk += __shfl_xor(lblk, 32);
        l_run = l_run * alpha + lblk;
        m_run = m_new;

        if (__ballot(alpha != 1.0f)) {
            // rescale O's rows (queries 8(r/4) + 4 half + r%4) by their query's alpha.  The
            // reads are asm: the compiler would make a plain LDS read wait for the key/value
            // DMA in flight (it cannot tell rs from the ring)
            rs[wave][l32] = alpha;
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // one wave writes and reads its slot
            const uint32_t ra = lds_addr32(&rs[wave][4 * half]);
            v8h t4[4];
#pragma unroll
            for (int g = 0; g < 4; g++) t4[g] = ds_read_v8h(ra + 32u * g);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            float al[16];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                asm volatile("" : "+v"(t4[g]));
                const float4 t = __builtin_bit_cast(float4, t4[g]);
                al[4 * g] = t.x, al[4 * g + 1] = t.y, al[4 * g + 2] = t.z, al[4 * g + 3] = t.w;
            }
#pragma unroll
            for (int n = 0; n < NT; n++)
#pragma unroll
                for (int r = 0; r < 16; r++) oacc[n][r] *= al[r];
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the slot is rewritten later
        }
#pragma unroll
        for (int t = 0; t < 2; t++) {
            float px[8];
#pragma unroll
            for (int j = 0; j < 8; j++) px[j] = p[8 * t + j];
            v8h ph, pl;
            split8(px, ph, pl);
            // term-major order: consecutive MFMAs write different accumulators
#pragma unroll
            for (int n = 0; n < NT; n++) oacc[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ph, fr[2 * (t * NT + n)], oacc[n], 0, 0, 0);
#pragma unroll
            for (int n = 0; n < NT; n++) oacc[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ph, fr[2 * (t * NT + n) + 1], oacc[n], 0, 0, 0);
#pragma unroll
            for (int n = 0; n < NT; n++) oacc[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pl, fr[2 * (t * NT + n)], oacc[n], 0, 0, 0);
        }
    };
    if constexpr (!RING) {
        const v8h *F = (const v8h *)((const _Float16 *)a.ws + (int64_t)(b * a.nkv + hk) * nblk * NFR * 512) + lane;
        for (int kb = 0; kb * 32 < kend; kb++) {
            if constexpr (MASK) {
                // a block that no query of the wave can see (a causal mask's upper triangle,
                // padding) is skipped whole.  The values are read again after the MFMAs (cache
                // hits) rather than kept live across them: at 2 waves per SIMD the 16 extra
                // registers spill.
                bool live = false;
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const int key = kb * 32 + 8 * (i / 4) + 4 * half + (i % 4);
                    live |= key < Tk && (float)mrow[min(key, Tk - 1)] != -INFINITY;
                }
                if (__ballot(live) == 0) continue;
            }
            const v8h *Fb = F + (int64_t)kb * NFR * 64;
            block(kb, [&](v8h(&fr)[NFR / 2], int f0) __attribute__((always_inline)) {
#pragma unroll
                for (int i = 0; i < NFR / 2; i++) fr[i] = Fb[(int64_t)(f0 + i) * 64];
            });
        }
    } else {
        // The workgroup's key blocks pass through a two-slot LDS ring: all 8 waves DMA block
        // kb + 1 (global_load_lds, 1 KB fragments; both heads' key/value heads, one copy when
        // they share it) while computing block kb from the other slot, one barrier per block.
        // Every wave walks the workgroup's whole key range (the longest causal range of its
        // query tiles) and computes only its own; an idle wave only moves data.
        const int gq = a.nq / a.nkv;
        const int hk0 = min(2 * (int)blockIdx.x, a.nq - 1) / gq, hk1 = min(2 * (int)blockIdx.x + 1, a.nq - 1) / gq;
        const int nfr = hk0 == hk1 ? NFR : 2 * NFR;  // fragments per block in a slot
        const int qbase = ((int)gridDim.z - 1 - (int)blockIdx.z) * 128;
        const int nkb = ((causal ? min(Tk, qbase + 128) : Tk) + 31) / 32;
        const _Float16 *G0 = (const _Float16 *)a.ws + (int64_t)(b * a.nkv + hk0) * nblk * NFR * 512 + lane * 8;
        const _Float16 *G1 = (const _Float16 *)a.ws + (int64_t)(b * a.nkv + hk1) * nblk * NFR * 512 + lane * 8;
        const uint32_t ring = lds_addr32(lds);
        const uint32_t mine = (hk == hk0 ? 0u : (uint32_t)NFR * 1024u) + (uint32_t)lane * 16u;
        auto issue = [&](int kb) __attribute__((always_inline)) {
            char *slot = lds + (kb & 1) * (2 * NFR * 1024);
            for (int f = wave; f < nfr; f += 8) {
                const _Float16 *src = f < NFR ? G0 + (int64_t)(kb * NFR + f) * 512 : G1 + (int64_t)(kb * NFR + f - NFR) * 512;
                __builtin_amdgcn_global_load_lds(src, (lds_void *)(slot + f * 1024), 16, 0, 0);
            }
        };
        issue(0);
        for (int kb = 0; kb < nkb; kb++) {
            // block kb has landed (this wave's DMAs; the barrier: every wave's), and every wave
            // is done reading the slot the next DMAs overwrite (block kb - 1)
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (kb + 1 < nkb) issue(kb + 1);
            if (idle || kb * 32 >= kend) continue;
            const uint32_t base = ring + (uint32_t)(kb & 1) * (2 * NFR * 1024) + mine;
            block(kb, [&](v8h(&fr)[NFR / 2], int f0) __attribute__((always_inline)) {
#pragma unroll
                for (int i = 0; i < NFR / 2; i++) fr[i] = ds_read_v8h(base + (uint32_t)(f0 + i) * 1024u);
                // the asm reads complete here; each fragment is tied to the wait
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
                for (int i = 0; i < NFR / 2; i++) asm volatile("" : "+v"(fr[i]));
            });
        }
        // the LDS ring is free for the epilogue's staging
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }

    rs[wave][l32] = l_run > 0.f ? 1.0f / l_run : 0.f;  // O and l both carry the factor 2^15
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    float inv[16];
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const float4 t = *(const float4 *)&rs[wave][8 * g + 4 * half];
        inv[4 * g] = t.x, inv[4 * g + 1] = t.y, inv[4 * g + 2] = t.z, inv[4 * g + 3] = t.w;
    }
    float *ob = a.out + (int64_t)b * a.o_sb + (int64_t)hq * a.o_sh + l32;
    if (!idle && (QO == AQ_NONE || !a.q_only)) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int q = q0 + 8 * (r / 4) + 4 * half + (r % 4);
            if (q >= Tq) continue;
            float *o = ob + (int64_t)q * a.o_st;
#pragma unroll
            for (int n = 0; n < NT; n++) o[32 * n] = oacc[n][r] * inv[r];
        }
    }
    if constexpr (QO == AQ_Q8_0) {
        // The same values quantized for the projection that reads them: 32 head dims of one
        // query are one Q8_0 block of output row b * Tq + q, chunk h * NT + n.  The wave's
        // 32 x 32 tile goes through LDS so that lane l holds query l % 32, dims 16 (l / 32) ..,
        // its 16 bytes of the activation fragment.
        constexpr int QST = 36;
        __shared__ __attribute__((aligned(16))) float stg[8][32 * QST];
        float *tile = stg[wave];
        const int q = q0 + l32;
        const int64_t row = (int64_t)b * Tq + q;
#pragma unroll
        for (int n = 0; n < NT; n++) {
#pragma unroll
            for (int r = 0; r < 16; r++) tile[(8 * (r / 4) + 4 * half + (r % 4)) * QST + l32] = oacc[n][r] * inv[r];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            float v[16];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float4 t4 = *(const float4 *)(tile + l32 * QST + 16 * half + 4 * u);
                v[4 * u] = t4.x, v[4 * u + 1] = t4.y, v[4 * u + 2] = t4.z, v[4 * u + 3] = t4.w;
            }
            uint4 pk;
            const float d = requant_q8_0(v, true, MQ_PRE_NONE, a.q_var, pk);
            if (q < Tq && !idle) {
                const int64_t chunk = (int64_t)h * NT + n;
                *(uint4 *)(a.qo + (((row >> 5) * a.q_kch + chunk) << 10) + (((row & 31) + 32 * half) << 4)) = pk;
                if (half == 0) a.qd[chunk * a.q_m_pad + row] = d;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    }
    if constexpr (QO == AQ_Q8_K) {
        // Output columns 256 bx .. 256 bx + 255 (heads 2 bx and 2 bx + 1, 128 dims each) are one
        // Q8_K superblock of every output row.  The two waves of a query tile (head slot hs)
        // stage their 32 x 128 halves side by side in LDS; after the barrier each quantizes 16 of
        // the tile's 32 rows over all 256 values, lane l holding values 4l .. 4l + 3 (the tiled
        // activation quantizer's arithmetic and lane layout), straight into the workspace.  Every
        // wave of the workgroup reaches the barrier: the host launches this form only for an even
        // nq and Tq a multiple of 128.
        static_assert(HD == 128, "a superblock is two heads of 128");
        constexpr int SST = 260;  // staging row stride in floats (the LDS ring's space, free now)
        float *tile = (float *)lds + qt * (32 * SST);
        const int hs = wave >> 2;
#pragma unroll
        for (int n = 0; n < NT; n++)
#pragma unroll
            for (int r = 0; r < 16; r++)
                tile[(8 * (r / 4) + 4 * half + (r % 4)) * SST + hs * HD + 32 * n + l32] = oacc[n][r] * inv[r];
        __syncthreads();
        const int64_t sb = blockIdx.x;
        int8_t *qbase = a.qo + ((sb * 8 + (lane >> 3)) << 10) + ((32 * ((lane >> 2) & 1)) << 4) + 4 * (lane & 3);
#pragma unroll 2
        for (int i = 0; i < 16; i++) {
            const int rr = hs * 16 + i;
            const int64_t row = (int64_t)b * Tq + q0 + rr, rt = row >> 5;
            const int r32 = (int)(row & 31);
            const float4 v = *(const float4 *)(tile + rr * SST + 4 * lane);
            q8_K_block_row(v, lane, r32, qbase + ((rt * a.q_kch) << 10) + (r32 << 4), a.qd + sb * a.q_m_pad + row,
                           a.qmin + ((rt * a.q_nsb + sb) << 9));
        }
    }
}

// Split-key form for grids too small to fill the GPU (one sequence, few heads) and for masked
// head_dim 128: a workgroup of NW waves owns one (head, 32-query tile); wave w runs the same
// online softmax over key blocks w, w + NW, ... and the NW partial (max, sum, O) are merged
// through LDS:
//   m = max_w m_w,  O = sum_w 2^(m_w - m) O_w,  l = sum_w 2^(m_w - m) l_w,  out = O / l.
// With a mask (MK = 1), each wave first classifies its first 64 key blocks from the mask values
// of the tile's 32 rows (all loads in flight together): no finite value -> the block is skipped;
// all values 0 -> it runs unmasked, with no mask reads; else it adds the mask as it goes.  A
// causal mask thus costs one pass over it, not a dependent load per key block.  With the mask's
// block lists (MK = 2, launch_mask_blocks: the same classification, made once for all heads and
// every attention that reads the mask) the waves take the tile's live blocks in turn: a
// block-diagonal batch mask over thousands of keys then costs the tile's own blocks only.
// QO (head_dim 32 / 64): the merged rows also leave as the Q8_0 activation of the projection
// that reads them (AttnArgs::qo), as the 8-wave kernel's store writes it.
template <int HD, int MK, int NW, bool QO = false>
__global__ __launch_bounds__(64 * NW, 2) void k_attn_split(const AttnArgs a, int nblk, float qscale) {
    constexpr bool MASK = MK != 0;
    constexpr int NS = HD / 16, NT = HD / 32, HALF = HD / 2, NFR = kv_frags<HD>();
    constexpr float LOG2E = 1.4426950408889634f;
    __shared__ __attribute__((aligned(16))) float rs[NW][32];
    __shared__ float mls[NW][2][32];
    __shared__ __attribute__((aligned(16))) float ored[NW][NT][16][64];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, l32 = lane & 31,
              half = lane >> 5;
    const int h = blockIdx.x, b = blockIdx.y;
    const int Tq = a.Tq, Tk = a.Tk, causal = a.causal;
    const int q0 = ((int)gridDim.z - 1 - (int)blockIdx.z) * 32;  // longest causal ranges first
    const int hk = h / (a.nq / a.nkv), qi = q0 + l32;
    const int qrow = min(qi, Tq - 1);
    const float2 *cs = a.cs ? a.cs + (int64_t)b * a.cs_sb : nullptr;

    // the tile's query fragments (hi, lo per 16-dim step), the same for every wave: once in LDS
    // (in the merge buffer, free until the merge), read back per key block
    v8h *qf = (v8h *)&ored[0][0][0][0];
    // wave p < NS / 2 prepares dim steps p and p + NS / 2 (the pair RoPE rotates together);
    // the RMS norm's sum of squares is reduced across those waves through ssp
    {
        constexpr int NP = NS / 2;
        static_assert(NP <= NW, "one dim-step pair per wave");
        float *ssp = (float *)(qf + 2 * NS * 64);
        const bool act = wave < NP;
        const int st0 = act ? wave : 0, st1 = st0 + NP;
        const float *qp = a.q + (int64_t)b * a.q_sb + (int64_t)qrow * a.q_st + (int64_t)h * a.q_sh + 8 * half;
        float x[2][8];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int st = t ? st1 : st0;
            const float4 u = *(const float4 *)(qp + 16 * st), w = *(const float4 *)(qp + 16 * st + 4);
            x[t][0] = u.x, x[t][1] = u.y, x[t][2] = u.z, x[t][3] = u.w;
            x[t][4] = w.x, x[t][5] = w.y, x[t][6] = w.z, x[t][7] = w.w;
        }
        float2 rot[8];  // loaded with q, before the norm's reduction
        if (cs)
#pragma unroll
            for (int j = 0; j < 8; j++) rot[j] = cs[(int64_t)qrow * HALF + 16 * st0 + 8 * half + j];
        if (a.qw) {
            float ss = 0.f;
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int j = 0; j < 8; j++) ss += x[t][j] * x[t][j];
            ssp[wave * 64 + lane] = act ? ss : 0.f;
            __syncthreads();
            float tot = 0.f;
#pragma unroll
            for (int w = 0; w < NP; w++) tot += ssp[w * 64 + lane] + ssp[w * 64 + (lane ^ 32)];
            const float scale = 1.0f / sqrtf(tot / (float)HD + a.eps);
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const int st = t ? st1 : st0;
#pragma unroll
                for (int j = 0; j < 8; j++) x[t][j] = x[t][j] * scale * a.qw[16 * st + 8 * half + j];
            }
        }
        if (cs) {
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float x0 = x[0][j], x1 = x[1][j];
                x[0][j] = x0 * rot[j].x - x1 * rot[j].y;
                x[1][j] = x0 * rot[j].y + x1 * rot[j].x;
            }
        }
        if (act)
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const int st = t ? st1 : st0;
#pragma unroll
                for (int j = 0; j < 8; j++) x[t][j] *= qscale;
                v8h qh, ql;
                split8(x[t], qh, ql);
                qf[(2 * st) * 64 + lane] = qh, qf[(2 * st + 1) * 64 + lane] = ql;
            }
    }
    __syncthreads();
    const _Float16 *mrow = nullptr;
    if constexpr (MASK)
        mrow = (const _Float16 *)a.mask + (int64_t)b * a.m_sb + (int64_t)h * a.m_sh + (int64_t)qrow * a.m_sq;
    v16f oacc[NT];
#pragma unroll
    for (int n = 0; n < NT; n++) oacc[n] = (v16f){};
    float m_run = -INFINITY, l_run = 0.f;
    const int kend = causal ? min(Tk, q0 + 32) : Tk;
    const v8h *F = (const v8h *)((const _Float16 *)a.ws + (int64_t)(b * a.nkv + hk) * nblk * NFR * 512) + lane;

    // bit j: the wave's key block wave + NW j is fully masked (dead) / has an all-zero mask.
    // Rows 16-byte aligned (m_al): lane l reads 8 keys (16 bytes) of row l / 4 and of row
    // l / 4 + 16, coalesced; else each lane its own row's 16 keys of the block, 2 bytes at a time.
    uint64_t dead = 0, zero = 0;
    if constexpr (MK == 1) {
        constexpr int CJ = 2;  // blocks classified per pass
        const int nj = min((kend - 32 * wave + 32 * NW - 1) / (32 * NW), 64);
        const uint16_t *mbase = a.mask + (int64_t)b * a.m_sb + (int64_t)h * a.m_sh;
        for (int j0 = 0; j0 < nj; j0 += CJ) {
            bool live[CJ], nz[CJ];
#pragma unroll
            for (int jj = 0; jj < CJ; jj++) {
                live[jj] = false, nz[jj] = false;
                const int kb = wave + NW * (j0 + jj);
                if (a.m_al && kb * 32 + 32 <= Tk) {
#pragma unroll
                    for (int r = 0; r < 2; r++) {
                        const int row = min(q0 + (lane >> 2) + 16 * r, Tq - 1);
                        const uint4 u = *(const uint4 *)(mbase + (int64_t)row * a.m_sq + kb * 32 + 8 * (lane & 3));
                        const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            // f16 -inf is 0xFC00; +-0 have no bits outside the sign
                            live[jj] |= (w4[e] & 0xFFFFu) != 0xFC00u || (w4[e] >> 16) != 0xFC00u;
                            nz[jj] |= (w4[e] & 0x7FFF7FFFu) != 0u;
                        }
                    }
                    if (j0 + jj >= nj) live[jj] = false, nz[jj] = false;
                } else {
#pragma unroll
                    for (int i = 0; i < 16; i++) {
                        const int key = kb * 32 + 8 * (i / 4) + 4 * half + (i % 4);
                        const bool in = j0 + jj < nj && key < Tk;
                        const float m = (float)mrow[min(key, Tk - 1)];
                        live[jj] |= in && m != -INFINITY;
                        nz[jj] |= in && m != 0.0f;
                    }
                }
            }
#pragma unroll
            for (int jj = 0; jj < CJ; jj++) {
                dead |= (uint64_t)(__ballot(live[jj]) == 0) << (j0 + jj);
                zero |= (uint64_t)(__ballot(nz[jj]) == 0) << (j0 + jj);
            }
        }
    }

    // key block kb (mixed: it adds the mask) into the wave's running (max, sum, O)
    auto run_block = [&](const int kb, const bool mixed) __attribute__((always_inline)) {
        const v8h *Fb = F + (int64_t)kb * NFR * 64;
        v16f s_hh = (v16f){}, s_hl = (v16f){}, s_lh = (v16f){};
        // an address the compiler cannot see through, so the fragment reads stay in the loop
        uint32_t qa = lds_addr32(qf) + 16u * lane;
        asm volatile("" : "+v"(qa));
        const __attribute__((address_space(3))) v8h *ql3 = (const __attribute__((address_space(3))) v8h *)qa;
#pragma unroll
        for (int st = 0; st < NS; st++) {
            const v8h ah = Fb[(2 * st) * 64], al = Fb[(2 * st + 1) * 64];
            const v8h qh = ql3[(2 * st) * 64], ql = ql3[(2 * st + 1) * 64];
            s_hh = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, qh, s_hh, 0, 0, 0);
            s_hl = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, ql, s_hl, 0, 0, 0);
            s_lh = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, qh, s_lh, 0, 0, 0);
        }
        v8h bh[2][NT], bl[2][NT];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int n = 0; n < NT; n++) {
                bh[t][n] = Fb[(2 * NS + 2 * (t * NT + n)) * 64];
                bl[t][n] = Fb[(2 * NS + 2 * (t * NT + n) + 1) * 64];
            }
        const v16f sc = s_hh + (s_hl + s_lh);
        v8h mh[2] = {};  // the block's mask values, as stored (f16)
        if constexpr (MASK)
            if (mixed) {
                if (a.m_al && kb * 32 + 32 <= Tk) {
#pragma unroll
                    for (int g = 0; g < 4; g++) {
                        const uint2 u = *(const uint2 *)(mrow + kb * 32 + 8 * g + 4 * half);
                        const v4h hv = __builtin_bit_cast(v4h, u);
#pragma unroll
                        for (int e = 0; e < 4; e++) mh[g / 2][4 * (g % 2) + e] = hv[e];
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 16; i++) {
                        const int key = kb * 32 + 8 * (i / 4) + 4 * half + (i % 4);
                        mh[i / 8][i % 8] = mrow[min(key, Tk - 1)];  // keys past Tk: p = -inf below
                    }
                }
            }
        float p[16], mblk = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int key = kb * 32 + 8 * (i / 4) + 4 * half + (i % 4);
            if (key >= Tk || (causal && key > qi)) {
                p[i] = -INFINITY;
            } else {
                p[i] = sc[i];
                if constexpr (MASK)
                    if (mixed) p[i] += LOG2E * (float)mh[i / 8][i % 8];
            }
            mblk = fmaxf(mblk, p[i]);
        }
        mblk = fmaxf(mblk, __shfl_xor(mblk, 32));
        const float m_new = fmaxf(m_run, mblk);
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = exp2f(m_run - m_use);
        float lblk = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            p[i] = exp2f(p[i] - m_use);
            lblk += p[i];
        }
        lblk += __shfl_xor(lblk, 32);
        l_run = l_run * alpha + lblk;
        m_run = m_new;
        if (__ballot(alpha != 1.0f)) {
            rs[wave][l32] = alpha;
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            float al[16];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const float4 t = *(const float4 *)&rs[wave][8 * g + 4 * half];
                al[4 * g] = t.x, al[4 * g + 1] = t.y, al[4 * g + 2] = t.z, al[4 * g + 3] = t.w;
            }
#pragma unroll
            for (int n = 0; n < NT; n++)
#pragma unroll
                for (int r = 0; r < 16; r++) oacc[n][r] *= al[r];
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
#pragma unroll
        for (int t = 0; t < 2; t++) {
            float px[8];
#pragma unroll
            for (int j = 0; j < 8; j++) px[j] = p[8 * t + j] * 32768.0f;
            v8h ph, pl;
            split8(px, ph, pl);
#pragma unroll
            for (int n = 0; n < NT; n++) oacc[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ph, bh[t][n], oacc[n], 0, 0, 0);
#pragma unroll
            for (int n = 0; n < NT; n++) oacc[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ph, bl[t][n], oacc[n], 0, 0, 0);
#pragma unroll
            for (int n = 0; n < NT; n++) oacc[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pl, bh[t][n], oacc[n], 0, 0, 0);
        }
    };
    if constexpr (MK == 2) {
        const uint32_t *lst = a.blist + ((int64_t)(a.m_sb ? b : 0) * a.bl_nqt + (q0 >> 5)) * a.bl_stride;
        const int nl = (int)lst[0];
        for (int j = wave; j < nl; j += NW) {
            const uint32_t e = lst[1 + j];
            run_block((int)(e & 0x7FFFFFFFu), (e >> 31) != 0);
        }
    } else {
        for (int j = 0, kb = wave; kb * 32 < kend; j++, kb += NW) {
            bool mixed = MASK;
            if constexpr (MASK) {
                if (j < 64) {
                    if ((dead >> j) & 1) continue;
                    mixed = !((zero >> j) & 1);
                } else {  // past the classified blocks: the same test here
                    bool live = false;
#pragma unroll
                    for (int i = 0; i < 16; i++) {
                        const int key = kb * 32 + 8 * (i / 4) + 4 * half + (i % 4);
                        live |= key < Tk && (float)mrow[min(key, Tk - 1)] != -INFINITY;
                    }
                    if (__ballot(live) == 0) continue;
                }
            }
            run_block(kb, mixed);
        }
    }

    // merge the waves' partial results: wave w reduces columns 32 (w % NT) .. + 31 of rows
    // r = w / NT, w / NT + NW / NT, ... of the 16 accumulator rows (after every wave's last
    // query-fragment read)
    __syncthreads();
    if (half == 0) mls[wave][0][l32] = m_run, mls[wave][1][l32] = l_run;
#pragma unroll
    for (int n = 0; n < NT; n++)
#pragma unroll
        for (int r = 0; r < 16; r++) ored[wave][n][r][lane] = oacc[n][r];
    __syncthreads();
    constexpr int RS = NW >= NT ? NW / NT : 1;
    for (int n = wave % NT; n < NT; n += NW >= NT ? NT : NW) {
        // not unrolled: at short sequences each wave runs this code once, and the kernel's
        // time goes to fetching its instructions
#pragma unroll 1
        for (int r = NW >= NT ? wave / NT : 0; r < 16; r += RS) {
            const int qq = 8 * (r / 4) + 4 * half + (r % 4), q = q0 + qq;
            float mx = -INFINITY;
#pragma unroll
            for (int w = 0; w < NW; w++) mx = fmaxf(mx, mls[w][0][qq]);
            float o = 0.f, l = 0.f;
            if (mx != -INFINITY) {
#pragma unroll
                for (int w = 0; w < NW; w++) {
                    const float f = exp2f(mls[w][0][qq] - mx);  // 0 for a wave that saw no key
                    o += f * ored[w][n][r][lane];
                    l += f * mls[w][1][qq];
                }
            }
            const float val = l > 0.f ? o / (l * 32768.0f) : 0.f;
            if (q < Tq) {
                float *ob = a.out + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)q * a.o_st + l32 + 32 * n;
                *ob = val;
            }
            // QO: the merged value also goes to LDS for the quantizer below, into this (n, r)'s
            // slot of wave 0's partial -- read above by this lane alone (each (n, r) has one wave)
            if constexpr (QO) ored[0][n][r][lane] = val;
        }
    }
    if constexpr (QO) {
        // the merged 32 x HD tile quantized as the projection's Q8_0 activation, as the 8-wave
        // kernel's store writes it: wave n < NT takes dims 32 n .. + 31 (one Q8_0 block of output
        // row b Tq + q, chunk h NT + n), lane l query l % 32 and its 16 values 16 (l / 32) ..
        // (row r = 4 (q / 8) + q % 4, lane 32 ((q / 4) % 2) + dim of the merge above)
        __syncthreads();
        if (wave < NT) {
            const int n = wave, qq = l32, q = q0 + qq;
            const float *src = &ored[0][n][4 * (qq >> 3) + (qq & 3)][32 * ((qq >> 2) & 1) + 16 * half];
            float v[16];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float4 t4 = *(const float4 *)(src + 4 * u);
                v[4 * u] = t4.x, v[4 * u + 1] = t4.y, v[4 * u + 2] = t4.z, v[4 * u + 3] = t4.w;
            }
            uint4 pk;
            const float d = requant_q8_0(v, true, MQ_PRE_NONE, a.q_var, pk);
            if (q < Tq) {
                const int64_t row = (int64_t)b * Tq + q, chunk = (int64_t)h * NT + n;
                *(uint4 *)(a.qo + (((row >> 5) * a.q_kch + chunk) << 10) + (((row & 31) + 32 * half) << 4)) = pk;
                if (half == 0) a.qd[chunk * a.q_m_pad + row] = d;
            }
        }
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

size_t attn_workspace_bytes(int B, int Tk, int nkv, int hd) {
    const int nfr = hd == 128 ? kv_frags<128>() : hd == 64 ? kv_frags<64>() : kv_frags<32>();
    return (size_t)B * nkv * ((Tk + 31) / 32) * nfr * 1024;
}

hipError_t launch_rope_table(float2 *cs, int T, int hd, float theta_base, hipStream_t s) {
    const float theta_scale = powf(theta_base, -2.0f / (float)hd);
    hipLaunchKernelGGL(k_rope_table, dim3((unsigned)((T * (hd / 2) + 255) / 256)), dim3(256), 0, s, cs, T, hd / 2,
                       theta_scale);
    return hipGetLastError();
}

// The unmasked 8-wave kernel with its dynamic LDS: at head_dim 128 the two-slot key/value ring
// (two heads' fragments per slot), or the Q8_K store's staging where that is larger (the limit
// raised once per device).
template <int HD, int QO>
static hipError_t launch_attn_8w(dim3 grid, const AttnArgs &a, int nblk, float qscale, hipStream_t s) {
    constexpr int RING = HD == 128 ? 2 * 2 * kv_frags<HD>() * 1024 : 0, STG = QO == AQ_Q8_K ? 4 * 32 * 260 * 4 : 0;
    constexpr int BYTES = RING > STG ? RING : STG;
    static std::atomic<bool> attr_set[MQ_MAX_DEVICES];
    const hipError_t e = dyn_lds_once((const void *)k_attn_frag<HD, false, QO>, BYTES, attr_set);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((k_attn_frag<HD, false, QO>), grid, dim3(512), BYTES, s, a, nblk, qscale);
    return hipGetLastError();
}

// The split-key form when the regular grid (2 heads x 128 queries per workgroup) would leave
// most CUs idle, there are several key blocks to share out and the split grid (a head and 32
// queries per workgroup) fits one round of two workgroups per CU (MI355X, 32 sequences x 128
// tokens, 6 heads of 64: 96 regular workgroups 15.4 us against 768 split ones 19.4 us), for
// masked head_dim 128 (the 8-wave kernel's mask addressing does not fit its 256 registers and
// spills), and for a mask
// shared by every head over 1024 keys or more (a packed batch's block-diagonal mask: the split
// form runs only the blocks the mask leaves live, the 8-wave kernel tests every key block);
// MQ_ATTN_SPLIT=0/1 forces either form (measurements)
bool attn_split_form(const AttnArgs &a) {
    const int nblk = (a.Tk + 31) / 32;
    const int64_t wgs = (int64_t)((a.nq + 1) / 2) * a.B * ((a.Tq + 127) / 128);
    // a mask shared by the heads (a padding, causal or packed mask) takes the split form at every
    // length: its key blocks are classified once per graph (block lists), where the 8-wave kernel
    // reads the mask of every block for every head (MI355X, 32 ragged sequences x 128 tokens,
    // head_dim 32: 38.5 -> 16.6 us; head_dim 64: 42.8 -> 22.7 us)
    const int64_t split_wgs = (int64_t)a.nq * a.B * ((a.Tq + 31) / 32);
    bool split = (wgs < 128 && nblk >= 4 && split_wgs <= 512) || (a.hd == 128 && a.mask) || (a.mask && a.m_sh == 0);
    if (const char *e = getenv("MQ_ATTN_SPLIT"))
        if (*e) split = atoi(e) != 0;
    return split;
}

template <int HD, int NW, bool QO>
static void launch_attn_split_q(dim3 g, const AttnArgs &a, int nblk, float qscale, hipStream_t s) {
    if (a.mask && a.blist) hipLaunchKernelGGL((k_attn_split<HD, 2, NW, QO>), g, dim3(64 * NW), 0, s, a, nblk, qscale);
    else if (a.mask) hipLaunchKernelGGL((k_attn_split<HD, 1, NW, QO>), g, dim3(64 * NW), 0, s, a, nblk, qscale);
    else hipLaunchKernelGGL((k_attn_split<HD, 0, NW, QO>), g, dim3(64 * NW), 0, s, a, nblk, qscale);
}

template <int HD, int NW>
static void launch_attn_split(dim3 g, const AttnArgs &a, int nblk, float qscale, hipStream_t s) {
    if constexpr (HD <= 64) {
        if (a.qo) return launch_attn_split_q<HD, NW, true>(g, a, nblk, qscale, s);
    }
    launch_attn_split_q<HD, NW, false>(g, a, nblk, qscale, s);
}

template <int HD>
static hipError_t launch_attn_hd(const AttnArgs &a, int nblk, float qscale, hipStream_t s) {
    const dim3 gk((unsigned)nblk, (unsigned)a.nkv, (unsigned)a.B);
    if (!a.kv_ready) hipLaunchKernelGGL((k_kv_frag<HD>), gk, dim3(256), 0, s, a, nblk);
    if (attn_split_form(a)) {
        // 8 waves per workgroup (half the key blocks per wave) while the grid is at most a few
        // workgroups per CU; MQ_ATTN_SPLIT_WAVES=4/8 forces either (measurements)
        const dim3 g((unsigned)a.nq, (unsigned)a.B, (unsigned)((a.Tq + 31) / 32));
        int nw = (int64_t)g.x * g.y * g.z <= 1024 ? 8 : 4;
        if (const char *e = getenv("MQ_ATTN_SPLIT_WAVES"))
            if (*e) nw = atoi(e) == 4 ? 4 : 8;
        if (nw == 8) launch_attn_split<HD, 8>(g, a, nblk, qscale, s);
        else launch_attn_split<HD, 4>(g, a, nblk, qscale, s);
        return hipGetLastError();
    }
    const dim3 ga((unsigned)((a.nq + 1) / 2), (unsigned)a.B, (unsigned)((a.Tq + 127) / 128));
    if constexpr (HD <= 64) {
        if (a.qo) {  // quantized output: the unmasked / masked forms with the Q8_0 store
            if (!a.mask) return launch_attn_8w<HD, AQ_Q8_0>(ga, a, nblk, qscale, s);
            hipLaunchKernelGGL((k_attn_frag<HD, true, AQ_Q8_0>), ga, dim3(512), 0, s, a, nblk, qscale);
            return hipGetLastError();
        }
    } else {
        if (a.qo)  // the Q8_K store (attn_frag_form: no mask, even nq, Tq a multiple of 128)
            return launch_attn_8w<HD, AQ_Q8_K>(ga, a, nblk, qscale, s);
    }
    if (!a.mask) return launch_attn_8w<HD, AQ_NONE>(ga, a, nblk, qscale, s);
    hipLaunchKernelGGL((k_attn_frag<HD, true>), ga, dim3(512), 0, s, a, nblk, qscale);
    return hipGetLastError();
}

// true when launch_attn_hd takes the 8-wave fragment kernel with a store of the output
// quantized for a weight of type q_type (AttnArgs::qo): Q8_0 at head_dim 32 / 64; Q8_K at
// head_dim 128 when the workgroup's two heads make whole superblocks of complete query tiles
// (even nq, Tq a multiple of 128, no mask).  Otherwise the caller quantizes the fp32 output.
static bool attn_frag_form(const AttnArgs &a, int q_type) {
    if (q_type == MQ_TYPE_Q8_0 && a.hd <= 64) return true;  // both forms store Q8_0 rows
    if (attn_split_form(a)) return false;
    return a.hd == 128 && a.nq % 2 == 0 && a.Tq % 128 == 0 && !a.mask;
}

// One workgroup per (mask plane, tile of 32 query rows): each wave classifies key blocks wave,
// wave + 4, ... (lane l: row l / 2 of the tile, keys 16 (l % 2) .. + 15 of the block; f16 -inf is
// 0xFC00, +-0 have no bits outside the sign) into LDS, then wave 0 writes the live ones in order.
__global__ __launch_bounds__(256) void k_mask_blocks(const uint16_t *__restrict__ mask, int64_t m_sq, int64_t m_sb,
                                                     int m_al, int Tq, int Tk, int nkb, uint32_t *__restrict__ out,
                                                     int stride) {
    extern __shared__ uint8_t cls[];  // nkb: 0 dead, 1 all zero, 2 mixed
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = threadIdx.x & 63;
    const int qt = blockIdx.x, bm = blockIdx.y;
    const int row = min(qt * 32 + (lane >> 1), Tq - 1), k0 = 16 * (lane & 1);
    const uint16_t *mrow = mask + (int64_t)bm * m_sb + (int64_t)row * m_sq;
    for (int kb = wave; kb < nkb; kb += 4) {
        bool live = false, nz = false;
        if (m_al && kb * 32 + 32 <= Tk) {
            const uint4 *p = (const uint4 *)(mrow + kb * 32 + k0);
            const uint4 u0 = p[0], u1 = p[1];
            const uint32_t w[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                live |= (w[e] & 0xFFFFu) != 0xFC00u || (w[e] >> 16) != 0xFC00u;
                nz |= (w[e] & 0x7FFF7FFFu) != 0u;
            }
        } else {
            for (int i = 0; i < 16; i++) {
                const int key = kb * 32 + k0 + i;
                if (key < Tk) {
                    const uint16_t v = mrow[key];
                    live |= v != 0xFC00u;
                    nz |= (v & 0x7FFFu) != 0u;
                }
            }
        }
        const bool any_live = __ballot(live) != 0, any_nz = __ballot(nz) != 0;
        if (lane == 0) cls[kb] = any_live ? (any_nz ? 2 : 1) : 0;
    }
    __syncthreads();
    if (wave != 0) return;
    uint32_t *lst = out + ((int64_t)bm * gridDim.x + qt) * stride;
    uint32_t n = 0;
    for (int base = 0; base < nkb; base += 64) {
        const int kb = base + lane;
        const int c = kb < nkb ? cls[kb] : 0;
        const uint64_t m = __ballot(c != 0);
        const uint32_t before = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
        if (c) lst[1 + n + before] = (uint32_t)kb | (c == 2 ? 0x80000000u : 0u);
        n += (uint32_t)__popcll(m);
    }
    if (lane == 0) lst[0] = n;
}

// A wave per row: every lane walks its share of the row's keys (16-byte loads when the rows are
// aligned), counting the finite values and noting the first and last of them and whether any
// finite value is not +-0; the row is a run of zeros ending on the diagonal when every finite
// value is zero, the last one is at key r and they are contiguous (count = r - first + 1).
__global__ __launch_bounds__(256) void k_mask_rows(const uint16_t *__restrict__ mask, int64_t m_sq, int m_al, int T,
                                                   int32_t *__restrict__ first) {
    const int lane = threadIdx.x & 63, r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= T) return;
    const uint16_t *row = mask + (int64_t)r * m_sq;
    int lo = INT_MAX, hi = -1, cnt = 0;
    bool nz = false;
    auto see = [&](int key, uint32_t v) {
        if (v != 0xFC00u) {
            lo = min(lo, key), hi = max(hi, key), cnt++;
            nz |= (v & 0x7FFFu) != 0u;
        }
    };
    if (m_al) {
        const int n8 = T / 8;
        for (int c = lane; c < n8; c += 64) {
            const uint4 u = *(const uint4 *)(row + 8 * c);
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int e = 0; e < 4; e++) see(8 * c + 2 * e, w[e] & 0xFFFFu), see(8 * c + 2 * e + 1, w[e] >> 16);
        }
        for (int key = 8 * n8 + lane; key < T; key += 64) see(key, row[key]);
    } else {
        for (int key = lane; key < T; key += 64) see(key, row[key]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        lo = min(lo, __shfl_xor(lo, o)), hi = max(hi, __shfl_xor(hi, o));
        cnt += __shfl_xor(cnt, o);
    }
    const bool any_nz = __ballot(nz) != 0;
    if (lane == 0) first[r] = (!any_nz && hi == r && cnt == r - lo + 1) ? lo : -1;
}

// A wave per (row, plane) of the Tq x Tk region an attention reads of an F16 mask: any value that
// is not +-0 sets *nonzero (a plain store of 1 from any lane that sees one).
__global__ __launch_bounds__(256) void k_mask_nonzero(const uint16_t *__restrict__ mask, int64_t m_sq, int64_t m_s2,
                                                      int64_t m_s3, int ne2, int Tq, int Tk, int *__restrict__ nonzero) {
    const int lane = threadIdx.x & 63, r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= Tq) return;
    const int p2 = (int)(blockIdx.y % ne2), p3 = (int)(blockIdx.y / ne2);
    const uint16_t *row = mask + (int64_t)p3 * m_s3 + (int64_t)p2 * m_s2 + (int64_t)r * m_sq;
    bool nz = false;
    for (int key = lane; key < Tk; key += 64) nz |= (row[key] & 0x7FFFu) != 0u;
    if (nz) *nonzero = 1;
}

hipError_t launch_mask_nonzero(const uint16_t *mask, int64_t m_sq, int64_t m_s2, int64_t m_s3, int ne2, int ne3, int Tq,
                               int Tk, int *nonzero, hipStream_t s) {
    if (Tq <= 0 || Tk <= 0 || ne2 <= 0 || ne3 <= 0 || (int64_t)ne2 * ne3 > 65535) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_mask_nonzero, dim3((unsigned)((Tq + 3) / 4), (unsigned)(ne2 * ne3)), dim3(256), 0, s, mask, m_sq,
                       m_s2, m_s3, ne2, Tq, Tk, nonzero);
    return hipGetLastError();
}

hipError_t launch_mask_rows(const uint16_t *mask, int64_t m_sq, bool m_al, int T, int32_t *first, hipStream_t s) {
    if (T <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_mask_rows, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, s, mask, m_sq, (int)m_al, T, first);
    return hipGetLastError();
}

// at most 16384 key blocks (LDS of the classification)
size_t mask_blocks_bytes(int Bm, int Tq, int Tk) {
    const int64_t nkb = ((int64_t)Tk + 31) / 32, nqt = ((int64_t)Tq + 31) / 32;
    if (Bm <= 0 || Tq <= 0 || Tk <= 0 || nkb > 16384 || Bm > 65535 || nqt > INT32_MAX) return 0;
    return (size_t)Bm * nqt * (nkb + 1) * 4;
}

hipError_t launch_mask_blocks(const uint16_t *mask, int64_t m_sq, int64_t m_sb, bool m_al, int Bm, int Tq, int Tk,
                              uint32_t *blocks, hipStream_t s) {
    if (mask_blocks_bytes(Bm, Tq, Tk) == 0) return hipErrorInvalidValue;
    const int nkb = (Tk + 31) / 32, nqt = (Tq + 31) / 32;
    hipLaunchKernelGGL(k_mask_blocks, dim3((unsigned)nqt, (unsigned)Bm), dim3(256), (size_t)nkb, s, mask, m_sq, m_sb,
                       (int)m_al, Tq, Tk, nkb, blocks, nkb + 1);
    return hipGetLastError();
}

hipError_t launch_attn(const AttnArgs &a, hipStream_t s) {
    if (a.B <= 0 || a.Tq <= 0 || a.Tk <= 0) return hipSuccess;
    const bool q_ok = ((uintptr_t)a.q & 15) == 0 && a.q_sb % 4 == 0 && a.q_st % 4 == 0 && a.q_sh % 4 == 0;
    if (a.nkv <= 0 || a.nq % a.nkv != 0 || !q_ok || ((uintptr_t)a.ws & 15) != 0 || a.B > 65535 ||
        (a.causal && a.Tq != a.Tk))
        return hipErrorInvalidValue;
    const int nblk = (a.Tk + 31) / 32;
    const float qscale = a.scale * 1.4426950408889634f;  // softmax in base 2
    AttnArgs b = a;
    bool quant_after = false;
    b.qo = nullptr;
    if (a.q_ws) {
        const int64_t rows = (int64_t)a.B * a.Tq, K = (int64_t)a.nq * a.hd;
        if (a.q_type != MQ_TYPE_Q8_0 && a.q_type != MQ_TYPE_Q4_K && a.q_type != MQ_TYPE_Q6_K)
            return hipErrorInvalidValue;
        const ActPlanes ap = act_planes(a.q_type, rows, K, true);
        if (ap.kb_pad != K || a.o_st != K || a.o_sh != a.hd || a.o_sb != a.Tq * K || ((uintptr_t)a.q_ws & 255))
            return hipErrorInvalidValue;
        if (attn_frag_form(a, a.q_type)) {
            b.qo = (int8_t *)((uint8_t *)a.q_ws + ap.xq);
            b.qd = (float *)((uint8_t *)a.q_ws + ap.xd);
            b.qmin = a.q_type == MQ_TYPE_Q8_0 ? nullptr : (_Float16 *)((uint8_t *)a.q_ws + ap.xmin);
            b.q_m_pad = ap.m_pad;
            b.q_kch = (int)(K / 32);
            b.q_nsb = (int)(K / QK_K);
        } else {
            quant_after = true;  // the Q8_K store needs the 8-wave form
        }
    }
    hipError_t e;
    switch (b.hd) {
        case 128: e = launch_attn_hd<128>(b, nblk, qscale, s); break;
        case 64: e = launch_attn_hd<64>(b, nblk, qscale, s); break;
        case 32: e = launch_attn_hd<32>(b, nblk, qscale, s); break;
        default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
    if (quant_after) {
        const int64_t rows = (int64_t)a.B * a.Tq, K = (int64_t)a.nq * a.hd;
        return launch_quantize_act_planar(a.q_type, a.out, K, a.q_ws, rows, K, a.q_var, true, s);
    }
    return hipGetLastError();
}

// The fused q|k|v rows of the decoder (row stride ld floats: nq query heads, then nkv key
// heads, then nkv value heads, hd floats each) as strided operands.
hipError_t launch_attn_frag(const float *qkv, int64_t ld, float *out, int64_t ldo, int B, int T, int nq, int nkv,
                            int hd, float scale, int causal, const float *qw, const float *kw, float eps,
                            const float2 *cs, void *ws, hipStream_t s, void *q_ws, int q_type, bool q_only) {
    AttnArgs a;
    a.q = qkv;
    a.k = qkv + (int64_t)nq * hd;
    a.v = qkv + (int64_t)(nq + nkv) * hd;
    a.q_sb = a.k_sb = a.v_sb = (int64_t)T * ld;
    a.q_st = a.k_st = a.v_st = ld;
    a.q_sh = a.k_sh = a.v_sh = hd;
    a.out = out;
    a.o_sb = (int64_t)T * ldo, a.o_st = ldo, a.o_sh = hd;
    a.B = B, a.Tq = a.Tk = T, a.nq = nq, a.nkv = nkv, a.hd = hd;
    a.scale = scale, a.causal = causal, a.qw = qw, a.kw = kw, a.eps = eps, a.cs = cs, a.ws = ws;
    a.q_ws = q_ws, a.q_type = q_type, a.q_only = q_only, a.q_var = mq_q8_0_variant();
    return launch_attn(a, s);
}

hipError_t launch_last_rmsnorm_l2(const float *x, const float *w, float eps, float *out, int B, int T, int H,
                                  hipStream_t s) {
    if (B <= 0) return hipSuccess;
    MQ_RMS_DISPATCH(k_last_rmsnorm_l2, dim3((unsigned)B), dim3(64), x, w, eps, out, T, H);
    return hipGetLastError();
}
#undef MQ_RMS_DISPATCH

}  // namespace mq
