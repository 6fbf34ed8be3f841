// mq_encoder.hip -- the non-MUL_MAT ops of a post-LN BERT encoder on gfx950, in fp32.
//
// CrispEmbed's encoder graph (src/crispembed.cpp:1043-1468) around the mul_mats:
//   embeddings   GET_ROWS(token) + GET_ROWS(pos) + GET_ROWS(type), NORM, MUL, ADD
//   attention    ADD(bias) on q/k/v, FLASH_ATTN_EXT(scale 1/sqrt(head_dim), no mask
//                for full-length sequences), the heads concatenated back to [H, T]
//   residual     ADD(bias), ADD(residual), NORM(eps), MUL(w), ADD(b)   (post-LN)
//   FFN          ADD(bias), GELU_ERF
//   pooling      mean over the sequence, L2 normalised with sqrtf(max(sum x^2, 1e-12))
//                (pool_and_norm, src/crispembed.cpp:2024-2045)
// Each group is one kernel here (fused): the data stays in registers/LDS between ops.
// All arithmetic is fp32; NORM follows ggml's two-pass mean / variance form.
#include "mq_internal.h"
#include "mq_wave.h"

namespace mq {

constexpr int LN_MAXV = 16;  // values per lane: rows up to 1024 wide

// One wave per row: y = (x - mean) / sqrt(var + eps) * w + b, x held in registers
// (V values per lane, rows up to 64*V wide).
template <int V>
__device__ __forceinline__ void ln_row(float (&v)[V], int n, int lane, const float *w, const float *b, float eps,
                                       float *out) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < V; i++)
        if (lane + 64 * i < n) s += v[i];
    const float mean = wave_sum_f(s) / (float)n;
    float s2 = 0.f;
#pragma unroll
    for (int i = 0; i < V; i++)
        if (lane + 64 * i < n) {
            v[i] -= mean;
            s2 += v[i] * v[i];
        }
    const float rstd = 1.0f / sqrtf(wave_sum_f(s2) / (float)n + eps);
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int c = lane + 64 * i;
        if (c < n) out[c] = v[i] * rstd * w[c] + b[c];
    }
}

template <int V>
__global__ __launch_bounds__(256) void k_embed_ln(const int32_t *__restrict__ ids, const int32_t *__restrict__ types,
                                                  const float *__restrict__ word, const float *__restrict__ pos,
                                                  const float *__restrict__ type, const float *__restrict__ lw,
                                                  const float *__restrict__ lb, float eps, float *__restrict__ out,
                                                  int64_t rows, int T, int H, int n_vocab, int n_type) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    // ids outside the tables are clamped: a bad id reads a valid row, never out of bounds
    const int64_t id = min(max(ids[row], 0), n_vocab - 1);
    const int p = (int)(row % T);
    const int64_t ty = types ? min(max(types[row], 0), max(n_type, 1) - 1) : 0;
    float v[V];
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int c = lane + 64 * i;
        v[i] = 0.f;
        if (c < H) {
            float x = word[id * H + c];
            if (pos) x += pos[(int64_t)p * H + c];
            if (type) x += type[ty * H + c];
            v[i] = x;
        }
    }
    ln_row(v, H, lane, lw, lb, eps, out + row * H);
}

// out = LN(y + bias + res) * w + b   (out may alias res)
template <int V>
__global__ __launch_bounds__(256) void k_bias_res_ln(const float *__restrict__ y, const float *__restrict__ bias,
                                                     const float *res, const float *__restrict__ lw,
                                                     const float *__restrict__ lb, float eps, float *out, int64_t rows,
                                                     int H) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    float v[V];
#pragma unroll
    for (int i = 0; i < V; i++) {
        const int c = lane + 64 * i;
        v[i] = 0.f;
        if (c < H) v[i] = res[row * H + c] + (y[row * H + c] + (bias ? bias[c] : 0.f));
    }
    ln_row(v, H, lane, lw, lb, eps, out + row * H);
}

// Attention of one (sequence, head): qkv rows [T][3H] (q | k | v, bias not yet added),
// out rows [T][H] at this head's columns.  K and V of the head sit in LDS.  Thread t takes
// query row t % T and the t / T-th of KS equal key ranges, walks its keys in blocks of
// ATT_KB with an online softmax (running max, rescaled sum and output; all threads of a
// wave read the same K / V row at a time, an LDS broadcast), then the KS partial states of
// each row are merged through LDS (the K / V space, free by then):
//   m = max m_s,  l = sum l_s e^(m_s - m),  o = sum o_s e^(m_s - m) / l.
constexpr int ATT_KB = 16;
template <int HD, int KS>
__global__ __launch_bounds__(512) void k_attention(const float *__restrict__ qkv, const float *__restrict__ bqkv,
                                                   float *__restrict__ out, int T, int H, int nh, float scale) {
    extern __shared__ float sm[];
    const int b = blockIdx.x / nh, h = blockIdx.x % nh;
    float *Ks = sm;               // [T][HD]
    float *Vs = Ks + T * HD;      // [T][HD]
    const int64_t ld = 3 * (int64_t)H;
    const float *base = qkv + (int64_t)b * T * ld;
    for (int e = threadIdx.x; e < T * HD; e += blockDim.x) {
        const int j = e / HD, d = e % HD;
        Ks[e] = base[j * ld + H + h * HD + d] + bqkv[H + h * HD + d];
        Vs[e] = base[j * ld + 2 * H + h * HD + d] + bqkv[2 * H + h * HD + d];
    }
    __syncthreads();
    const int i = threadIdx.x % T, ks = threadIdx.x / T;
    const int span = T / KS, j_lo = ks * span, j_hi = j_lo + span;
    float q[HD], o[HD];
    const float4 *qr = (const float4 *)(base + i * ld + h * HD);
    const float4 *qb = (const float4 *)(bqkv + h * HD);
#pragma unroll
    for (int d4 = 0; d4 < HD / 4; d4++) {
        const float4 a4 = qr[d4], b4 = qb[d4];
        q[4 * d4] = (a4.x + b4.x) * scale;
        q[4 * d4 + 1] = (a4.y + b4.y) * scale;
        q[4 * d4 + 2] = (a4.z + b4.z) * scale;
        q[4 * d4 + 3] = (a4.w + b4.w) * scale;
        o[4 * d4] = o[4 * d4 + 1] = o[4 * d4 + 2] = o[4 * d4 + 3] = 0.f;
    }
    float mx = -INFINITY, l = 0.f;
    for (int j0 = j_lo; j0 < j_hi; j0 += ATT_KB) {
        const int nk = min(ATT_KB, j_hi - j0);
        float sc[ATT_KB];
        float bm = -INFINITY;
#pragma unroll
        for (int jj = 0; jj < ATT_KB; jj++) {
            sc[jj] = -INFINITY;
            if (jj < nk) {
                const float4 *kr = (const float4 *)(Ks + (j0 + jj) * HD);
                float sv = 0.f;
#pragma unroll
                for (int d4 = 0; d4 < HD / 4; d4++) {
                    const float4 kv = kr[d4];
                    sv += q[4 * d4] * kv.x + q[4 * d4 + 1] * kv.y + q[4 * d4 + 2] * kv.z + q[4 * d4 + 3] * kv.w;
                }
                sc[jj] = sv;
                bm = fmaxf(bm, sv);
            }
        }
        const float mnew = fmaxf(mx, bm);
        const float corr = expf(mx - mnew);  // 0 on the first block (mx = -inf)
        l *= corr;
#pragma unroll
        for (int d = 0; d < HD; d++) o[d] *= corr;
        mx = mnew;
#pragma unroll
        for (int jj = 0; jj < ATT_KB; jj++) {
            if (jj < nk) {
                const float p = expf(sc[jj] - mx);
                l += p;
                const float4 *vr = (const float4 *)(Vs + (j0 + jj) * HD);
#pragma unroll
                for (int d4 = 0; d4 < HD / 4; d4++) {
                    const float4 vv = vr[d4];
                    o[4 * d4] += p * vv.x;
                    o[4 * d4 + 1] += p * vv.y;
                    o[4 * d4 + 2] += p * vv.z;
                    o[4 * d4 + 3] += p * vv.w;
                }
            }
        }
    }
    float4 *orow = (float4 *)(out + ((int64_t)b * T + i) * H + h * HD);
    if constexpr (KS == 1) {
        const float inv = 1.0f / l;
#pragma unroll
        for (int d4 = 0; d4 < HD / 4; d4++)
            orow[d4] = make_float4(o[4 * d4] * inv, o[4 * d4 + 1] * inv, o[4 * d4 + 2] * inv, o[4 * d4 + 3] * inv);
    } else {
        __syncthreads();  // every thread is done with K / V: reuse the space for partial states
        float *st = sm + (int64_t)((ks - 1) * T + i) * (HD + 2);  // [KS-1][T][HD+2]
        if (ks > 0) {
            st[0] = mx;
            st[1] = l;
#pragma unroll
            for (int d = 0; d < HD; d++) st[2 + d] = o[d];
        }
        __syncthreads();
        if (ks == 0) {
            float m = mx;
#pragma unroll
            for (int k = 1; k < KS; k++) m = fmaxf(m, sm[(int64_t)((k - 1) * T + i) * (HD + 2)]);
            float w0 = expf(mx - m), lt = l * w0;
#pragma unroll
            for (int d = 0; d < HD; d++) o[d] *= w0;
#pragma unroll
            for (int k = 1; k < KS; k++) {
                const float *sk = sm + (int64_t)((k - 1) * T + i) * (HD + 2);
                const float w = expf(sk[0] - m);
                lt += sk[1] * w;
#pragma unroll
                for (int d = 0; d < HD; d++) o[d] += sk[2 + d] * w;
            }
            const float inv = 1.0f / lt;
#pragma unroll
            for (int d4 = 0; d4 < HD / 4; d4++)
                orow[d4] = make_float4(o[4 * d4] * inv, o[4 * d4 + 1] * inv, o[4 * d4 + 2] * inv, o[4 * d4 + 3] * inv);
        }
    }
}

// Mean over each sequence's T rows, then v / sqrt(max(sum v^2, 1e-12)): the 16 waves of a
// workgroup split the rows (loads of 4 rows in flight per wave), lanes the columns; the
// partial sums meet in LDS.
constexpr int POOL_MAXC = 16;  // columns per lane: H up to 1024
constexpr int POOL_WAVES = 16;
__global__ __launch_bounds__(64 * POOL_WAVES) void k_mean_pool_l2(const float *__restrict__ x, float *__restrict__ out,
                                                                  int T, int H) {
    __shared__ float part[POOL_WAVES][512];
    __shared__ float sq[POOL_WAVES];
    const int b = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int c0 = 0; c0 < H; c0 += 512) {  // column chunks of 512 (8 per lane)
        float acc[8];
#pragma unroll
        for (int i = 0; i < 8; i++) acc[i] = 0.f;
        int t = wave;
        for (; t + 3 * POOL_WAVES < T; t += 4 * POOL_WAVES) {
            float v[4][8];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float *row = x + ((int64_t)b * T + t + u * POOL_WAVES) * H + c0;
#pragma unroll
                for (int i = 0; i < 8; i++) v[u][i] = (c0 + lane + 64 * i < H) ? row[lane + 64 * i] : 0.f;
            }
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int i = 0; i < 8; i++) acc[i] += v[u][i];
        }
        for (; t < T; t += POOL_WAVES) {
            const float *row = x + ((int64_t)b * T + t) * H + c0;
#pragma unroll
            for (int i = 0; i < 8; i++)
                if (c0 + lane + 64 * i < H) acc[i] += row[lane + 64 * i];
        }
#pragma unroll
        for (int i = 0; i < 8; i++) part[wave][lane + 64 * i] = acc[i];
        __syncthreads();
        for (int c = threadIdx.x; c < 512 && c0 + c < H; c += blockDim.x) {
            float sum = 0.f;
#pragma unroll
            for (int w = 0; w < POOL_WAVES; w++) sum += part[w][c];
            out[(int64_t)b * H + c0 + c] = sum / (float)T;
        }
        __syncthreads();
    }
    float ss = 0.f;
    for (int c = threadIdx.x; c < H; c += blockDim.x) {
        const float v = out[(int64_t)b * H + c];
        ss += v * v;
    }
    ss = wave_sum_f(ss);
    if (lane == 0) sq[wave] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < POOL_WAVES; w++) tot += sq[w];
    const float norm = sqrtf(fmaxf(tot, 1e-12f));
    for (int c = threadIdx.x; c < H; c += blockDim.x) out[(int64_t)b * H + c] /= norm;
}

// LDS of k_attention: K and V of one head, or (after the key loops) the KS-1 partial states
size_t attention_lds_bytes(int T, int hd, int ks) {
    const size_t kv = 2 * (size_t)T * hd, st = (size_t)(ks - 1) * T * (hd + 2);
    return sizeof(float) * (kv > st ? kv : st);
}

// V (values per lane) from the row width: the register arrays stay as small as the row.
#define MQ_LN_DISPATCH(KERNEL, ...)                                                                          \
    do {                                                                                                     \
        const dim3 g((unsigned)((rows + 3) / 4)), b(256);                                                   \
        if (H <= 128) hipLaunchKernelGGL(KERNEL<2>, g, b, 0, s, __VA_ARGS__);                                 \
        else if (H <= 256) hipLaunchKernelGGL(KERNEL<4>, g, b, 0, s, __VA_ARGS__);                            \
        else if (H <= 384) hipLaunchKernelGGL(KERNEL<6>, g, b, 0, s, __VA_ARGS__);                            \
        else if (H <= 512) hipLaunchKernelGGL(KERNEL<8>, g, b, 0, s, __VA_ARGS__);                            \
        else if (H <= 768) hipLaunchKernelGGL(KERNEL<12>, g, b, 0, s, __VA_ARGS__);                           \
        else hipLaunchKernelGGL(KERNEL<16>, g, b, 0, s, __VA_ARGS__);                                         \
    } while (0)

hipError_t launch_embed_ln(const int32_t *ids, const int32_t *types, const float *word, const float *pos,
                           const float *type, const float *lw, const float *lb, float eps, float *out, int64_t rows,
                           int T, int H, int n_vocab, int n_type, hipStream_t s) {
    if (H > 64 * LN_MAXV || T <= 0 || n_vocab <= 0) return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    MQ_LN_DISPATCH(k_embed_ln, ids, types, word, pos, type, lw, lb, eps, out, rows, T, H, n_vocab, n_type);
    return hipGetLastError();
}

hipError_t launch_bias_res_ln(const float *y, const float *bias, const float *res, const float *lw, const float *lb,
                              float eps, float *out, int64_t rows, int H, hipStream_t s) {
    if (H > 64 * LN_MAXV) return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    MQ_LN_DISPATCH(k_bias_res_ln, y, bias, res, lw, lb, eps, out, rows, H);
    return hipGetLastError();
}
#undef MQ_LN_DISPATCH

template <int HD, int KS>
static hipError_t attention_cfg(const float *qkv, const float *bqkv, float *out, int B, int T, int H, int nh,
                                hipStream_t s) {
    static std::atomic<bool> attr_set[MQ_MAX_DEVICES];
    const hipError_t e = dyn_lds_once((const void *)k_attention<HD, KS>, 160 * 1024, attr_set);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((k_attention<HD, KS>), dim3((unsigned)(B * nh)), dim3(T * KS), attention_lds_bytes(T, HD, KS), s,
                       qkv, bqkv, out, T, H, nh, 1.0f / sqrtf((float)HD));
    return hipGetLastError();
}

template <int HD>
static hipError_t attention_hd(const float *qkv, const float *bqkv, float *out, int B, int T, int H, int nh,
                               hipStream_t s) {
    // KS key ranges per row: the largest of 4, 2, 1 that keeps T*KS <= 512 threads and
    // divides T into equal ranges
    if (T * 4 <= 512 && T % 4 == 0) return attention_cfg<HD, 4>(qkv, bqkv, out, B, T, H, nh, s);
    if (T * 2 <= 512 && T % 2 == 0) return attention_cfg<HD, 2>(qkv, bqkv, out, B, T, H, nh, s);
    if (T <= 512) return attention_cfg<HD, 1>(qkv, bqkv, out, B, T, H, nh, s);
    return hipErrorInvalidValue;
}

hipError_t launch_attention(const float *qkv, const float *bqkv, float *out, int B, int T, int H, int nh,
                            hipStream_t s) {
    if (nh <= 0 || H % nh != 0 || T <= 0 || T > 512) return hipErrorInvalidValue;
    const int hd = H / nh;
    if (attention_lds_bytes(T, hd, 4) > 160 * 1024) return hipErrorInvalidValue;
    if (((uintptr_t)qkv | (uintptr_t)bqkv | (uintptr_t)out) % 16 != 0 || H % 4 != 0) return hipErrorInvalidValue;
    switch (hd) {
        case 32: return attention_hd<32>(qkv, bqkv, out, B, T, H, nh, s);
        case 64: return attention_hd<64>(qkv, bqkv, out, B, T, H, nh, s);
        default: return hipErrorInvalidValue;  // head_dim 32 or 64 (BERT / XLM-R families)
    }
}

hipError_t launch_mean_pool_l2(const float *x, float *out, int B, int T, int H, hipStream_t s) {
    if (H > 64 * POOL_MAXC) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_mean_pool_l2, dim3((unsigned)B), dim3(64 * POOL_WAVES), 0, s, x, out, T, H);
    return hipGetLastError();
}

}  // namespace mq
