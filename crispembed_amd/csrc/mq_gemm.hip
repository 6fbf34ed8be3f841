// mq_gemm.hip -- batched-token MFMA GEMM for GGML_OP_MUL_MAT on gfx950.
//
// Y[m][n] = sum_k X[m][k] * W[n][k], X requantized to ggml's vec_dot_type.
//
// Integer formats run v_mfma_i32_32x32x32_i8 with K = 32 per instruction:
//   Q8_0  one Q8_0 block per MFMA; the int32 block dot is scaled in fp32 by
//         d_x * d_w right after the block (ggml_vec_dot_q8_0_q8_0 semantics).
//   Q4_K  the weight plane holds sc_j*q4 (10 bits) split into two int8 limbs,
//         lo in [0,127] and hi in [0,7] (value = lo + 128*hi), prepared once at
//         load.  Two int32 accumulators run over a whole 256-value superblock, so
//         the 6-bit sub-block scales cost no per-sub-block VALU work; the exact
//         integer sum_j sc_j * sum q4*q8 is lo + (hi << 7).  The min term
//         sum_j m_j * bsum32_j is one v_mfma_f32_32x32x16_f16 per superblock whose
//         operands (m_j <= 63; bsum32 split as (B & 63) + 64*(B >> 6)) are exact in
//         fp16 and whose fp32 sums stay below 2^24, i.e. exact.  Then per
//         superblock: acc += d_x * (d_w * I - dmin_w * Imin) in fp32.
//   Q6_K  sc*(q6-32) (13 bits signed) in two limbs, same scheme, no min term.
// F16 runs v_mfma_f32_32x32x16_f16 on fp16 activations (ggml converts X to fp16).
//
// Tiling: 256 threads = 4 waves in a 2x2 grid, each wave 64x64 outputs = 2x2
// MFMA tiles; workgroup tile 128 tokens x 128 features; K staged 128 bytes at a
// time through LDS with a 144-byte row pitch (ds_read_b128 conflict-free).
// MFMA operand mapping: lane l feeds row (l % 32) of its tile with the 16 bytes
// at offset 16*(l / 32) of each 32-byte K chunk, identically for both operands,
// so the dot runs over exactly that chunk whatever byte order the unit uses.
// Output mapping of a 32x32 MFMA: register r of lane l holds
// row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#include "mq_internal.h"

namespace mq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

enum { FMT_Q8_0 = 0, FMT_Q4_K = 1, FMT_Q6_K = 2, FMT_F16 = 3 };

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int KT = 128;             // bytes of K per LDS stage
constexpr int PITCH = KT + 16;      // LDS row pitch in bytes
constexpr int NTHREADS = 256;

struct GemmArgs {
    const int8_t *xq;     // activation plane: int8 [M][K] or fp16 [M][K]
    const float *xd;      // Q8_0: [M][K/32]; K-quants: [M][K/256]
    const int16_t *xbs;   // Q4_K: ggml bsums [M][K/16]
    const int8_t *wlo;    // weight plane / lo limb
    const int8_t *whi;    // hi limb
    const float *wd;      // K-quants: d per superblock [N][K/256]
    const float *wdmin;   // Q4_K: dmin per superblock
    const _Float16 *wmins;  // Q4_K: m_j [N][K/256][8]
    const uint16_t *wd16;   // Q8_0: fp16 d [N][K/32]
    float *y;
    int M, N, K, ldy;
};

template <int FMT>
struct Smem {
    static constexpr bool limbs = (FMT == FMT_Q4_K || FMT == FMT_Q6_K);
    alignas(16) int8_t xs[BM * PITCH];
    alignas(16) int8_t ws[BN * PITCH];
    alignas(16) int8_t wh[limbs ? BN * PITCH : 16];
    // Q8_0: 4 blocks per stage [4][rows]; K-quants: one superblock [rows]
    alignas(16) float xd[FMT == FMT_Q8_0 ? 4 * BM : BM];
    alignas(16) float wd[FMT == FMT_Q8_0 ? 4 * BN : BN];
    alignas(16) float wdmin[FMT == FMT_Q4_K ? BN : 4];
    alignas(16) _Float16 xmin[FMT == FMT_Q4_K ? BM * 16 : 8];
    alignas(16) _Float16 wmin[FMT == FMT_Q4_K ? BN * 8 : 8];
};

__device__ __forceinline__ void load_tile(const int8_t *__restrict__ base, int64_t rowbytes, int row0, int nrows,
                                          int8_t *lds, int64_t kb0, int tid) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int c = tid + NTHREADS * i;
        const int r = c >> 3, cc = c & 7;
        const int64_t grow = min(row0 + r, nrows - 1);  // clamp: tail rows are computed, never stored
        const int64_t kb = kb0 + cc * 16;
        v4i v = {0, 0, 0, 0};
        if (kb < rowbytes) v = *(const v4i *)(base + grow * rowbytes + kb);
        *(v4i *)(lds + r * PITCH + cc * 16) = v;
    }
}

template <int FMT>
__global__ __launch_bounds__(NTHREADS, (FMT == FMT_Q4_K || FMT == FMT_Q6_K) ? 1 : 2) void k_gemm(const GemmArgs a) {
    __shared__ Smem<FMT> sm;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int n0 = blockIdx.x * BN;
    const int m0 = blockIdx.y * BM;
    const int lrow = lane & 31;   // tile row/col this lane feeds
    const int lhalf = lane >> 5;  // which 16-byte half of a 32-byte K chunk
    const int64_t rowbytes = (FMT == FMT_F16) ? 2 * (int64_t)a.K : (int64_t)a.K;
    const int nstages = (int)((rowbytes + KT - 1) / KT);

    v16f acc[2][2];
    v16i alo[2][2], ahi[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            acc[i][j] = (v16f){};
            alo[i][j] = (v16i){};
            ahi[i][j] = (v16i){};
        }

    for (int st = 0; st < nstages; st++) {
        const int64_t kb0 = (int64_t)st * KT;
        __syncthreads();
        load_tile(a.xq, rowbytes, m0, a.M, sm.xs, kb0, tid);
        load_tile(a.wlo, rowbytes, n0, a.N, sm.ws, kb0, tid);
        if constexpr (Smem<FMT>::limbs) load_tile(a.whi, rowbytes, n0, a.N, sm.wh, kb0, tid);
        if constexpr (FMT == FMT_Q8_0) {
            const int nbr = a.K / QK8_0;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int c = tid + NTHREADS * i;  // 512 = 4 blocks x 128 rows
                const int r = c & 127, bb = c >> 7;
                const int blk = st * 4 + bb;
                const int xr = min(m0 + r, a.M - 1), wr = min(n0 + r, a.N - 1);
                float xv = 0.f, wv = 0.f;
                if (blk < nbr) {
                    xv = a.xd[(int64_t)xr * nbr + blk];
                    wv = (float)__builtin_bit_cast(_Float16, a.wd16[(int64_t)wr * nbr + blk]);
                }
                sm.xd[bb * BM + r] = xv;
                sm.wd[bb * BN + r] = wv;
            }
        } else if constexpr (Smem<FMT>::limbs) {
            if ((st & 1) == 0) {
                const int nsb = a.K / QK_K, sb = st >> 1;
                if (tid < BM) {
                    const int xr = min(m0 + tid, a.M - 1), wr = min(n0 + tid, a.N - 1);
                    sm.xd[tid] = a.xd[(int64_t)xr * nsb + sb];
                    sm.wd[tid] = a.wd[(int64_t)wr * nsb + sb];
                    if constexpr (FMT == FMT_Q4_K) {
                        sm.wdmin[tid] = a.wdmin[(int64_t)wr * nsb + sb];
                        const v8h mv = *(const v8h *)(a.wmins + ((int64_t)wr * nsb + sb) * 8);
                        *(v8h *)(sm.wmin + tid * 8) = mv;
                    }
                } else if constexpr (FMT == FMT_Q4_K) {
                    // min-term operand: per row, bsum32_j split into exact fp16 limbs
                    const int r = tid - BM;
                    const int xr = min(m0 + r, a.M - 1);
                    const int16_t *bs = a.xbs + (int64_t)xr * (a.K / 16) + sb * 16;
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        const int B = bs[2 * j] + bs[2 * j + 1];
                        sm.xmin[r * 16 + j] = (_Float16)(B & 63);
                        sm.xmin[r * 16 + 8 + j] = (_Float16)((B >> 6) * 64);
                    }
                }
            }
        }
        __syncthreads();

#pragma unroll
        for (int kc = 0; kc < KT / 32; kc++) {
            const int koff = kc * 32 + lhalf * 16;
            v4i xa[2], wb[2], wbh[2];
#pragma unroll
            for (int i = 0; i < 2; i++) xa[i] = *(const v4i *)(sm.xs + (wm * 64 + i * 32 + lrow) * PITCH + koff);
#pragma unroll
            for (int j = 0; j < 2; j++) {
                wb[j] = *(const v4i *)(sm.ws + (wn * 64 + j * 32 + lrow) * PITCH + koff);
                if constexpr (Smem<FMT>::limbs) wbh[j] = *(const v4i *)(sm.wh + (wn * 64 + j * 32 + lrow) * PITCH + koff);
            }
            if constexpr (FMT == FMT_F16) {
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, xa[i]),
                                                                          __builtin_bit_cast(v8h, wb[j]), acc[i][j],
                                                                          0, 0, 0);
            } else if constexpr (FMT == FMT_Q8_0) {
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const float dw = sm.wd[kc * BN + wn * 64 + j * 32 + lrow];
#pragma unroll
                    for (int i = 0; i < 2; i++) {
                        const v16i t = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa[i], wb[j], (v16i){}, 0, 0, 0);
#pragma unroll
                        for (int g = 0; g < 4; g++) {
                            const float4 dx4 =
                                *(const float4 *)(sm.xd + kc * BM + wm * 64 + i * 32 + 8 * g + 4 * lhalf);
                            acc[i][j][4 * g + 0] += (float)t[4 * g + 0] * (dx4.x * dw);
                            acc[i][j][4 * g + 1] += (float)t[4 * g + 1] * (dx4.y * dw);
                            acc[i][j][4 * g + 2] += (float)t[4 * g + 2] * (dx4.z * dw);
                            acc[i][j][4 * g + 3] += (float)t[4 * g + 3] * (dx4.w * dw);
                        }
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        alo[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa[i], wb[j], alo[i][j], 0, 0, 0);
                        ahi[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa[i], wbh[j], ahi[i][j], 0, 0, 0);
                    }
            }
        }

        if constexpr (Smem<FMT>::limbs) {
            if (st & 1) {
                // superblock complete: scale and fold into the fp32 accumulators
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int wc = wn * 64 + j * 32 + lrow;
                    const float dw = sm.wd[wc];
                    float dmn = 0.f;
                    v8h bmin = {};
                    if constexpr (FMT == FMT_Q4_K) {
                        dmn = sm.wdmin[wc];
                        bmin = *(const v8h *)(sm.wmin + wc * 8);
                    }
#pragma unroll
                    for (int i = 0; i < 2; i++) {
                        v16f fmin = {};
                        if constexpr (FMT == FMT_Q4_K) {
                            const v8h amin = *(const v8h *)(sm.xmin + (wm * 64 + i * 32 + lrow) * 16 + lhalf * 8);
                            fmin = __builtin_amdgcn_mfma_f32_32x32x16_f16(amin, bmin, (v16f){}, 0, 0, 0);
                        }
#pragma unroll
                        for (int g = 0; g < 4; g++) {
                            const float4 dx4 = *(const float4 *)(sm.xd + wm * 64 + i * 32 + 8 * g + 4 * lhalf);
                            const float dxs[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
#pragma unroll
                            for (int q = 0; q < 4; q++) {
                                const int r = 4 * g + q;
                                const int isum = alo[i][j][r] + (ahi[i][j][r] << 7);
                                float t = dw * (float)isum;
                                if constexpr (FMT == FMT_Q4_K) t -= dmn * fmin[r];
                                acc[i][j][r] += dxs[q] * t;
                            }
                        }
                        alo[i][j] = (v16i){};
                        ahi[i][j] = (v16i){};
                    }
                }
            }
        }
    }

    // store: lanes 0..31 of a register write 32 consecutive floats of one row
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int col = n0 + wn * 64 + j * 32 + lrow;
            if (col >= a.N) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lhalf + (r & 3);
                if (row < a.M) a.y[(int64_t)row * a.ldy + col] = acc[i][j][r];
            }
        }
}

hipError_t launch_gemm(int type, const void *image, int64_t n, int64_t k, const void *ws, int64_t m, float *y,
                       int64_t ldy, hipStream_t s) {
    if (m <= 0 || n <= 0) return hipSuccess;
    const WeightPlanes p = weight_planes(type, n, k);
    const ActPlanes ap = act_planes(type, m, k);
    const uint8_t *wb = (const uint8_t *)image;
    const uint8_t *xb = (const uint8_t *)ws;
    GemmArgs a{};
    a.xq = (const int8_t *)(xb + ap.xq);
    a.xd = (const float *)(xb + ap.xd);
    a.xbs = (const int16_t *)(xb + ap.xbs);
    a.y = y;
    a.M = (int)m;
    a.N = (int)n;
    a.K = (int)k;
    a.ldy = (int)ldy;
    const dim3 grid((unsigned)((n + BN - 1) / BN), (unsigned)((m + BM - 1) / BM));
    const dim3 block(NTHREADS);
    switch (type) {
        case MQ_TYPE_Q8_0:
            a.wlo = (const int8_t *)(wb + p.qs);
            a.wd16 = (const uint16_t *)(wb + p.d16);
            hipLaunchKernelGGL(k_gemm<FMT_Q8_0>, grid, block, 0, s, a);
            break;
        case MQ_TYPE_Q4_K:
            a.wlo = (const int8_t *)(wb + p.qs);
            a.whi = (const int8_t *)(wb + p.hi);
            a.wd = (const float *)(wb + p.dw);
            a.wdmin = (const float *)(wb + p.dmin);
            a.wmins = (const _Float16 *)(wb + p.mins);
            hipLaunchKernelGGL(k_gemm<FMT_Q4_K>, grid, block, 0, s, a);
            break;
        case MQ_TYPE_Q6_K:
            a.wlo = (const int8_t *)(wb + p.qs);
            a.whi = (const int8_t *)(wb + p.hi);
            a.wd = (const float *)(wb + p.dw);
            hipLaunchKernelGGL(k_gemm<FMT_Q6_K>, grid, block, 0, s, a);
            break;
        case MQ_TYPE_F16:
            a.wlo = (const int8_t *)wb;  // GGUF F16 rows
            hipLaunchKernelGGL(k_gemm<FMT_F16>, grid, block, 0, s, a);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mq
