// mq_gemm.hip -- batched-token MFMA GEMM for GGML_OP_MUL_MAT on gfx950.
//
// Y[m][n] = sum_k X[m][k] * W[n][k], X requantized to ggml's vec_dot_type.
//
// Arithmetic (exact integer block dots, fp32 scales, as ggml_vec_dot_*):
//   Q8_0  v_mfma_i32_32x32x32_i8, one Q8_0 block (K = 32) per MFMA; the int32
//         block dot is scaled by d_x * d_w in fp32 right after the block.
//   Q4_K  the weight operand is sc_j*q4 (10 bits) split at load time into two
//         int8 limbs, lo in [0,127] and hi in [0,7] (value = lo + 128*hi).  Two
//         int32 accumulators run over a whole 256-value superblock, so the 6-bit
//         sub-block scales cost no per-sub-block VALU work, and the exact integer
//         sum_j sc_j * sum(q4*q8) is lo + (hi << 7).  The min term
//         sum_j m_j * B_j (B_j = sum of the 32 activation quants of sub-block j) is
//         one v_mfma_f32_32x32x16_f16 per superblock: m_j <= 63 and B_j split as
//         (B_j & 63) + 64*(B_j >> 6) are exact in fp16, every product and partial
//         sum stays below 2^24, so the fp32 result is exact.  Per superblock:
//         acc += d_x * (d_w * I - dmin_w * Imin) in fp32.
//   Q6_K  sc*(q6-32) (13 bits signed) in two limbs, same scheme, no min term.
//   F16   v_mfma_f32_32x32x16_f16 on fp16 activations (ggml's F16 vec_dot_type).
//
// Data movement: both operands sit in HBM in the tiled layout (1 KB fragments, see
// mq_internal.h), written by the activation quantizer and by the weight
// preparation at load.  Each wave moves whole fragments global -> LDS with
// global_load_lds_dwordx4 (no register staging); MFMA operands are read back
// with one ds_read_b128 per lane at lane*16 (bank-conflict free).  K advances
// 128 bytes per stage; stages are double-buffered so the DMA of stage s+1
// overlaps the MFMAs of stage s.  The superblock epilogue operands (scales and
// min-term fragments) ride along with the even stage into their own
// double-buffered LDS region.
//
// Tiling: WM x WN waves, each wave 64x64 outputs = 2x2 MFMA tiles (rows: tokens,
// columns: output features).  WG tile 256x128 (8 waves, one WG per CU, 2 waves
// per SIMD) or 128x128 (4 waves) for small grids.  Work-group order: consecutive
// workgroup ids go round-robin over the 8 XCDs, so ids are remapped to give each
// XCD a contiguous range of tiles, walked in groups of GROUP_M token tiles x all
// feature tiles, keeping each XCD's working set inside its 4 MB L2.
// Output mapping of a 32x32 MFMA: register r of lane l holds
// row 8*(r/4) + 4*(l/32) + r%4, column l%32.
#include "mq_internal.h"

namespace mq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_void;

enum { FMT_Q8_0 = 0, FMT_Q4_K = 1, FMT_Q6_K = 2, FMT_F16 = 3 };

struct GemmArgs {
    const int8_t *xq;       // tiled activations
    const float *xd;        // activation scales [blocks or superblocks][m_pad]
    const _Float16 *xmin;   // Q4_K: activation min-term fragments
    const int8_t *wq;       // tiled weights / lo limb
    const int8_t *whi;      // hi limb
    const float *wd;        // weight scales [blocks or superblocks][n_pad]
    const float *wdmin;     // Q4_K
    const _Float16 *wmin;   // Q4_K: weight min-term fragments
    float *y;
    int M, N, ldy;
    int m_pad, n_pad;
    int kch;      // 32-byte K chunks per row (kb_pad / 32)
    int nstages;  // kb_pad / 128
    int nsb;      // K / 256
    int tiles_m, tiles_n, group_m;
};

// WM x WN waves per workgroup, each wave TM x TN MFMA tiles of 32x32.
template <int FMT, int WM, int WN, int TM, int TN>
struct Cfg {
    static constexpr int NW = WM * WN, NT = 64 * NW, BM = 32 * TM * WM, BN = 32 * TN * WN;
    static constexpr bool limbs = (FMT == FMT_Q4_K || FMT == FMT_Q6_K);
    static constexpr int NPL = limbs ? 2 : 1;
    static constexpr int XF = (BM / 32) * 4, WF = (BN / 32) * 4;  // fragments per stage
    static constexpr int X_BYTES = XF * 1024, W_BYTES = WF * 1024;
    static constexpr int SCX = (FMT == FMT_Q8_0) ? 4 * BM * 4 : 0;
    static constexpr int SCW = (FMT == FMT_Q8_0) ? 4 * BN * 4 : 0;
    static constexpr int STAGE = X_BYTES + NPL * W_BYTES + SCX + SCW;
    static constexpr int EP_DX = limbs ? BM * 4 : 0;
    static constexpr int EP_DW = limbs ? BN * 4 : 0;
    static constexpr int EP_DMIN = (FMT == FMT_Q4_K) ? BN * 4 : 0;
    static constexpr int EP_AMIN = (FMT == FMT_Q4_K) ? (BM / 32) * 1024 : 0;
    static constexpr int EP_BMIN = (FMT == FMT_Q4_K) ? (BN / 32) * 1024 : 0;
    static constexpr int EP = EP_DX + EP_DW + EP_DMIN + EP_AMIN + EP_BMIN;
    static constexpr int LDS = 2 * STAGE + 2 * EP;
    static_assert(LDS <= 160 * 1024, "LDS budget");
    static_assert(BM <= 256 && BN <= 256, "one 64-lane DMA covers a scale row");
};

__device__ __forceinline__ void dma16(const void *g, void *lds) {
    __builtin_amdgcn_global_load_lds(g, (lds_void *)lds, 16, 0, 0);
}

// Issue the DMA of stage s into buffer p.  Wave-uniform branches only.
template <class C, int FMT>
__device__ __forceinline__ void issue_stage(const GemmArgs &a, int8_t *smem, int s, int p, int m0, int n0, int wave,
                                            int lane) {
    int8_t *st = smem + p * C::STAGE;
    constexpr int TOT = C::XF + C::NPL * C::WF;
#pragma unroll
    for (int f = wave; f < TOT; f += C::NW) {
        const int8_t *g;
        int8_t *l;
        if (f < C::XF) {
            const int rt = f >> 2, kc = f & 3;
            g = a.xq + ((int64_t)((m0 >> 5) + rt) * a.kch + s * 4 + kc) * 1024;
            l = st + f * 1024;
        } else {
            const int f2 = f - C::XF;
            const int pl = f2 / C::WF, f3 = f2 % C::WF;
            const int ct = f3 >> 2, kc = f3 & 3;
            g = (pl ? a.whi : a.wq) + ((int64_t)((n0 >> 5) + ct) * a.kch + s * 4 + kc) * 1024;
            l = st + C::X_BYTES + pl * C::W_BYTES + f3 * 1024;
        }
        dma16(g + lane * 16, l);
    }
    if constexpr (FMT == FMT_Q8_0) {
        // per-block scales of this stage: 4 blocks x BM (X side) and 4 x BN (W side)
        for (int f = wave; f < 8; f += C::NW) {
            const float *src;
            int8_t *dst;
            int pieces;
            if (f < 4) {
                src = a.xd + (int64_t)(s * 4 + f) * a.m_pad + m0;
                dst = st + C::X_BYTES + C::W_BYTES + f * C::BM * 4;
                pieces = C::BM / 4;
            } else {
                src = a.wd + (int64_t)(s * 4 + f - 4) * a.n_pad + n0;
                dst = st + C::X_BYTES + C::W_BYTES + C::SCX + (f - 4) * C::BN * 4;
                pieces = C::BN / 4;
            }
            if (lane < pieces) dma16(src + lane * 4, dst);
        }
    }
    if constexpr (C::limbs) {
        if ((s & 1) == 0) {
            const int sb = s >> 1;
            int8_t *ep = smem + 2 * C::STAGE + (sb & 1) * C::EP;
            constexpr int NI = (FMT == FMT_Q4_K) ? 3 + C::BM / 32 + C::BN / 32 : 2;
            for (int f = wave; f < NI; f += C::NW) {
                if (f == 0) {
                    if (lane < C::BM / 4) dma16(a.xd + (int64_t)sb * a.m_pad + m0 + lane * 4, ep);
                } else if (f == 1) {
                    if (lane < C::BN / 4) dma16(a.wd + (int64_t)sb * a.n_pad + n0 + lane * 4, ep + C::EP_DX);
                } else if (f == 2) {
                    if (lane < C::BN / 4)
                        dma16(a.wdmin + (int64_t)sb * a.n_pad + n0 + lane * 4, ep + C::EP_DX + C::EP_DW);
                } else if (f < 3 + C::BM / 32) {
                    const int rt = f - 3;
                    dma16((const int8_t *)a.xmin + ((int64_t)((m0 >> 5) + rt) * a.nsb + sb) * 1024 + lane * 16,
                          ep + C::EP_DX + C::EP_DW + C::EP_DMIN + rt * 1024);
                } else {
                    const int ct = f - 3 - C::BM / 32;
                    dma16((const int8_t *)a.wmin + ((int64_t)((n0 >> 5) + ct) * a.nsb + sb) * 1024 + lane * 16,
                          ep + C::EP_DX + C::EP_DW + C::EP_DMIN + C::EP_AMIN + ct * 1024);
                }
            }
        }
    }
}

__device__ __forceinline__ void wait_dma_and_barrier() {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
}

template <int FMT, int WM, int WN, int TM, int TN, int MINB>
__global__ __launch_bounds__(64 * WM * WN, MINB) void k_gemm(const GemmArgs a) {
    using C = Cfg<FMT, WM, WN, TM, TN>;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int lrow = lane & 31;
    const int lhalf = lane >> 5;

    // tile order: XCD-contiguous ranges, grouped GROUP_M token tiles x all feature tiles
    int t = blockIdx.x;
    const int nt = gridDim.x;
    if ((nt & 7) == 0) t = (t & 7) * (nt >> 3) + (t >> 3);
    const int per_group = a.group_m * a.tiles_n;
    const int grp = t / per_group, r = t - grp * per_group;
    const int gm = min(a.group_m, a.tiles_m - grp * a.group_m);
    const int tm = grp * a.group_m + r % gm, tn = r / gm;
    const int m0 = tm * C::BM, n0 = tn * C::BN;

    v16f acc[TM][TN];
    v16i alo[TM][TN], ahi[C::limbs ? TM : 1][C::limbs ? TN : 1];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            acc[i][j] = (v16f){};
            alo[i][j] = (v16i){};
            if constexpr (C::limbs) ahi[i][j] = (v16i){};
        }
    const int xfrag0 = wm * TM * 4 * 1024 + lane * 16;  // LDS byte offset of this wave's first X fragment
    const int wfrag0 = C::X_BYTES + wn * TN * 4 * 1024 + lane * 16;

    issue_stage<C, FMT>(a, smem, 0, 0, m0, n0, wave, lane);
    wait_dma_and_barrier();

    for (int s = 0; s < a.nstages; s++) {
        if (s + 1 < a.nstages) issue_stage<C, FMT>(a, smem, s + 1, (s + 1) & 1, m0, n0, wave, lane);
        const int8_t *st = smem + (s & 1) * C::STAGE;
#pragma unroll
        for (int kc = 0; kc < 4; kc++) {
            v4i xa[TM];
#pragma unroll
            for (int i = 0; i < TM; i++) xa[i] = *(const v4i *)(st + xfrag0 + (i * 4 + kc) * 1024);
            if constexpr (FMT == FMT_F16) {
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const v4i wb = *(const v4i *)(st + wfrag0 + (j * 4 + kc) * 1024);
#pragma unroll
                    for (int i = 0; i < TM; i++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, xa[i]),
                                                                          __builtin_bit_cast(v8h, wb), acc[i][j], 0,
                                                                          0, 0);
                }
            } else if constexpr (FMT == FMT_Q8_0) {
                const float *scx = (const float *)(st + C::X_BYTES + C::W_BYTES) + kc * C::BM;
                const float *scw = (const float *)(st + C::X_BYTES + C::W_BYTES + C::SCX) + kc * C::BN;
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const v4i wb = *(const v4i *)(st + wfrag0 + (j * 4 + kc) * 1024);
                    const float dw = scw[(wn * TN + j) * 32 + lrow];
#pragma unroll
                    for (int i = 0; i < TM; i++) {
                        const v16i tq = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa[i], wb, (v16i){}, 0, 0, 0);
#pragma unroll
                        for (int g = 0; g < 4; g++) {
                            const float4 dx4 = *(const float4 *)(scx + (wm * TM + i) * 32 + 8 * g + 4 * lhalf);
                            acc[i][j][4 * g + 0] += (float)tq[4 * g + 0] * (dx4.x * dw);
                            acc[i][j][4 * g + 1] += (float)tq[4 * g + 1] * (dx4.y * dw);
                            acc[i][j][4 * g + 2] += (float)tq[4 * g + 2] * (dx4.z * dw);
                            acc[i][j][4 * g + 3] += (float)tq[4 * g + 3] * (dx4.w * dw);
                        }
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const v4i wl = *(const v4i *)(st + wfrag0 + (j * 4 + kc) * 1024);
#pragma unroll
                    for (int i = 0; i < TM; i++)
                        alo[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa[i], wl, alo[i][j], 0, 0, 0);
                    const v4i wh = *(const v4i *)(st + C::W_BYTES + wfrag0 + (j * 4 + kc) * 1024);
#pragma unroll
                    for (int i = 0; i < TM; i++)
                        ahi[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa[i], wh, ahi[i][j], 0, 0, 0);
                }
            }
        }
        if constexpr (C::limbs) {
            if (s & 1) {
                // superblock s/2 complete: scale and fold into the fp32 accumulators
                const int8_t *ep = smem + 2 * C::STAGE + ((s >> 1) & 1) * C::EP;
                const float *edx = (const float *)ep;
                const float *edw = (const float *)(ep + C::EP_DX);
                const float *edm = (const float *)(ep + C::EP_DX + C::EP_DW);
                const int8_t *eam = ep + C::EP_DX + C::EP_DW + C::EP_DMIN;
                const int8_t *ebm = eam + C::EP_AMIN;
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const int wc = (wn * TN + j) * 32 + lrow;
                    const float dw = edw[wc];
                    float dmn = 0.f;
                    v8h bmin = {};
                    if constexpr (FMT == FMT_Q4_K) {
                        dmn = edm[wc];
                        bmin = *(const v8h *)(ebm + (wn * TN + j) * 1024 + lane * 16);
                    }
#pragma unroll
                    for (int i = 0; i < TM; i++) {
                        v16f fmin = {};
                        if constexpr (FMT == FMT_Q4_K) {
                            const v8h amin = *(const v8h *)(eam + (wm * TM + i) * 1024 + lane * 16);
                            fmin = __builtin_amdgcn_mfma_f32_32x32x16_f16(amin, bmin, (v16f){}, 0, 0, 0);
                        }
#pragma unroll
                        for (int g = 0; g < 4; g++) {
                            const float4 dx4 = *(const float4 *)(edx + (wm * TM + i) * 32 + 8 * g + 4 * lhalf);
                            const float dxs[4] = {dx4.x, dx4.y, dx4.z, dx4.w};
#pragma unroll
                            for (int q = 0; q < 4; q++) {
                                const int rr = 4 * g + q;
                                const int isum = alo[i][j][rr] + (ahi[i][j][rr] << 7);
                                float tv = dw * (float)isum;
                                if constexpr (FMT == FMT_Q4_K) tv -= dmn * fmin[rr];
                                acc[i][j][rr] += dxs[q] * tv;
                            }
                        }
                        alo[i][j] = (v16i){};
                        ahi[i][j] = (v16i){};
                    }
                }
            }
        }
        wait_dma_and_barrier();
    }

    // store: lanes 0..31 of a register write 32 consecutive floats of one row
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int col = n0 + (wn * TN + j) * 32 + lrow;
            if (col >= a.N) continue;
#pragma unroll
            for (int rr = 0; rr < 16; rr++) {
                const int row = m0 + (wm * TM + i) * 32 + 8 * (rr >> 2) + 4 * lhalf + (rr & 3);
                if (row < a.M) a.y[(int64_t)row * a.ldy + col] = acc[i][j][rr];
            }
        }
}

template <int FMT, int WM, int WN, int TM, int TN, int MINB>
static hipError_t launch_cfg(GemmArgs a, hipStream_t s) {
    using C = Cfg<FMT, WM, WN, TM, TN>;
    static bool attr_set = false;
    if (!attr_set) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_gemm<FMT, WM, WN, TM, TN, MINB>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    a.tiles_m = (a.M + C::BM - 1) / C::BM;
    a.tiles_n = (a.N + C::BN - 1) / C::BN;
    a.group_m = 8;
    const unsigned grid = (unsigned)(a.tiles_m * a.tiles_n);
    hipLaunchKernelGGL((k_gemm<FMT, WM, WN, TM, TN, MINB>), dim3(grid), dim3(C::NT), C::LDS, s, a);
    return hipGetLastError();
}

// Tile configuration, selectable with MQ_GEMM_CFG for measurements:
//   1: 8 waves x (64x64)  WG 256x128, 2 waves/SIMD
//   2: 4 waves x (128x64) WG 256x128, 1 wave/SIMD, 512 registers
//   3: 4 waves x (64x64)  WG 128x128, 2 WGs/CU
static int gemm_cfg_env() {
    const char *e = getenv("MQ_GEMM_CFG");  // read per launch so a process can compare configurations
    return (e && *e) ? atoi(e) : 0;
}

template <int FMT>
static hipError_t launch_fmt(GemmArgs a, hipStream_t s) {
    int cfg = gemm_cfg_env();
    if (cfg < 1 || cfg > 3) {
        // 256x128 tiles when that still gives every CU a tile, else 128x128
        const int64_t big = (int64_t)((a.M + 255) / 256) * ((a.N + 127) / 128);
        cfg = (big >= 256) ? (FMT == FMT_Q4_K || FMT == FMT_Q6_K ? 2 : 1) : 3;
    }
    if (cfg == 1) return launch_cfg<FMT, 4, 2, 2, 2, 1>(a, s);
    if (cfg == 2) return launch_cfg<FMT, 2, 2, 4, 2, 1>(a, s);
    return launch_cfg<FMT, 2, 2, 2, 2, 2>(a, s);
}

hipError_t launch_gemm(int type, const void *image, int64_t n, int64_t k, const void *ws, int64_t m, float *y,
                       int64_t ldy, hipStream_t s) {
    if (m <= 0 || n <= 0) return hipSuccess;
    const WeightPlanes p = weight_planes(type, n, k);
    const ActPlanes ap = act_planes(type, m, k, true);
    const uint8_t *wb = (const uint8_t *)image;
    const uint8_t *xb = (const uint8_t *)ws;
    GemmArgs a{};
    a.xq = (const int8_t *)(xb + ap.xq);
    a.xd = (const float *)(xb + ap.xd);
    a.xmin = (const _Float16 *)(xb + ap.xmin);
    a.wq = (const int8_t *)(wb + p.tq);
    a.whi = (const int8_t *)(wb + p.thi);
    a.wd = (const float *)(wb + p.tdw);
    a.wdmin = (const float *)(wb + p.tdmin);
    a.wmin = (const _Float16 *)(wb + p.tmin);
    a.y = y;
    a.M = (int)m;
    a.N = (int)n;
    a.ldy = (int)ldy;
    a.m_pad = (int)ap.m_pad;
    a.n_pad = (int)p.n_pad;
    a.kch = (int)(p.kb_pad / 32);
    a.nstages = (int)(p.kb_pad / KSTAGE);
    a.nsb = (int)(k / QK_K);
    switch (type) {
        case MQ_TYPE_Q8_0: return launch_fmt<FMT_Q8_0>(a, s);
        case MQ_TYPE_Q4_K: return launch_fmt<FMT_Q4_K>(a, s);
        case MQ_TYPE_Q6_K: return launch_fmt<FMT_Q6_K>(a, s);
        case MQ_TYPE_F16: return launch_fmt<FMT_F16>(a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mq
