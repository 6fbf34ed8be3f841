// mq_gemm.hip -- batched-token MFMA GEMM for GGML_OP_MUL_MAT on gfx950.
//
// Y[m][n] = sum_k X[m][k] * W[n][k], X requantized to ggml's vec_dot_type.
//
// Arithmetic (exact integer block dots, fp32 scales, as ggml_vec_dot_*):
//   Q8_0  v_mfma_i32_32x32x32_i8, one Q8_0 block (K = 32) per MFMA; the int32
//         block dot is scaled by d_x * d_w in fp32 right after the block.  The
//         32x32 tile of scale products d_x[r] * d_w[c] comes from a rank-1
//         v_mfma_f32_32x32x2_f32 (exact: both scales are fp16 values), which leaves
//         two VALU ops per output and block (convert, fma) instead of three: the
//         per-block scaling, not the int8 MFMA, bounds this format.
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
#include "mq_act.h"
#include "mq_q8k.h"

#include <climits>
#include <type_traits>

namespace mq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_void;

enum { FMT_Q8_0 = 0, FMT_Q4_K = 1, FMT_Q6_K = 2, FMT_F16 = 3 };

constexpr int GEMM_GROUPS = 4;

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
    const float *bias;  // NULL, or N floats added to every row in the store
    // quantized output (qo not NULL, one weight group): v = op(acc + bias) is stored as the
    // activation of a following mat-mul in its GEMM layout instead of as floats in y; q_pre is
    // MQ_PRE_NONE or MQ_PRE_GELU_ERF.  q_fmt 0: Q8_0 (quants tiled [q_m_pad][32 q_kch], scales
    // [q_kch][q_m_pad], q_var the rounding variant); q_fmt 1: Q8_K (quants tiled, scales
    // [q_ncb][q_m_pad], min-term fragments qmin [q_m_pad / 32][q_ncb]; needs BN = 256, a
    // workgroup owning whole 256-value superblocks of its rows)
    int8_t *qo;
    float *qd;
    _Float16 *qmin;
    int q_m_pad, q_kch, q_pre, q_var, q_fmt, q_ncb;
    // attention K/V as MFMA operand fragments (kvf not NULL, one weight group): output columns
    // [kv_col0, kv_col0 + kv_nkv kv_hd) are K, the next kv_nkv kv_hd columns V, row b kv_T + key
    // (kv_T a multiple of 32).  They leave split hi / lo in the attention's fragment layout
    // (as k_kv_frag writes them: kv_nblk 32-key blocks per (sequence, head)), not as floats;
    // the columns before kv_col0 are stored as usual.
    _Float16 *kvf;
    int kv_col0, kv_T, kv_hd, kv_nkv, kv_nblk;
    // mixture of experts (moe not NULL, one weight group): the rows are sorted by expert in
    // segments of whole BM-row tiles; moe[0] = the number of live row tiles, moe[1 + tm] = the
    // expert of row tile tm, whose weight planes lie moe_stride bytes past the previous
    // expert's (row tiles from moe[0] on are skipped)
    const int *moe;
    int64_t moe_stride;
    int M, N, ldy;
    int m_pad, n_pad;
    int kch;      // 32-byte K chunks per row (kb_pad / 32)
    int nstages;  // kb_pad / 128
    int nsb;      // K / 256
    int tiles_m, tiles_n, group_m;
    // grouped launch (GEMM_GROUPS weights on the same activation and k): group g > 0 has its
    // own weight planes, output, bias and N in grp[g - 1] and owns the feature tiles
    // [tn_start[g], tn_start[g + 1]); tn_start[g] = INT_MAX past the last group
    int ngroups;
    int tn_start[GEMM_GROUPS];
    struct Group {
        const int8_t *wq, *whi;
        const float *wd, *wdmin;
        const _Float16 *wmin;
        float *y;
        const float *bias;
        int N, n_pad, ldy;
        int kv_col0;  // as GemmArgs::kv_col0, for this group's columns
    } grp[GEMM_GROUPS - 1];
};


// WM x WN waves per workgroup, each wave TM x TN MFMA tiles of 32x32; stages of KC 32-byte
// K chunks (64 bytes by default; 32 halves the ring so two workgroups share a CU); a ring of NB
// stages in LDS with D of them in flight ahead of the one being computed (4 and 3 by default;
// a shorter ring leaves room for more workgroups per CU).  KG > 1 (Q8_0, one 32x32 tile per
// wave): KG groups of WM x WN waves split each stage's KC chunks, group g taking chunks
// g KC/KG .. (g + 1) KC/KG - 1 of every stage, and their partial sums meet in LDS at the end.
template <int FMT, int WM, int WN, int TM, int TN, int KCT = 2, int NBT = 4, int DT = 3, int KGT = 1>
struct Cfg {
    static constexpr int NB = NBT, D = DT;
    static_assert(D + 1 <= NB, "stage ring: D stages in flight plus the one being computed");
    static constexpr int KC = KCT;              // 32-byte K chunks per stage
    static constexpr int SPB = 256 / (32 * KC);  // stages per 256-value superblock
    static constexpr int KG = KGT, NTW = WM * WN;  // K groups, waves per K group
    static_assert(KG == 1 || (FMT == FMT_Q8_0 && TM == 1 && TN == 1 && KC % KG == 0), "K groups: Q8_0, one tile per wave");
    static constexpr int NW = NTW * KG, NT = 64 * NW, BM = 32 * TM * WM, BN = 32 * TN * WN;
    static constexpr bool limbs = (FMT == FMT_Q4_K || FMT == FMT_Q6_K);
    static constexpr int NPL = limbs ? 2 : 1;
    static constexpr int XF = (BM / 32) * KC, WF = (BN / 32) * KC;  // data fragments per stage
    static constexpr int X_BYTES = XF * 1024, W_BYTES = WF * 1024;
    // Q8_0 scale rows move as full 64-lane DMAs, so no DMA is lane-masked: one row of BM or BN
    // floats per 1 KB slot (filling its first BM*4 / BN*4 bytes), or with packed scales (the
    // K-group forms: BM, BN <= 64, KC <= 4) the KC rows of a stage in one slot, 256 bytes each
    // (lane l fetches a piece of chunk l / 16's row), so a stage's scales are two DMAs
    static constexpr bool PSC = KG > 1;
    static_assert(!PSC || (BM <= 64 && BN <= 64 && KC <= 4), "packed scale slots: 4 rows of <= 64 floats");
    static constexpr int SCROW = PSC ? 256 : 1024;  // bytes from one chunk's scale row to the next
    static constexpr int NSC = (FMT == FMT_Q8_0) ? (PSC ? 2 : 2 * KC) : 0;  // Q8_0 scale DMAs per stage
    static constexpr int SCX = (FMT == FMT_Q8_0) ? (PSC ? 1024 : KC * 1024) : 0;
    static constexpr int SCW = SCX;
    static constexpr int STAGE = X_BYTES + NPL * W_BYTES + SCX + SCW;
    static constexpr int NITEM = XF + NPL * WF + NSC;               // DMA instructions per stage
    static constexpr int IPW = (NITEM + NW - 1) / NW;               // per wave (upper bound)
    static constexpr int EP_DX = limbs ? 1024 : 0;
    static constexpr int EP_DW = limbs ? 1024 : 0;
    static constexpr int EP_DMIN = (FMT == FMT_Q4_K) ? 1024 : 0;
    static constexpr int EP_AMIN = (FMT == FMT_Q4_K) ? (BM / 32) * 1024 : 0;
    static constexpr int EP_BMIN = (FMT == FMT_Q4_K) ? (BN / 32) * 1024 : 0;
    static constexpr int EP = EP_DX + EP_DW + EP_DMIN + EP_AMIN + EP_BMIN;
    static constexpr int NEPI = (FMT == FMT_Q4_K) ? 3 + BM / 32 + BN / 32 : (limbs ? 2 : 0);
    static constexpr int EPW = (NEPI + NW - 1) / NW;
    static constexpr int LDS_RING = NB * STAGE + 2 * EP;
    // the quantized-output and K-fragment epilogues stage a 32 x 36-float tile per wave in the
    // same memory once the ring is drained
    static constexpr int LDS_STG = NW * 32 * 36 * 4;
    // the Q8_K-output epilogue (BN = 256) stages the whole BM x 256 fp32 tile, then the tile's
    // min-term fragments and row scales
    static constexpr int LDS_Q8K = BN == 256 ? BM * 1024 + (BM / 32) * 1024 + BM * 4 : 0;
    static constexpr int LDS_E0 = LDS_STG > LDS_Q8K ? LDS_STG : LDS_Q8K;
    // K groups 1 .. KG-1 leave their 32x32 partial sums (4 KB per wave) for group 0
    static constexpr int LDS_PART = (KG - 1) * NTW * 4096;
    static constexpr int LDS_E = LDS_E0 > LDS_PART ? LDS_E0 : LDS_PART;
    static constexpr int LDS = LDS_RING > LDS_E ? LDS_RING : LDS_E;
    // DMAs issued per stage by every wave, and the count still in flight when stage
    // position q (of a superblock) may be computed: those of the D-1 later stages.
    static constexpr int dmas(int stage_pos) { return IPW + ((limbs && stage_pos % SPB == 0) ? EPW : 0); }
    template <int D>
    static constexpr int waits(int q) {
        int w = 0;
        for (int x = 1; x < D; x++) w += dmas(q + x);
        return w;
    }
    static_assert(LDS <= 160 * 1024, "LDS budget");
    static_assert(BM <= 256 && BN <= 256, "one 64-lane DMA covers a scale row");
    static_assert((BM & (BM - 1)) == 0 && (BN & (BN - 1)) == 0, "scale rows of 2^k floats (lane masks)");
};

__device__ __forceinline__ void dma16(const void *g, void *lds) {
    __builtin_amdgcn_global_load_lds(g, (lds_void *)lds, 16, 0, 0);
}

// compile-time loop: f(integral_constant<int, Q>) for Q in [B, E)
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// s_waitcnt with a compile-time count
template <int N>
__device__ __forceinline__ void wait_vmcnt_c() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// LDS reads of DMA-filled epilogue data.  Written as asm so the compiler does not
// guard them with a wait for every outstanding DMA (its LDS-DMA alias tracking
// cannot tell the epilogue region from the stages still in flight); the data was
// ordered by the explicit vmcnt wait + barrier at the top of the iteration.
typedef __attribute__((address_space(3))) const char lds_cchar;
__device__ __forceinline__ uint32_t lds_addr(const void *p) { return (uint32_t)(uintptr_t)(lds_cchar *)p; }
__device__ __forceinline__ v4i ds_read128(uint32_t a) {
    v4i r;
    asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(a));
    return r;
}
__device__ __forceinline__ float ds_read32(uint32_t a) {
    float r;
    asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(a));
    return r;
}
// the same with a constant byte offset (one address register for many reads)
template <int OFF>
__device__ __forceinline__ float ds_read32_o(uint32_t a) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offsets are 16 bits");
    float r;
    asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(r) : "v"(a), "n"(OFF));
    return r;
}

// Workgroup barrier that does not wait for outstanding DMAs (a fenced
// __syncthreads would wait for every one of them, i.e. empty the pipeline).  It
// does wait for this wave's own LDS reads: after the barrier other waves refill
// the ring slot this wave read last, and the compiler may leave those reads in
// flight up to here.
__device__ __forceinline__ void barrier_nofence() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// One DMA item: a stage-relative source (advancing `step` bytes per stage) and a
// stage-relative LDS offset.  Every item moves 64 lanes x 16 bytes; for rows
// shorter than 1 KB (`pieces` < 64) the upper lanes re-read the row's first bytes
// into the unused tail of the 1 KB slot, so all DMAs run with a full exec mask.
struct DmaItem {
    const int8_t *g0;
    int64_t step;
    int lds;
    int pieces;
    int loff;  // this lane's byte offset from g0, (lane % pieces) 16 unless remapped (used by GLU kernels)
};

// Weight tile (32 rows) of the workgroup's 32-column block c.  GLU (a gated FFN's gate|up
// weight, N = 2 n_ff: gate rows, then up rows): block c holds gate tile n0 / 64 + c / 2 for
// even c, the same up tile for odd c, so a wave's two column tiles (TN = 2) are the gate and up
// projections of the same 32 features.
template <bool GLU>
__device__ __forceinline__ int wtile(const GemmArgs &a, int n0, int c) {
    if constexpr (GLU) return (c & 1) * (a.N >> 6) + (n0 >> 6) + (c >> 1);
    else return (n0 >> 5) + c;
}

// GLU: byte offset of this lane's 16 bytes (4 columns) of a weight scale row of the
// workgroup's BN columns, from the row's start
template <bool GLU>
__device__ __forceinline__ int wrow_off(const GemmArgs &a, int n0, int lane, int pieces) {
    const int p = lane & (pieces - 1);
    return (wtile<GLU>(a, n0, p >> 3) * 32 + ((4 * p) & 31)) * 4;
}

template <class C, int FMT, bool GLU>
__device__ __forceinline__ DmaItem stage_item(const GemmArgs &a, int f, int m0, int n0, int lane) {
    DmaItem it;
    it.pieces = 64;
    it.loff = lane * 16;
    if (f < C::XF) {
        const int rt = f / C::KC, kc = f % C::KC;
        it.g0 = a.xq + ((int64_t)((m0 >> 5) + rt) * a.kch + kc) * 1024;
        it.step = C::KC * 1024;
        it.lds = f * 1024;
    } else if (f < C::XF + C::NPL * C::WF) {
        const int f2 = f - C::XF;
        const int pl = f2 / C::WF, f3 = f2 % C::WF;
        const int ct = f3 / C::KC, kc = f3 % C::KC;
        it.g0 = (pl ? a.whi : a.wq) + ((int64_t)wtile<GLU>(a, n0, ct) * a.kch + kc) * 1024;
        it.step = C::KC * 1024;
        it.lds = C::X_BYTES + pl * C::W_BYTES + f3 * 1024;
    } else {
        const int f4 = f - C::XF - C::NPL * C::WF;  // Q8_0 scale rows
        if constexpr (C::PSC) {
            // chunk (lane / 16) % 4's row: pieces of 16 bytes, lanes past a row's pieces re-read it
            const int kc = (lane >> 4) & 3, np = (f4 == 0 ? C::BM : C::BN) / 4;
            const int64_t ld = f4 == 0 ? a.m_pad : a.n_pad;
            it.g0 = (const int8_t *)(f4 == 0 ? a.xd + m0 : a.wd + n0);
            it.step = (int64_t)C::KC * ld * 4;
            it.lds = C::X_BYTES + C::W_BYTES + f4 * C::SCX;
            it.pieces = 64;
            it.loff = (int)(kc * ld * 4) + (lane & (np - 1)) * 16;
            return it;
        }
        if (f4 < C::KC) {
            it.g0 = (const int8_t *)(a.xd + (int64_t)f4 * a.m_pad + m0);
            it.step = (int64_t)C::KC * a.m_pad * 4;
            it.lds = C::X_BYTES + C::W_BYTES + f4 * 1024;
            it.pieces = C::BM / 4;
            it.loff = (lane & (it.pieces - 1)) * 16;
        } else {
            it.g0 = (const int8_t *)(a.wd + (int64_t)(f4 - C::KC) * a.n_pad + (GLU ? 0 : n0));
            it.step = (int64_t)C::KC * a.n_pad * 4;
            it.lds = C::X_BYTES + C::W_BYTES + C::SCX + (f4 - C::KC) * 1024;
            it.pieces = C::BN / 4;
            if constexpr (GLU) it.loff = wrow_off<GLU>(a, n0, lane, it.pieces);
        }
    }
    return it;
}

// Superblock epilogue item e for superblock sb (K-quants).
template <class C, int FMT, bool GLU>
__device__ __forceinline__ DmaItem epi_item(const GemmArgs &a, int e, int sb, int m0, int n0, int lane) {
    DmaItem it;
    it.step = 0;
    it.pieces = 64;
    it.loff = lane * 16;
    if (e == 0) {
        it.g0 = (const int8_t *)(a.xd + (int64_t)sb * a.m_pad + m0);
        it.lds = 0;
        it.pieces = C::BM / 4;
        it.loff = (lane & (it.pieces - 1)) * 16;
    } else if (e == 1) {
        it.g0 = (const int8_t *)(a.wd + (int64_t)sb * a.n_pad + (GLU ? 0 : n0));
        it.lds = C::EP_DX;
        it.pieces = C::BN / 4;
        if constexpr (GLU) it.loff = wrow_off<GLU>(a, n0, lane, it.pieces);
    } else if (e == 2) {
        it.g0 = (const int8_t *)(a.wdmin + (int64_t)sb * a.n_pad + (GLU ? 0 : n0));
        it.lds = C::EP_DX + C::EP_DW;
        it.pieces = C::BN / 4;
        if constexpr (GLU) it.loff = wrow_off<GLU>(a, n0, lane, it.pieces);
    } else if (e < 3 + C::BM / 32) {
        const int rt = e - 3;
        it.g0 = (const int8_t *)a.xmin + ((int64_t)((m0 >> 5) + rt) * a.nsb + sb) * 1024;
        it.lds = C::EP_DX + C::EP_DW + C::EP_DMIN + rt * 1024;
    } else {
        const int ct = e - 3 - C::BM / 32;
        it.g0 = (const int8_t *)a.wmin + ((int64_t)wtile<GLU>(a, n0, ct) * a.nsb + sb) * 1024;
        it.lds = C::EP_DX + C::EP_DW + C::EP_DMIN + C::EP_AMIN + ct * 1024;
    }
    return it;
}

// GLU: a.N = 2 n_ff columns of a gate|up weight; y receives silu(gate) * up, n_ff columns (the
// gated FFN's down-projection input, src/decoder_embed.cpp:793-802), and no gate or up value
// is stored.
template <int FMT, int WM, int WN, int TM, int TN, int MINB, int KCT = 2, bool GLU = false, int NBT = 4, int DT = 3,
          int KG = 1>
__global__ __launch_bounds__(64 * WM * WN * KG, MINB) void k_gemm(const GemmArgs a0) {
    using C = Cfg<FMT, WM, WN, TM, TN, KCT, NBT, DT, KG>;
    constexpr int NBUF = C::NB, DIST = C::D;
    static_assert(!GLU || TN == 2, "GLU: each wave holds a gate and an up column tile");
    constexpr int KC = C::KC, SPB = C::SPB;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // uniform: SALU addressing
    const int wt = wave % C::NTW, kg = wave / C::NTW;  // tile wave, K group
    const int wm = wt / WN, wn = wt % WN;
    const int kc0 = kg * (C::KC / KG);  // the K group's first chunk of every stage
    const int lrow = lane & 31;
    const int lhalf = lane >> 5;

    // tile order: XCD-contiguous ranges, grouped GROUP_M token tiles x all feature tiles
    int t = blockIdx.x;
    const int nt = gridDim.x;
    if ((nt & 7) == 0) t = (t & 7) * (nt >> 3) + (t >> 3);
    const int per_group = a0.group_m * a0.tiles_n;
    const int grp = t / per_group, r = t - grp * per_group;
    const int gm = min(a0.group_m, a0.tiles_m - grp * a0.group_m);
    const int tm = grp * a0.group_m + r % gm;
    int tn = r / gm;
    // the weight group owning feature tile tn (uniform: scalar selects)
    GemmArgs a = a0;
    if (a0.ngroups > 1) {
        int g = 0;
#pragma unroll
        for (int i = 1; i < GEMM_GROUPS; i++) g += tn >= a0.tn_start[i];
        if (g > 0) {
            const GemmArgs::Group &G = a0.grp[g - 1];
            a.wq = G.wq, a.whi = G.whi, a.wd = G.wd, a.wdmin = G.wdmin, a.wmin = G.wmin;
            a.y = G.y, a.bias = G.bias, a.N = G.N, a.n_pad = G.n_pad, a.ldy = G.ldy, a.kv_col0 = G.kv_col0;
            tn -= a0.tn_start[g];
        }
    }
    if (a0.moe) {
        if (tm >= a0.moe[0]) return;  // uniform: before any DMA or barrier
        const int64_t off = (int64_t)a0.moe[1 + tm] * a0.moe_stride;
        a.wq += off;
        if (a.whi) a.whi += off;
        a.wd = (const float *)((const char *)a.wd + off);
        if (a.wdmin) a.wdmin = (const float *)((const char *)a.wdmin + off);
        if (a.wmin) a.wmin = (const _Float16 *)((const char *)a.wmin + off);
    }
    const int m0 = tm * C::BM, n0 = tn * C::BN;
    const int nst = a.nstages;

    // This wave's DMA items.  Every wave issues exactly IPW stage DMAs per stage
    // (plus EPW epilogue DMAs with the first stage of each superblock): a wave
    // past the item count repeats an item (same source, same LDS bytes, same
    // data).  The number of DMAs in flight is then the same on every wave at
    // every point, so each wait below is a compile-time constant.
    DmaItem items[C::IPW];
#pragma unroll
    for (int i = 0; i < C::IPW; i++) items[i] = stage_item<C, FMT, GLU>(a, (wave + C::NW * i) % C::NITEM, m0, n0, lane);

    // Stages past the end are issued too, re-reading the last stage into the
    // slot of a stage that is never computed, so the DMA count per stage stays
    // uniform through the tail.
    // always_inline: a call would move the accumulators to scratch memory
    auto issue = [&](int s) __attribute__((always_inline)) {
        int8_t *st = smem + (s % NBUF) * C::STAGE;
        const int64_t sc = s < nst ? s : nst - 1;
        if constexpr (C::limbs) {
            if (s % SPB == 0) {
                const int sb = s / SPB;
                int8_t *ep = smem + NBUF * C::STAGE + (sb & 1) * C::EP;
                const int sbc = sb < a.nsb ? sb : a.nsb - 1;
#pragma unroll
                for (int i = 0; i < C::EPW; i++) {
                    const DmaItem it = epi_item<C, FMT, GLU>(a, (wave + C::NW * i) % C::NEPI, sbc, m0, n0, lane);
                    if constexpr (GLU) dma16(it.g0 + it.loff, ep + it.lds);
                    else dma16(it.g0 + (lane & (it.pieces - 1)) * 16, ep + it.lds);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < C::IPW; i++) {
            if constexpr (GLU || C::PSC) dma16(items[i].g0 + sc * items[i].step + items[i].loff, st + items[i].lds);
            else dma16(items[i].g0 + sc * items[i].step + (lane & (items[i].pieces - 1)) * 16, st + items[i].lds);
        }
    };

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
    const int xfrag0 = (wm * TM * KC + kc0) * 1024 + lane * 16;  // LDS offset of this wave's first X fragment
    const int wfrag0 = C::X_BYTES + (wn * TN * KC + kc0) * 1024 + lane * 16;

    // Q8_0 stage: per block and 32x32 tile, an int8 MFMA (block dot), a rank-1 f32
    // MFMA (scale products) and the convert + fma of the 16 outputs per lane.  The
    // steps are software-pipelined: the MFMAs of step u+1 are issued before the
    // VALU work of step u, so the matrix and vector pipes overlap within a wave.
    auto compute_q8_0 = [&](const int8_t *st) __attribute__((always_inline)) {
        constexpr int NTL = TM * TN, NSTEP = KC * NTL;
        v4i xa[KC][TM], wb[KC][TN];
        float dx[KC][TM], dw[KC][TN];
#pragma unroll
        for (int kc = 0; kc < KC; kc++) {
            // scale reads (asm: see ds_read128); lane l < 32 holds the k = 0 operands of
            // the rank-1 MFMA, d_x of row l and d_w of column l; A's k = 1 half is zero
            const uint32_t scx = lds_addr(st + C::X_BYTES + C::W_BYTES + kc * 1024);
            const uint32_t scw = lds_addr(st + C::X_BYTES + C::W_BYTES + C::SCX + kc * 1024);
#pragma unroll
            for (int j = 0; j < TN; j++) dw[kc][j] = ds_read32(scw + ((wn * TN + j) * 32 + lrow) * 4);
#pragma unroll
            for (int i = 0; i < TM; i++) dx[kc][i] = ds_read32(scx + ((wm * TM + i) * 32 + lrow) * 4);
#pragma unroll
            for (int i = 0; i < TM; i++) xa[kc][i] = *(const v4i *)(st + xfrag0 + (i * KC + kc) * 1024);
#pragma unroll
            for (int j = 0; j < TN; j++) wb[kc][j] = *(const v4i *)(st + wfrag0 + (j * KC + kc) * 1024);
        }
        // (the occupancy and K-group forms use compute_q8_0_occ instead)
        static_assert(FMT != FMT_Q8_0 || MINB >= 4 || KG > 1 || (KC == 2 && TM <= 2 && TN <= 2),
                      "the wait below names every scale register");
        // each register named once: an operand listed twice is copied (v_mov) before the wait,
        // i.e. read before its ds_read has landed, and that stale copy is what gets used
        if constexpr (TM == 2 && TN == 2)
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(dw[0][0]), "+v"(dw[0][TN - 1]), "+v"(dx[0][0]), "+v"(dx[0][TM - 1]), "+v"(dw[1][0]),
                           "+v"(dw[1][TN - 1]), "+v"(dx[1][0]), "+v"(dx[1][TM - 1]));
        else if constexpr (TM == 2)
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(dw[0][0]), "+v"(dx[0][0]), "+v"(dx[0][TM - 1]), "+v"(dw[1][0]), "+v"(dx[1][0]),
                           "+v"(dx[1][TM - 1]));
        else if constexpr (TN == 2)
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(dw[0][0]), "+v"(dw[0][TN - 1]), "+v"(dx[0][0]), "+v"(dw[1][0]), "+v"(dw[1][TN - 1]),
                           "+v"(dx[1][0]));
        else
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(dw[0][0]), "+v"(dx[0][0]), "+v"(dw[1][0]), "+v"(dx[1][0]));
#pragma unroll
        for (int kc = 0; kc < KC; kc++)
#pragma unroll
            for (int i = 0; i < TM; i++) dx[kc][i] = lhalf ? 0.0f : dx[kc][i];
        v16i tq[2];
        v16f sc[2];
        auto mfma = [&](auto uc) __attribute__((always_inline)) {
            constexpr int u = decltype(uc)::value, kc = u / NTL, i = u % TM, j = (u % NTL) / TM;
            tq[u & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa[kc][i], wb[kc][j], (v16i){}, 0, 0, 0);
            sc[u & 1] = __builtin_amdgcn_mfma_f32_32x32x2f32(dx[kc][i], dw[kc][j], (v16f){}, 0, 0, 0);
        };
        auto scale = [&](auto uc) __attribute__((always_inline)) {
            constexpr int u = decltype(uc)::value, i = u % TM, j = (u % NTL) / TM;
#pragma unroll
            for (int rr = 0; rr < 16; rr++) acc[i][j][rr] += (float)tq[u & 1][rr] * sc[u & 1][rr];
        };
        mfma(std::integral_constant<int, 0>{});
        static_for<1, NSTEP>([&](auto uc) __attribute__((always_inline)) {
            constexpr int u = decltype(uc)::value;
            mfma(std::integral_constant<int, u>{});
            __builtin_amdgcn_sched_barrier(0);
            scale(std::integral_constant<int, u - 1>{});
            __builtin_amdgcn_sched_barrier(0);
        });
        scale(std::integral_constant<int, NSTEP - 1>{});
    };

    // Q8_0 occupancy form (MINB >= 4: the one-wave-tile workgroup within 80 registers, so six
    // workgroups share a CU): one block at a time -- its operands, its two MFMAs, the convert +
    // fma of its 16 outputs per lane -- so only one step's results are live, and the other
    // waves of the SIMD fill the latency a single wave leaves.  Scale reads at constant offsets
    // from one address register per operand side.
    const uint32_t scx_base = lds_addr(smem + kc0 * C::SCROW + (wm * TM * 32 + lrow) * 4);
    const uint32_t scw_base = lds_addr(smem + kc0 * C::SCROW + (wn * TN * 32 + lrow) * 4);
    auto compute_q8_0_occ = [&](auto slotc) __attribute__((always_inline)) {
        constexpr int slot = decltype(slotc)::value;
        static_assert(TM == 1 && TN == 1, "one 32x32 tile per wave");
        const int8_t *st = smem + slot * C::STAGE;
        static_for<0, KC / KG>([&](auto kcc) __attribute__((always_inline)) {
            constexpr int kc = decltype(kcc)::value;
            constexpr int sco = slot * C::STAGE + C::X_BYTES + C::W_BYTES + kc * C::SCROW;
            float dw = ds_read32_o<sco + C::SCX>(scw_base);
            float dx = ds_read32_o<sco>(scx_base);
            v4i xa = *(const v4i *)(st + xfrag0 + kc * 1024);
            const v4i wb = *(const v4i *)(st + wfrag0 + kc * 1024);
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(dw), "+v"(dx));
            // the MFMAs are pure: tie them after the previous block's fmas (no instruction), or
            // the compiler hoists every block's MFMAs and keeps all their results live
            // (scalar operands: a 64-byte vector operand is not valid in the host pass)
            if constexpr (kc > 0) {
                const v16f &c = acc[0][0];
                asm volatile("" : "+v"(xa) : "v"(c[0]), "v"(c[1]), "v"(c[2]), "v"(c[3]), "v"(c[4]), "v"(c[5]), "v"(c[6]),
                             "v"(c[7]), "v"(c[8]), "v"(c[9]), "v"(c[10]), "v"(c[11]), "v"(c[12]), "v"(c[13]), "v"(c[14]),
                             "v"(c[15]));
            }
            dx = lhalf ? 0.0f : dx;  // the rank-1 MFMA's k = 1 half is zero
            const v16i tq = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa, wb, (v16i){}, 0, 0, 0);
            const v16f sc = __builtin_amdgcn_mfma_f32_32x32x2f32(dx, dw, (v16f){}, 0, 0, 0);
#pragma unroll
            for (int rr = 0; rr < 16; rr++) acc[0][0][rr] += (float)tq[rr] * sc[rr];
            __builtin_amdgcn_sched_barrier(0);
        });
    };

    // MFMAs of one stage
    auto compute = [&](const int8_t *st) __attribute__((always_inline)) {
        if constexpr (FMT == FMT_Q8_0) {
            compute_q8_0(st);
            return;
        }
#pragma unroll
        for (int kc = 0; kc < KC; kc++) {
            v4i xa[TM];
#pragma unroll
            for (int i = 0; i < TM; i++) xa[i] = *(const v4i *)(st + xfrag0 + (i * KC + kc) * 1024);
            if constexpr (FMT == FMT_F16) {
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const v4i wb = *(const v4i *)(st + wfrag0 + (j * KC + kc) * 1024);
#pragma unroll
                    for (int i = 0; i < TM; i++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, xa[i]),
                                                                          __builtin_bit_cast(v8h, wb), acc[i][j], 0,
                                                                          0, 0);
                }
            } else {
                v4i wl[TN], wh[TN];
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    wl[j] = *(const v4i *)(st + wfrag0 + (j * KC + kc) * 1024);
                    wh[j] = *(const v4i *)(st + C::W_BYTES + wfrag0 + (j * KC + kc) * 1024);
                }
#pragma unroll
                for (int j = 0; j < TN; j++)
#pragma unroll
                    for (int i = 0; i < TM; i++) {
                        alo[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa[i], wl[j], alo[i][j], 0, 0, 0);
                        ahi[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa[i], wh[j], ahi[i][j], 0, 0, 0);
                    }
            }
        }
    };

    // Superblock epilogue (K-quants): scale the exact integer sums and fold them
    // into the fp32 accumulators.  Per row tile, the limbs are combined first and
    // the min-term MFMAs issued, so their latency overlaps the scale reads.
    auto epilogue = [&](int sb) __attribute__((always_inline)) {
        const uint32_t ep = lds_addr(smem + NBUF * C::STAGE + (sb & 1) * C::EP);
        const uint32_t edx = ep, edw = ep + C::EP_DX, edm = ep + C::EP_DX + C::EP_DW;
        const uint32_t eam = ep + C::EP_DX + C::EP_DW + C::EP_DMIN, ebm = eam + C::EP_AMIN;
#pragma unroll
        for (int i = 0; i < TM; i++) {
            v4i amin = {};
            if constexpr (FMT == FMT_Q4_K) amin = ds_read128(eam + (wm * TM + i) * 1024 + lane * 16);
            v4i dx4[4];
#pragma unroll
            for (int g = 0; g < 4; g++) dx4[g] = ds_read128(edx + ((wm * TM + i) * 32 + 8 * g + 4 * lhalf) * 4);
            // exact integer sum in place of the lo limb (the hi limb is dead after this)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int rr = 0; rr < 16; rr++) alo[i][j][rr] += ahi[i][j][rr] << 7;
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int wc = (wn * TN + j) * 32 + lrow;
                float dw = ds_read32(edw + wc * 4), dmn = 0.0f;
                v4i bmin = {};
                if constexpr (FMT == FMT_Q4_K) {
                    dmn = ds_read32(edm + wc * 4);
                    bmin = ds_read128(ebm + (wn * TN + j) * 1024 + lane * 16);
                }
                // the asm reads above complete here; the operands tie every result to the wait
                if (j == 0)
                    asm volatile("s_waitcnt lgkmcnt(0)"
                                 : "+v"(dx4[0]), "+v"(dx4[1]), "+v"(dx4[2]), "+v"(dx4[3]), "+v"(amin), "+v"(bmin),
                                   "+v"(dw), "+v"(dmn));
                else
                    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(bmin), "+v"(dw), "+v"(dmn));
                v16f fmin = {};
                if constexpr (FMT == FMT_Q4_K)
                    fmin = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, amin),
                                                                 __builtin_bit_cast(v8h, bmin), (v16f){}, 0, 0, 0);
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const float4 d4 = __builtin_bit_cast(float4, dx4[g]);
                    const float dxs[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const int rr = 4 * g + q;
                        float tv = dw * (float)alo[i][j][rr];
                        if constexpr (FMT == FMT_Q4_K) tv -= dmn * fmin[rr];
                        acc[i][j][rr] += dxs[q] * tv;
                    }
                }
                alo[i][j] = (v16i){};
                ahi[i][j] = (v16i){};
            }
        }
    };

#pragma unroll
    for (int x = 0; x < DIST; x++) issue(x);
    // UNR stages per iteration (a whole superblock for the K-quants), so the
    // stage slot and the DMA count still in flight are constants per position.
    constexpr int UNR = C::limbs ? SPB : NBUF;
    static_assert(UNR % NBUF == 0, "slot of each unrolled stage is its position modulo NBUF");
    for (int s0 = 0; s0 < nst; s0 += UNR) {
        static_for<0, UNR>([&](auto qc) __attribute__((always_inline)) {
            constexpr int q = decltype(qc)::value;
            const int s = s0 + q;
            if (C::limbs || s < nst) {  // nst is a multiple of NBUF/2 (Q8_0 / F16), of SPB (K-quants)
                // stage s has landed once only the DMAs of stages s+1 .. s+DIST-1 are outstanding
                wait_vmcnt_c<C::template waits<DIST>(q)>();
                barrier_nofence();  // stage s landed for every wave; stage s-1 fully consumed
                issue(s + DIST);
                // s0 is a multiple of NBUF: stage s sits in slot q % NBUF
                if constexpr (FMT == FMT_Q8_0 && (MINB >= 4 || KG > 1)) compute_q8_0_occ(std::integral_constant<int, q % NBUF>{});
                else compute(smem + (q % NBUF) * C::STAGE);
            }
        });
        if constexpr (C::limbs) epilogue(s0 / SPB);
    }
    if constexpr (KG > 1) {
        // K groups 1 .. KG-1 hand their partial sums to group 0 through LDS (the ring, once every
        // wave's DMAs have landed and every wave is past its last stage); group 0 adds them in
        // group order and stores.  The other groups end here: a later workgroup barrier (the
        // quantized-output and K/V-fragment stores) waits for the waves still running.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        float *part = (float *)smem;
        if (kg > 0) {
#pragma unroll
            for (int rr = 0; rr < 16; rr++) part[(((kg - 1) * C::NTW + wt) * 16 + rr) * 64 + lane] = acc[0][0][rr];
        }
        __syncthreads();
        if (kg > 0) return;  // uniform per wave
#pragma unroll
        for (int g = 1; g < KG; g++)
#pragma unroll
            for (int rr = 0; rr < 16; rr++) acc[0][0][rr] += part[(((g - 1) * C::NTW + wt) * 16 + rr) * 64 + lane];
    }
    // the bias of the lane's output columns, loaded before the wait below so that its latency
    // overlaps the last DMAs instead of stalling the stores
    float bv[TN];
#pragma unroll
    for (int j = 0; j < TN; j++) {
        const int col = GLU ? wtile<GLU>(a, n0, wn * TN + j) * 32 + lrow : n0 + (wn * TN + j) * 32 + lrow;
        bv[j] = (a.bias && col < a.N) ? a.bias[col] : 0.f;
    }
    // no DMA may still be writing this workgroup's LDS when it exits
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // the bias goes into the accumulators in one uniform block: used inside the exec-masked
    // store blocks below, each of them would get its own wait for the load, and a wait for
    // the load is a wait for every store issued before it (vmcnt counts both)
    if (a.bias) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int rr = 0; rr < 16; rr++) acc[i][j][rr] += bv[j];
    }

    if constexpr (GLU) {
        // silu(gate) * up of the wave's 32 features (column tile 0: gate, 1: up, same layout)
        const int col = ((n0 >> 6) + wn) * 32 + lrow;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int rr = 0; rr < 16; rr++) {
                const int row = m0 + (wm * TM + i) * 32 + 8 * (rr >> 2) + 4 * lhalf + (rr & 3);
                if (row < a.M) a.y[(int64_t)row * a.ldy + col] = silu_mul_f32(acc[i][0][rr], acc[i][1][rr]);
            }
        return;
    }

    if (a.qo && a.q_fmt == 1) {
        // Q8_K output: the workgroup's BN = 256 columns are one superblock of the next product's
        // K, so every row's Q8_K block is formed here.  The waves stage the BM x 256 tile in LDS
        // as op(acc + bias) (rows past M as zeros, the activation quantizer's pad rows), then
        // each wave quantizes RQ rows as k_quantize_tiled<TQ_Q8_K> does (q8_K_rows: the same
        // bytes), storing its 4 quants per lane and row in place in the fragments; the min-term
        // fragments and scales leave from LDS at the end.
        if constexpr (C::BN == 256 && C::BM % C::NW == 0 && 32 % (C::BM / C::NW) == 0 && (C::BM / C::NW) % 8 == 0) {
            constexpr int RQ = C::BM / C::NW, NTL = C::BM / 32;  // rows per wave, 32-row tiles
            static_assert(C::LDS_Q8K <= C::LDS, "Q8_K staging fits");
            float *stg = (float *)smem;                                  // [BM][256]
            _Float16 *msh = (_Float16 *)(smem + C::BM * 1024);           // [NTL][512]
            float *dsh = (float *)(smem + C::BM * 1024 + NTL * 1024);    // [BM]
            const int kb = n0 >> 8;  // the superblock along the next product's K
            __syncthreads();         // every wave past its last stage: the ring is free
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
#pragma unroll
                    for (int rr = 0; rr < 16; rr++) {
                        const int rl = (wm * TM + i) * 32 + 8 * (rr >> 2) + 4 * lhalf + (rr & 3);
                        float x = acc[i][j][rr];
                        if (a.q_pre == MQ_PRE_GELU_ERF) x = gelu_erf_f32(x);
                        stg[rl * 256 + (wn * TN + j) * 32 + lrow] = m0 + rl < a.M ? x : 0.f;
                    }
            __syncthreads();
            const int rl0 = wave * RQ, tl = rl0 >> 5, rt = (m0 >> 5) + tl;  // the wave's rows: one tile
            const int c = lane >> 3, cbyte = (4 * lane) & 31;
            int8_t *qdst = a.qo + (((int64_t)rt * a.q_kch + kb * 8 + c) << 10) + (32 * (cbyte >> 4) << 4) + (cbyte & 15);
            const bool live = rt * 32 < a.q_m_pad;  // uniform
#pragma unroll
            for (int r8 = 0; r8 < RQ; r8 += 8) {
                float4 v[8];
                uint32_t q[8];
                int bs[8];
                float d[8];
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] = *(const float4 *)(stg + (rl0 + r8 + i) * 256 + 4 * lane);
                q8_K_rows<8>(v, lane, q, bs, d);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const int r = (rl0 + r8 + i) & 31;  // row within the tile
                    if (live) *(uint32_t *)(qdst + (r << 4)) = q[i];
                    if (lane == 0) dsh[rl0 + r8 + i] = d[i];
                    if ((lane & 7) == 0) {
                        const int jj = lane >> 3;
                        msh[tl * 512 + (r << 3) + jj] = (_Float16)(bs[i] & 63);
                        msh[tl * 512 + ((32 + r) << 3) + jj] = (_Float16)((bs[i] >> 6) * 64);
                    }
                }
            }
            __syncthreads();
            const int t = threadIdx.x;
            if (t < C::BM && m0 + t < a.q_m_pad) a.qd[(int64_t)kb * a.q_m_pad + m0 + t] = dsh[t];
            if (t < NTL * 64) {
                const int tt = t >> 6, rtt = (m0 >> 5) + tt;
                if (rtt * 32 < a.q_m_pad)
                    ((int4 *)(a.qmin + (((int64_t)rtt * a.q_ncb + kb) << 9)))[t & 63] = ((const int4 *)(msh + tt * 512))[t & 63];
            }
        }
        return;
    }

    if (a.qo) {
        // Quantized output.  Each wave stages a 32x32 tile in LDS (the stage ring is free once
        // every wave is past its last stage), then lane l takes row l % 32, values
        // 16 (l / 32) .. +15 of it: exactly the 16 bytes lane l owns in the tile's 1 KB
        // fragment, so the fragment leaves as one coalesced store per wave.
        constexpr int QST = 36;  // staging row stride in floats (16-byte aligned rows, spread banks)
        static_assert(C::LDS >= C::NW * 32 * QST * 4, "staging tiles fit in the stage ring");
        __syncthreads();
        float *tile = (float *)smem + wave * (32 * QST);
        const int qr = lane & 31, qh = lane >> 5;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int rt = (m0 >> 5) + wm * TM + i;  // 32-row tile of the output
                const int kb = (n0 >> 5) + wn * TN + j;  // its Q8_0 block along the next product's K
                if (rt * 32 >= a.q_m_pad || kb >= a.q_kch) continue;  // uniform
#pragma unroll
                for (int rr = 0; rr < 16; rr++)
                    tile[(8 * (rr >> 2) + 4 * lhalf + (rr & 3)) * QST + lrow] = acc[i][j][rr];
                // other lanes' values are read back: keep the compiler from moving the reads
                // above the writes (the LDS itself serves one wave's accesses in order)
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                float v[16];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const float4 t4 = *(const float4 *)(tile + qr * QST + 16 * qh + 4 * u);
                    v[4 * u] = t4.x, v[4 * u + 1] = t4.y, v[4 * u + 2] = t4.z, v[4 * u + 3] = t4.w;
                }
                const int row = rt * 32 + qr;
                uint4 q;
                const float d = requant_q8_0(v, row < a.M, a.q_pre, a.q_var, q);
                *(uint4 *)(a.qo + (((int64_t)rt * a.q_kch + kb) << 10) + lane * 16) = q;
                if (qh == 0) a.qd[(int64_t)kb * a.q_m_pad + row] = d;
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
        return;
    }

    // K / V fragments for the attention: K (attention A operand, lane = key) is transposed
    // through a per-wave LDS tile, V (lane = head dim, register 8 t + j = key 16 t + ...) is
    // already in its fragment order in the accumulators.
    constexpr int KST = 36;
    if (a.kvf) __syncthreads();  // the stage ring becomes the staging area (uniform branch)
    float *ktile = (float *)smem + wave * (32 * KST);
    auto kv_store = [&](int i, int j) __attribute__((always_inline)) {
        const int row0 = m0 + (wm * TM + i) * 32, cb = n0 + (wn * TN + j) * 32;
        const int b = row0 / a.kv_T, kb = (row0 - b * a.kv_T) >> 5;
        const int hdk = a.kv_nkv * a.kv_hd, c = cb - a.kv_col0;
        const bool isv = c >= hdk;
        const int cc = isv ? c - hdk : c, hk = cc / a.kv_hd, dn = cc - hk * a.kv_hd;
        const int ns = a.kv_hd >> 4, nt = a.kv_hd >> 5, nfr = 2 * ns + 4 * nt;
        _Float16 *F = a.kvf + ((int64_t)(b * a.kv_nkv + hk) * a.kv_nblk + kb) * nfr * 512 + lane * 8;
        if (isv) {
#pragma unroll
            for (int t = 0; t < 2; t++) {
                float x[8];
#pragma unroll
                for (int e = 0; e < 8; e++) x[e] = acc[i][j][8 * t + e];
                v8h h, l;
                split8(x, h, l);
                const int f = t * nt + (dn >> 5);
                *(v8h *)(F + (2 * ns + 2 * f) * 512) = h;
                *(v8h *)(F + (2 * ns + 2 * f + 1) * 512) = l;
            }
        } else {
#pragma unroll
            for (int rr = 0; rr < 16; rr++)
                ktile[(8 * (rr >> 2) + 4 * lhalf + (rr & 3)) * KST + lrow] = acc[i][j][rr];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int sp = 0; sp < 2; sp++) {
                const float4 u = *(const float4 *)(ktile + lrow * KST + 16 * sp + 8 * lhalf);
                const float4 w = *(const float4 *)(ktile + lrow * KST + 16 * sp + 8 * lhalf + 4);
                const float x[8] = {u.x, u.y, u.z, u.w, w.x, w.y, w.z, w.w};
                v8h h, l;
                split8(x, h, l);
                const int st = (dn >> 4) + sp;
                *(v8h *)(F + (2 * st) * 512) = h;
                *(v8h *)(F + (2 * st + 1) * 512) = l;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    };

    // store: lanes 0..31 of a register write 32 consecutive floats of one row.
    // (Staging the tile through LDS for 16-byte row stores was measured slower on
    // MI355X: the extra barrier and LDS pass cost more than the store instructions.)
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            if (a.kvf && n0 + (wn * TN + j) * 32 >= a.kv_col0) {  // uniform per wave
                if (m0 + (wm * TM + i) * 32 < a.M && n0 + (wn * TN + j) * 32 < a.N) kv_store(i, j);
                continue;
            }
            const int col = n0 + (wn * TN + j) * 32 + lrow;
            if (col >= a.N) continue;
#pragma unroll
            for (int rr = 0; rr < 16; rr++) {
                const int row = m0 + (wm * TM + i) * 32 + 8 * (rr >> 2) + 4 * lhalf + (rr & 3);
                if (row < a.M) a.y[(int64_t)row * a.ldy + col] = acc[i][j][rr];
            }
        }
}

template <int FMT, int WM, int WN, int TM, int TN, int MINB, int KCT = 2, bool GLU = false, int NBT = 4, int DT = 3,
          int KG = 1>
static hipError_t launch_cfg(GemmArgs a, hipStream_t s) {
    using C = Cfg<FMT, WM, WN, TM, TN, KCT, NBT, DT, KG>;
    if (KG > 1 && ((a.qo && a.q_fmt == 1) || a.moe)) return hipErrorInvalidValue;  // K groups: BN 64, no expert tiles
    static std::atomic<bool> attr_set[MQ_MAX_DEVICES];
    const hipError_t e = dyn_lds_once((const void *)k_gemm<FMT, WM, WN, TM, TN, MINB, KCT, GLU, NBT, DT, KG>, C::LDS, attr_set);
    if (e != hipSuccess) return e;
    a.tiles_m = (a.M + C::BM - 1) / C::BM;
    a.tiles_n = (a.N + C::BN - 1) / C::BN;
    for (int g = 1; g < GEMM_GROUPS; g++) {
        a.tn_start[g] = g < a.ngroups ? a.tiles_n : INT_MAX;
        if (g < a.ngroups) a.tiles_n += (a.grp[g - 1].N + C::BN - 1) / C::BN;
    }
    a.group_m = 8;
    a.nstages = a.kch / KCT;  // kb_pad is a multiple of 128 bytes
    const unsigned grid = (unsigned)(a.tiles_m * a.tiles_n);
    hipLaunchKernelGGL((k_gemm<FMT, WM, WN, TM, TN, MINB, KCT, GLU, NBT, DT, KG>), dim3(grid), dim3(C::NT), C::LDS, s, a);
    return hipGetLastError();
}

// Tile configuration, selectable with MQ_GEMM_CFG for measurements:
//   1: 8 waves x (64x64)  WG 256x128, 2 waves/SIMD
//   3: 4 waves x (64x64)  WG 128x128, 2 WGs/CU
//   4: 2 waves x (64x64)  WG 128x64
//   5: 1 wave  x (64x64)  WG 64x64
//   6: 4 waves x (64x64)  WG 128x128, 32-byte K stages: 70 KB of LDS, two workgroups per CU
//      (K-quants)
//   7: 4 waves x (32x32)  WG 64x64
//   8: as 7 with a 2-stage ring (one stage in flight): half the LDS, more workgroups per CU
//   9: as 7 with a 3-stage ring (two in flight; Q8_0 and F16)
//  12: as 8 within 80 registers, six workgroups per CU, one block at a time (Q8_0)
//  11: 8 waves x (64x64)  WG 128x256, 32-byte K stages (K-quants; the Q8_K-output GEMM's tiles)
//  15: WG 32x64: 2 waves x (32x32) x 4 K groups, 128-byte K stages, 3-stage ring (Q8_0; not
//      the Q8_K output)
static int gemm_cfg_env() {
    const char *e = getenv("MQ_GEMM_CFG");  // read per launch so a process can compare configurations
    return (e && *e) ? atoi(e) : 0;
}

static inline int64_t tiles(int64_t M, int64_t N, int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); }

template <int FMT>
static hipError_t launch_fmt(GemmArgs a, hipStream_t s) {
    int cfg = gemm_cfg_env();
    const bool kg_ok = !(a.qo && a.q_fmt == 1) && !a.moe;  // outputs the K-group forms (BN = 64) store
    if (cfg < 1 || cfg > 15 || cfg == 2 || cfg == 10 || cfg == 13 || cfg == 14 || (cfg == 11 && FMT != FMT_Q4_K && FMT != FMT_Q6_K) || (cfg == 6 && FMT != FMT_Q4_K && FMT != FMT_Q6_K) ||
        (cfg == 9 && FMT != FMT_Q8_0 && FMT != FMT_F16) || (cfg == 12 && FMT != FMT_Q8_0) ||
        (cfg == 15 && (FMT != FMT_Q8_0 || !kg_ok))) {
        // Small grids (under 512 tiles of 128x128): 64x64 workgroups of four 32x32 waves.
        // Every 32-deep K chunk costs a wave VALU work per output of its tile (the block
        // scales), so smaller wave tiles shorten the serial chain each wave walks; with few
        // output tiles that chain, not operand reuse, sets the time (MI355X, Q8_0 4096x384x1536
        // 32 -> 17 us, Q4_K 512x1024x3072 37 -> 16 us).  For Q8_0 with a 2-stage ring: half the
        // LDS, twice the workgroups per CU (17.9 -> 16.2 us at 4096x1536x384; the K-quants and
        // F16 measured slower with it at 512 rows).  Q8_0 grids of 768 or more such workgroups:
        // the one-block-at-a-time form within 80 registers, all of them resident at once
        // (4096x1536x384 16.4 -> 15.6 us, 4096x1152x384 15.0 -> 13.6 us; equal at 768).
        // Fewer Q8_0 tiles with K >= 768 or at most 1024 rows: 32x64 workgroups whose K chunks
        // are split over four wave groups, so more waves share each tile's serial chain
        // (4096x384x1536 18.2 -> 15.3 us, 384x384x1536 13.3 -> 8.1 us, 384x384x384 5.9 -> 4.9
        // us, 384x1152x384 6.1 -> 5.1 us; not at 4096x384x384, 7.9 against 8.1 us), whatever the
        // output (floats, the next product's Q8_0 activation, attention fragments), so the
        // outputs of one product come from the same sums; below 768 tiles the choice depends on
        // M and K only, so a grouped launch and its products' separate launches agree there.
        // Larger grids: 256x128 tiles when that still gives every CU (256) a workgroup, else
        // 128x128.
        int64_t n_all = a.N;
        for (int g = 1; g < a.ngroups; g++) n_all += a.grp[g - 1].N;
        if (tiles(a.M, n_all, 128, 128) < 512) {
            if (FMT != FMT_Q8_0) cfg = 7;
            else if (tiles(a.M, n_all, 64, 64) >= 768) cfg = 12;
            else if (!kg_ok) cfg = 8;
            else cfg = (a.kch >= 24 || a.M <= 1024) ? 15 : 8;
        } else {
            cfg = (tiles(a.M, n_all, 256, 128) >= 256) ? 1 : 3;
        }
    }
    switch (cfg) {
        case 1: return launch_cfg<FMT, 4, 2, 2, 2, 1>(a, s);
        case 3: return launch_cfg<FMT, 2, 2, 2, 2, 2>(a, s);
        case 4: return launch_cfg<FMT, 2, 1, 2, 2, 2>(a, s);
        case 6:
            if constexpr (FMT == FMT_Q4_K || FMT == FMT_Q6_K) return launch_cfg<FMT, 2, 2, 2, 2, 2, 1>(a, s);
            return hipErrorInvalidValue;

        case 7: return launch_cfg<FMT, 2, 2, 1, 1, 2>(a, s);
        case 8: return launch_cfg<FMT, 2, 2, 1, 1, 2, 2, false, 2, 1>(a, s);
        case 9:
            if constexpr (FMT == FMT_Q8_0 || FMT == FMT_F16) return launch_cfg<FMT, 2, 2, 1, 1, 2, 2, false, 3, 2>(a, s);
            return hipErrorInvalidValue;
        case 11:
            if constexpr (FMT == FMT_Q4_K || FMT == FMT_Q6_K) return launch_cfg<FMT, 2, 4, 2, 2, 1, 1, false, 4, 3>(a, s);
            return hipErrorInvalidValue;
        case 15:
            if constexpr (FMT == FMT_Q8_0) return launch_cfg<FMT, 1, 2, 1, 1, 3, 4, false, 3, 2, 4>(a, s);
            return hipErrorInvalidValue;
        case 12:
            if constexpr (FMT == FMT_Q8_0) return launch_cfg<FMT, 2, 2, 1, 1, 6, 2, false, 2, 1>(a, s);
            return hipErrorInvalidValue;


        default: return launch_cfg<FMT, 1, 1, 2, 2, 2>(a, s);
    }
}

static hipError_t gemm_group_kv(int type, int ngroups, const void *const *images, const int64_t *n, int64_t k,
                                const void *ws, int64_t m, float *const *y, const int64_t *ldy,
                                const float *const *bias, const int *kv_col0, _Float16 *kvf, int T, int hd, int nkv,
                                hipStream_t s);

hipError_t launch_gemm_group(int type, int ngroups, const void *const *images, const int64_t *n, int64_t k,
                             const void *ws, int64_t m, float *const *y, const int64_t *ldy, const float *const *bias,
                             hipStream_t s) {
    return gemm_group_kv(type, ngroups, images, n, k, ws, m, y, ldy, bias, nullptr, nullptr, 0, 0, 0, s);
}

hipError_t launch_gemm_qkv(int type, const void *const *images, const int64_t *n, int64_t k, const void *ws, int64_t m,
                           float *yq, int64_t ldyq, const float *const *bias, int T, int hd, int nkv, void *kv_frags,
                           hipStream_t s) {
    if (T <= 0 || T % 32 || m % T || (hd != 32 && hd != 64 && hd != 128) || n[1] != (int64_t)nkv * hd ||
        n[2] != n[1] || n[0] <= 0 || ((uintptr_t)kv_frags & 15))
        return hipErrorInvalidValue;
    // group 0 (Q) stores floats; group 1 (K) and group 2 (V) leave as fragments
    const int col0[3] = {INT_MAX, 0, -(int)n[1]};
    float *y[3] = {yq, nullptr, nullptr};
    const int64_t ld[3] = {ldyq, n[1], n[2]};
    return gemm_group_kv(type, 3, images, n, k, ws, m, y, ld, bias, col0, (_Float16 *)kv_frags, T, hd, nkv, s);
}

static hipError_t gemm_group_kv(int type, int ngroups, const void *const *images, const int64_t *n, int64_t k,
                                const void *ws, int64_t m, float *const *y, const int64_t *ldy,
                                const float *const *bias, const int *kv_col0, _Float16 *kvf, int T, int hd, int nkv,
                                hipStream_t s) {
    if (ngroups < 1 || ngroups > GEMM_GROUPS) return hipErrorInvalidValue;
    if (m <= 0) return hipSuccess;
    const ActPlanes ap = act_planes(type, m, k, true);
    const uint8_t *xb = (const uint8_t *)ws;
    GemmArgs a{};
    a.xq = (const int8_t *)(xb + ap.xq);
    a.xd = (const float *)(xb + ap.xd);
    a.xmin = (const _Float16 *)(xb + ap.xmin);
    a.M = (int)m;
    a.m_pad = (int)ap.m_pad;
    a.nsb = (int)(k / QK_K);
    // groups with n = 0 are dropped
    int ng = 0;
    for (int g = 0; g < ngroups; g++) {
        if (n[g] <= 0) continue;
        const WeightPlanes p = weight_planes(type, n[g], k);
        const uint8_t *wb = (const uint8_t *)images[g];
        GemmArgs::Group G;
        G.wq = (const int8_t *)(wb + p.tq);
        G.whi = (const int8_t *)(wb + p.thi);
        G.wd = (const float *)(wb + p.tdw);
        G.wdmin = (const float *)(wb + p.tdmin);
        G.wmin = (const _Float16 *)(wb + p.tmin);
        G.y = y[g];
        G.bias = bias ? bias[g] : nullptr;
        G.N = (int)n[g];
        G.n_pad = (int)p.n_pad;
        G.ldy = (int)ldy[g];
        G.kv_col0 = kv_col0 ? kv_col0[g] : INT_MAX;
        if (ng == 0) {
            a.wq = G.wq, a.whi = G.whi, a.wd = G.wd, a.wdmin = G.wdmin, a.wmin = G.wmin;
            a.y = G.y, a.bias = G.bias, a.N = G.N, a.n_pad = G.n_pad, a.ldy = G.ldy, a.kv_col0 = G.kv_col0;
            a.kch = (int)(p.kb_pad / 32);
            a.nstages = (int)(p.kb_pad / 64);  // set again per configuration
        } else {
            a.grp[ng - 1] = G;
        }
        ng++;
    }
    if (ng == 0) return hipSuccess;
    a.ngroups = ng;
    if (kvf) {
        if (ng != ngroups) return hipErrorInvalidValue;  // no empty group among q, k, v
        a.kvf = kvf;
        a.kv_T = T, a.kv_hd = hd, a.kv_nkv = nkv, a.kv_nblk = T / 32;
    }
    switch (type) {
        case MQ_TYPE_Q8_0: return launch_fmt<FMT_Q8_0>(a, s);
        case MQ_TYPE_Q4_K: return launch_fmt<FMT_Q4_K>(a, s);
        case MQ_TYPE_Q6_K: return launch_fmt<FMT_Q6_K>(a, s);
        case MQ_TYPE_F16: return launch_fmt<FMT_F16>(a, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemm(int type, const void *image, int64_t n, int64_t k, const void *ws, int64_t m, float *y,
                       int64_t ldy, hipStream_t s, const float *bias) {
    return launch_gemm_group(type, 1, &image, &n, k, ws, m, &y, &ldy, &bias, s);
}

// The experts' GEMM of a device-routed MUL_MAT_ID: rows sorted by expert in segments of whole
// moe_tile_rows-row tiles (x quantized in the tiled layout for m_rows rows), the tile table in
// moe (moe[0] live tiles, moe[1 + t] the expert of tile t), expert e's weight image at
// images + e * stride.  moe_tile_rows 256: the 256 x 128 workgroups; 64: 64 x 64.
int gemm_moe_tile_rows(int64_t rows, int64_t n, int n_used_experts) {
    return (rows >= (int64_t)1024 * n_used_experts && tiles(rows, n, 256, 128) >= 256) ? 256 : 64;
}

hipError_t launch_gemm_moe(int type, const void *images, size_t stride, int64_t n, int64_t k, const void *ws,
                           int64_t m_rows, int tile_rows, const int *moe, float *y, hipStream_t s) {
    if (m_rows <= 0 || n <= 0) return hipSuccess;
    if (m_rows % tile_rows || (tile_rows != 64 && tile_rows != 256) || stride % 256) return hipErrorInvalidValue;
    const ActPlanes ap = act_planes(type, m_rows, k, true);
    const WeightPlanes p = weight_planes(type, n, k);
    const uint8_t *xb = (const uint8_t *)ws, *wb = (const uint8_t *)images;
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
    a.moe = moe;
    a.moe_stride = (int64_t)stride;
    a.M = (int)m_rows;
    a.N = (int)n;
    a.ldy = (int)n;
    a.m_pad = (int)ap.m_pad;
    a.n_pad = (int)p.n_pad;
    a.kch = (int)(p.kb_pad / 32);
    a.nstages = (int)(p.kb_pad / 64);
    a.nsb = (int)(k / QK_K);
    a.ngroups = 1;
    const bool big = tile_rows == 256;
    switch (type) {
        case MQ_TYPE_Q8_0:
            return big ? launch_cfg<FMT_Q8_0, 4, 2, 2, 2, 1>(a, s) : launch_cfg<FMT_Q8_0, 2, 2, 1, 1, 2, 2, false, 2, 1>(a, s);
        case MQ_TYPE_Q4_K: return big ? launch_cfg<FMT_Q4_K, 4, 2, 2, 2, 1>(a, s) : launch_cfg<FMT_Q4_K, 2, 2, 1, 1, 2>(a, s);
        case MQ_TYPE_Q6_K: return big ? launch_cfg<FMT_Q6_K, 4, 2, 2, 2, 1>(a, s) : launch_cfg<FMT_Q6_K, 2, 2, 1, 1, 2>(a, s);
        case MQ_TYPE_F16: return big ? launch_cfg<FMT_F16, 4, 2, 2, 2, 1>(a, s) : launch_cfg<FMT_F16, 2, 2, 1, 1, 2>(a, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemm_kv(int type, const void *image, int64_t n, int64_t k, const void *ws, int64_t m, float *y,
                          int64_t ldy, const float *bias, int kv_col0, int T, int hd, int nkv, void *kv_frags,
                          hipStream_t s) {
    if (m <= 0 || n <= 0) return hipSuccess;
    if (T <= 0 || T % 32 || m % T || (hd != 32 && hd != 64 && hd != 128) || kv_col0 % 32 ||
        (int64_t)kv_col0 + 2 * (int64_t)nkv * hd != n || ((uintptr_t)kv_frags & 15))
        return hipErrorInvalidValue;
    const ActPlanes ap = act_planes(type, m, k, true);
    const WeightPlanes p = weight_planes(type, n, k);
    const uint8_t *xb = (const uint8_t *)ws, *wb = (const uint8_t *)image;
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
    a.bias = bias;
    a.kvf = (_Float16 *)kv_frags;
    a.kv_col0 = kv_col0, a.kv_T = T, a.kv_hd = hd, a.kv_nkv = nkv, a.kv_nblk = T / 32;
    a.M = (int)m;
    a.N = (int)n;
    a.ldy = (int)ldy;
    a.m_pad = (int)ap.m_pad;
    a.n_pad = (int)p.n_pad;
    a.kch = (int)(p.kb_pad / 32);
    a.nstages = (int)(p.kb_pad / 64);
    a.nsb = (int)(k / QK_K);
    a.ngroups = 1;
    switch (type) {
        case MQ_TYPE_Q8_0: return launch_fmt<FMT_Q8_0>(a, s);
        case MQ_TYPE_Q4_K: return launch_fmt<FMT_Q4_K>(a, s);
        case MQ_TYPE_Q6_K: return launch_fmt<FMT_Q6_K>(a, s);
        case MQ_TYPE_F16: return launch_fmt<FMT_F16>(a, s);
        default: return hipErrorInvalidValue;
    }
}

// Q8_K output: 128 x 256 workgroups (8 waves of 64 x 64, 32-byte K stages in a 4-stage ring),
// a workgroup per 256-value superblock of the output rows; grids of at least one workgroup per
// CU.  MI355X, Q4_K 8192 x 4096 x 1024 with GELU-erf: 144 us, against 110 us for the plain
// 256 x 128 GEMM plus 37.5 us for the quantizer pass over its fp32 output (the epilogue's GELU
// and quantization do not overlap MFMA work: one workgroup per CU; 64 x 256 tiles, two per CU,
// measured 164 us).
bool gemm_requant_q8k_fits(int type, int64_t m, int64_t n) {
    return (type == MQ_TYPE_Q4_K || type == MQ_TYPE_Q6_K) && m > 0 && n > 0 && n % QK_K == 0 &&
           tiles(m, n, 128, 256) >= 256 && n <= INT32_MAX;
}

hipError_t launch_gemm_requant(int type, const void *image, int64_t n, int64_t k, const void *ws, int64_t m,
                               const float *bias, int pre, int q8_0_variant, int out_type, void *out_ws, hipStream_t s) {
    if (m <= 0 || n <= 0) return hipSuccess;
    const bool q8k = out_type == MQ_TYPE_Q4_K || out_type == MQ_TYPE_Q6_K;
    if (!q8k && out_type != MQ_TYPE_Q8_0) return hipErrorInvalidValue;
    if (q8k && !gemm_requant_q8k_fits(type, m, n)) return hipErrorInvalidValue;
    if (n % KSTAGE != 0) return hipErrorInvalidValue;  // the output fills the next product's padded K
    const ActPlanes ap = act_planes(type, m, k, true), op = act_planes(out_type, m, n, true);
    if (op.kb_pad != n || op.m_pad != ap.m_pad) return hipErrorInvalidValue;
    const WeightPlanes p = weight_planes(type, n, k);
    const uint8_t *xb = (const uint8_t *)ws, *wb = (const uint8_t *)image;
    uint8_t *ob = (uint8_t *)out_ws;
    GemmArgs a{};
    a.xq = (const int8_t *)(xb + ap.xq);
    a.xd = (const float *)(xb + ap.xd);
    a.xmin = (const _Float16 *)(xb + ap.xmin);
    a.wq = (const int8_t *)(wb + p.tq);
    a.whi = (const int8_t *)(wb + p.thi);
    a.wd = (const float *)(wb + p.tdw);
    a.wdmin = (const float *)(wb + p.tdmin);
    a.wmin = (const _Float16 *)(wb + p.tmin);
    a.y = nullptr;
    a.bias = bias;
    a.qo = (int8_t *)(ob + op.xq);
    a.qd = (float *)(ob + op.xd);
    a.qmin = q8k ? (_Float16 *)(ob + op.xmin) : nullptr;
    a.q_m_pad = (int)op.m_pad;
    a.q_kch = (int)(n / 32);
    a.q_pre = pre;
    a.q_var = q8_0_variant;
    a.q_fmt = q8k ? 1 : 0;
    a.q_ncb = (int)(n / QK_K);
    a.M = (int)m;
    a.N = (int)n;
    a.ldy = (int)n;
    a.m_pad = (int)ap.m_pad;
    a.n_pad = (int)p.n_pad;
    a.kch = (int)(p.kb_pad / 32);
    a.nstages = (int)(p.kb_pad / 64);
    a.nsb = (int)(k / QK_K);
    a.ngroups = 1;
    if (q8k) {
        if (type == MQ_TYPE_Q4_K) return launch_cfg<FMT_Q4_K, 2, 4, 2, 2, 1, 1, false, 4, 3>(a, s);
        return launch_cfg<FMT_Q6_K, 2, 4, 2, 2, 1, 1, false, 4, 3>(a, s);
    }
    switch (type) {
        case MQ_TYPE_Q8_0: return launch_fmt<FMT_Q8_0>(a, s);
        case MQ_TYPE_Q4_K: return launch_fmt<FMT_Q4_K>(a, s);
        case MQ_TYPE_Q6_K: return launch_fmt<FMT_Q6_K>(a, s);
        case MQ_TYPE_F16: return launch_fmt<FMT_F16>(a, s);
        default: return hipErrorInvalidValue;
    }
}

// The gated FFN's gate|up GEMM with silu(gate) * up formed in its store (k_gemm<..., GLU>).  It
// runs on the large-grid configurations only (256x128 or 128x128 workgroups, whose waves hold
// 64-column pairs); shapes the launcher would give 64x64 workgroups are not fused.
bool gemm_swiglu_fits(int64_t m, int64_t n_ff) {
    return m > 0 && n_ff > 0 && n_ff % 64 == 0 && tiles(m, 2 * n_ff, 128, 128) >= 512 && 2 * n_ff <= INT32_MAX;
}

hipError_t launch_gemm_swiglu(int type, const void *image, int64_t n_ff, int64_t k, const void *ws, int64_t m, float *y,
                              int64_t ldy, hipStream_t s) {
    if (!gemm_swiglu_fits(m, n_ff) || ldy < n_ff) return hipErrorInvalidValue;
    const int64_t n = 2 * n_ff;
    const ActPlanes ap = act_planes(type, m, k, true);
    const WeightPlanes p = weight_planes(type, n, k);
    const uint8_t *xb = (const uint8_t *)ws, *wb = (const uint8_t *)image;
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
    a.nstages = (int)(p.kb_pad / 64);
    a.nsb = (int)(k / QK_K);
    a.ngroups = 1;
    int cfg = gemm_cfg_env();
    if (cfg != 1 && cfg != 3) cfg = (tiles(m, n, 256, 128) >= 256) ? 1 : 3;
    auto go = [&](auto fmt) -> hipError_t {
        constexpr int F = decltype(fmt)::value;
        if (cfg == 1) return launch_cfg<F, 4, 2, 2, 2, 1, 2, true>(a, s);
        return launch_cfg<F, 2, 2, 2, 2, 2, 2, true>(a, s);
    };
    switch (type) {
        case MQ_TYPE_Q8_0: return go(std::integral_constant<int, FMT_Q8_0>{});
        case MQ_TYPE_Q4_K: return go(std::integral_constant<int, FMT_Q4_K>{});
        case MQ_TYPE_Q6_K: return go(std::integral_constant<int, FMT_Q6_K>{});
        case MQ_TYPE_F16: return go(std::integral_constant<int, FMT_F16>{});
        default: return hipErrorInvalidValue;
    }
}

// Sustained int8 MFMA rate: each wave keeps 8 independent accumulator chains busy (a chain's
// next MFMA is 8 issues later, so the matrix pipe never waits on a result); the operands come
// from the thread index, the sums are written out so nothing is folded away.
__global__ __launch_bounds__(256) void k_mfma_probe(int iters, int *out) {
    const int t = threadIdx.x;
    const v4i a = {t, t * 3 + 1, t * 5 + 2, t * 7 + 3}, b = {t ^ 0x55, t + 9, t * 11, t ^ 0x33};
    v16i acc[8];
#pragma unroll
    for (int j = 0; j < 8; j++) acc[j] = (v16i){};
    for (int i = 0; i < iters; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[j], 0, 0, 0);
    int sum = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) sum += acc[j][0] + acc[j][15];
    out[blockIdx.x * blockDim.x + t] = sum;
}

hipError_t launch_mfma_probe(int iters, int *out, int ncu, hipStream_t s) {
    hipLaunchKernelGGL(k_mfma_probe, dim3((unsigned)ncu), dim3(256), 0, s, iters, out);
    return hipGetLastError();
}

}  // namespace mq
