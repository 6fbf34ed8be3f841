// mq_host_quant.cpp -- host weight quantization, the producer of GGUF blocks.
//
// Stands in for ggml_quantize_chunk(type, src, dst, 0, nrows, k, NULL) as
// CrispEmbed's tools/quantize.cpp:804-805 calls it, and for the from_float_ref
// trait the decoder's LoRA merge uses (src/decoder_embed.cpp:1149-1166).  With
// no importance matrix ggml runs its _ref quantizers; their published
// algorithms are restated here:
//   Q8_0  d = amax/127 (fp16), q = roundf(x / d)
//   Q4_K  per 32-value sub-block an asymmetric (scale, min) least-squares search
//         over 21 candidate inverse scales (rmin -1, step 0.1), 6-bit
//         quantization of scales and mins against the superblock maxima, then a
//         requantization pass with the stored fp16 d/dmin
//   Q6_K  per 16-value sub-block a symmetric search over 19 inverse scales
//         (nmax 32 +- 0.1*is, weights x^2), 8-bit scales against the largest
//         scale, requantization with the stored fp16 d
//   Q8_K  the activation quantizer (d = 1/iscale fp32, bsums)
//   F16   round to nearest even
// Compiled with -ffp-contract=off: each product and sum rounds separately.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "mq_internal.h"

namespace mq {
namespace host {

uint16_t fp32_to_fp16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    const int e = (int)(ax >> 23);
    if (e >= 113) {  // binary16 normal range (or overflow)
        if (e - 112 >= 31) return (uint16_t)(sign | 0x7c00u);
        uint32_t h = ((uint32_t)(e - 112) << 10) | ((ax >> 13) & 0x3ffu);
        const uint32_t rest = ax & 0x1fffu;
        h += (rest > 0x1000u) || (rest == 0x1000u && (h & 1u));
        return (uint16_t)(sign | h);
    }
    // binary16 subnormal: round(|f| * 2^24) to nearest even
    const uint32_t sig = (e == 0) ? (ax & 0x7fffffu) : ((ax & 0x7fffffu) | 0x800000u);
    const int sh = 126 - (e == 0 ? 0 : e);
    if (sh > 24) return (uint16_t)sign;
    uint32_t q = sig >> sh;
    const uint32_t rest = sig & ((1u << sh) - 1u), halfway = 1u << (sh - 1);
    q += (rest > halfway) || (rest == halfway && (q & 1u));
    return (uint16_t)(sign | q);
}

float fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    float mag;
    if (e == 0) mag = std::ldexp((float)m, -24);
    else if (e == 31) mag = m ? NAN : INFINITY;
    else mag = std::ldexp((float)(m | 0x400u), (int)e - 25);
    uint32_t bits;
    std::memcpy(&bits, &mag, 4);
    bits |= sign;
    std::memcpy(&mag, &bits, 4);
    return mag;
}

static inline int nearest_int(float f) {
    const float v = f + 12582912.f;
    int32_t i;
    std::memcpy(&i, &v, 4);
    return (i & 0x007fffff) - 0x00400000;
}

static inline int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

static void q8_0_row(const float *x, block_q8_0 *y, int64_t k) {
    for (int64_t b = 0; b < k / QK8_0; b++) {
        const float *xb = x + b * QK8_0;
        float amax = 0.f;
        for (int i = 0; i < QK8_0; i++) amax = std::max(amax, std::fabs(xb[i]));
        const float d = amax / 127.f;
        const float id = d != 0.f ? 1.0f / d : 0.0f;
        y[b].d = fp32_to_fp16(d);
        for (int i = 0; i < QK8_0; i++) y[b].qs[i] = (int8_t)std::round(xb[i] * id);
    }
}

static void q8_K_row(const float *x, block_q8_K *y, int64_t k) {
    for (int64_t b = 0; b < k / QK_K; b++) {
        const float *xb = x + b * QK_K;
        float amax = 0.f, vmax = 0.f;
        for (int i = 0; i < QK_K; i++) {
            if (std::fabs(xb[i]) > amax) {
                amax = std::fabs(xb[i]);
                vmax = xb[i];
            }
        }
        std::memset(&y[b], 0, sizeof(block_q8_K));
        if (amax == 0.f) continue;
        const float iscale = -127.f / vmax;
        for (int i = 0; i < QK_K; i++) y[b].qs[i] = (int8_t)std::min(127, nearest_int(iscale * xb[i]));
        for (int g = 0; g < 16; g++) {
            int s = 0;
            for (int i = 0; i < 16; i++) s += y[b].qs[16 * g + i];
            y[b].bsums[g] = (int16_t)s;
        }
        y[b].d = 1.0f / iscale;
    }
}

// Asymmetric search for one sub-block of 32 (nmax 15): returns the scale,
// writes levels L and the (non-negative) offset -min.
static float search_scale_min(const float *x, const float *w, uint8_t *L, float *neg_min) {
    constexpr int n = 32, nmax = 15, nstep = 20;
    constexpr float rmin = -1.f, rdelta = 0.1f;
    float lo = x[0], hi = x[0], sw = w[0], swx = w[0] * x[0];
    for (int i = 1; i < n; i++) {
        lo = std::min(lo, x[i]);
        hi = std::max(hi, x[i]);
        sw += w[i];
        swx += w[i] * x[i];
    }
    // (min/max above match the strict < / > scans: equal values change nothing)
    if (lo > 0) lo = 0;
    if (hi == lo) {
        std::fill(L, L + n, (uint8_t)0);
        *neg_min = -lo;
        return 0.f;
    }
    float iscale = nmax / (hi - lo);
    float scale = 1 / iscale;
    float best = 0;
    for (int i = 0; i < n; i++) {
        L[i] = (uint8_t)clampi(nearest_int(iscale * (x[i] - lo)), 0, nmax);
        const float diff = scale * L[i] + lo - x[i];
        best += w[i] * (diff * diff);
    }
    uint8_t Lc[n];
    for (int is = 0; is <= nstep; is++) {
        iscale = (rmin + rdelta * is + nmax) / (hi - lo);
        float sl = 0, sl2 = 0, sxl = 0;
        for (int i = 0; i < n; i++) {
            const int l = clampi(nearest_int(iscale * (x[i] - lo)), 0, nmax);
            Lc[i] = (uint8_t)l;
            sl += w[i] * l;
            sl2 += w[i] * l * l;
            sxl += w[i] * l * x[i];
        }
        const float D = sw * sl2 - sl * sl;
        if (!(D > 0)) continue;
        float cs = (sw * sxl - swx * sl) / D;
        float cm = (sl2 * swx - sl * sxl) / D;
        if (cm > 0) {
            cm = 0;
            cs = sxl / sl2;
        }
        float err = 0;
        for (int i = 0; i < n; i++) {
            const float diff = cs * Lc[i] + cm - x[i];
            err += w[i] * (diff * diff);
        }
        if (err < best) {
            std::memcpy(L, Lc, n);
            best = err;
            scale = cs;
            lo = cm;
        }
    }
    *neg_min = -lo;
    return scale;
}

static void unpack_scale_min(int j, const uint8_t *s, int &sc, int &mn) {
    if (j < 4) {
        sc = s[j] & 63;
        mn = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

static void q4_K_row(const float *x, block_q4_K *y, int64_t k) {
    for (int64_t b = 0; b < k / QK_K; b++, x += QK_K) {
        uint8_t L[QK_K];
        float scale[8], nmin[8], w[32];
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < 8; j++) {
            const float *xs = x + 32 * j;
            float s2 = 0;
            for (int l = 0; l < 32; l++) s2 += xs[l] * xs[l];
            const float av = std::sqrt(s2 / 32);
            for (int l = 0; l < 32; l++) w[l] = av + std::fabs(xs[l]);
            scale[j] = search_scale_min(xs, w, L + 32 * j, &nmin[j]);
            if (scale[j] > max_scale) max_scale = scale[j];
            if (nmin[j] > max_min) max_min = nmin[j];
        }
        const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
        const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
        uint8_t *s = y[b].scales;
        std::memset(s, 0, 12);
        for (int j = 0; j < 8; j++) {
            const uint8_t ls = (uint8_t)std::min<int>(63, (uint8_t)nearest_int(inv_scale * scale[j]));
            const uint8_t lm = (uint8_t)std::min<int>(63, (uint8_t)nearest_int(inv_min * nmin[j]));
            if (j < 4) {
                s[j] = ls;
                s[j + 4] = lm;
            } else {
                s[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
                s[j - 4] |= (uint8_t)((ls >> 4) << 6);
                s[j] |= (uint8_t)((lm >> 4) << 6);
            }
        }
        y[b].d = fp32_to_fp16(max_scale / 63.f);
        y[b].dmin = fp32_to_fp16(max_min / 63.f);
        const float D = fp16_to_fp32(y[b].d), DM = fp16_to_fp32(y[b].dmin);
        for (int j = 0; j < 8; j++) {
            int sc, mn;
            unpack_scale_min(j, s, sc, mn);
            const float dj = D * sc;
            if (!dj) continue;
            const float mj = DM * mn;
            for (int l = 0; l < 32; l++) L[32 * j + l] = (uint8_t)clampi(nearest_int((x[32 * j + l] + mj) / dj), 0, 15);
        }
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 32; l++) y[b].qs[32 * c + l] = (uint8_t)(L[64 * c + l] | (L[64 * c + 32 + l] << 4));
    }
}

// Symmetric search for one sub-block of 16 (nmax 32, weights x^2).
static float search_scale_sym(const float *x, int8_t *L) {
    constexpr int n = 16, nmax = 32;
    float amax = 0, vmax = 0;
    for (int i = 0; i < n; i++) {
        if (std::fabs(x[i]) > amax) {
            amax = std::fabs(x[i]);
            vmax = x[i];
        }
    }
    if (amax < 1e-15f) {
        std::fill(L, L + n, (int8_t)0);
        return 0.f;
    }
    float iscale = -nmax / vmax;
    float slx = 0, sl2 = 0;
    for (int i = 0; i < n; i++) {
        const int l = clampi(nearest_int(iscale * x[i]), -nmax, nmax - 1);
        L[i] = (int8_t)(l + nmax);
        const float w = x[i] * x[i];
        slx += w * x[i] * l;
        sl2 += w * l * l;
    }
    float scale = sl2 ? slx / sl2 : 0.0f;
    float best = scale * slx;
    for (int is = -9; is <= 9; is++) {
        if (is == 0) continue;
        iscale = -(nmax + 0.1f * is) / vmax;
        slx = sl2 = 0;
        for (int i = 0; i < n; i++) {
            const int l = clampi(nearest_int(iscale * x[i]), -nmax, nmax - 1);
            const float w = x[i] * x[i];
            slx += w * x[i] * l;
            sl2 += w * l * l;
        }
        if (sl2 > 0 && slx * slx > best * sl2) {
            for (int i = 0; i < n; i++) L[i] = (int8_t)(nmax + clampi(nearest_int(iscale * x[i]), -nmax, nmax - 1));
            scale = slx / sl2;
            best = scale * slx;
        }
    }
    return scale;
}

static void q6_K_row(const float *x, block_q6_K *y, int64_t k) {
    for (int64_t b = 0; b < k / QK_K; b++, x += QK_K) {
        int8_t L[QK_K];
        float scale[16];
        float max_scale = 0, max_abs = 0;
        for (int g = 0; g < 16; g++) {
            scale[g] = search_scale_sym(x + 16 * g, L + 16 * g);
            if (std::fabs(scale[g]) > max_abs) {
                max_abs = std::fabs(scale[g]);
                max_scale = scale[g];
            }
        }
        std::memset(&y[b], 0, sizeof(block_q6_K));
        if (max_abs < 1e-15f) continue;  // all-zero superblock: d = 0
        const float iscale = -128.f / max_scale;
        y[b].d = fp32_to_fp16(1 / iscale);
        for (int g = 0; g < 16; g++) y[b].scales[g] = (int8_t)std::min(127, nearest_int(iscale * scale[g]));
        const float D = fp16_to_fp32(y[b].d);
        for (int g = 0; g < 16; g++) {
            const float dg = D * y[b].scales[g];
            if (!dg) continue;
            for (int i = 0; i < 16; i++) L[16 * g + i] = (int8_t)(clampi(nearest_int(x[16 * g + i] / dg), -32, 31) + 32);
        }
        for (int half = 0; half < 2; half++) {
            const int8_t *Lh = L + 128 * half;
            uint8_t *ql = y[b].ql + 64 * half;
            uint8_t *qh = y[b].qh + 32 * half;
            for (int l = 0; l < 32; l++) {
                ql[l] = (uint8_t)((Lh[l] & 0xF) | ((Lh[l + 64] & 0xF) << 4));
                ql[l + 32] = (uint8_t)((Lh[l + 32] & 0xF) | ((Lh[l + 96] & 0xF) << 4));
                qh[l] = (uint8_t)(((Lh[l] >> 4) & 3) | (((Lh[l + 32] >> 4) & 3) << 2) | (((Lh[l + 64] >> 4) & 3) << 4) |
                                  (((Lh[l + 96] >> 4) & 3) << 6));
            }
        }
    }
}

static void f16_row(const float *x, uint16_t *y, int64_t k) {
    for (int64_t i = 0; i < k; i++) y[i] = fp32_to_fp16(x[i]);
}

size_t quantize_chunk(int type, const float *src, void *dst, int64_t nrows, int64_t k) {
    const int64_t bs = blck_size(type);
    if (!src || !dst || nrows < 0 || k <= 0 || bs == 0 || k % bs != 0) return 0;
    const size_t rs = row_size(type, k);
    auto work = [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; r++) {
            const float *x = src + r * k;
            uint8_t *y = (uint8_t *)dst + r * rs;
            switch (type) {
                case MQ_TYPE_Q8_0: q8_0_row(x, (block_q8_0 *)y, k); break;
                case MQ_TYPE_Q4_K: q4_K_row(x, (block_q4_K *)y, k); break;
                case MQ_TYPE_Q6_K: q6_K_row(x, (block_q6_K *)y, k); break;
                case MQ_TYPE_Q8_K: q8_K_row(x, (block_q8_K *)y, k); break;
                case MQ_TYPE_F16: f16_row(x, (uint16_t *)y, k); break;
                case MQ_TYPE_F32: std::memcpy(y, x, (size_t)k * 4); break;
                default: break;
            }
        }
    };
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const int64_t nt = std::min<int64_t>({(int64_t)hw, 64, std::max<int64_t>(1, nrows * k / (1 << 16))});
    if (nt <= 1) {
        work(0, nrows);
    } else {
        std::vector<std::thread> th;
        for (int64_t t = 0; t < nt; t++) th.emplace_back(work, nrows * t / nt, nrows * (t + 1) / nt);
        for (auto &t : th) t.join();
    }
    return rs * (size_t)nrows;
}

// Host dequantization of GGUF rows to fp32, as ggml's dequantize_row_* (the get_rows of an
// embedding table): Q8_0 d*q; Q4_K d*sc_j*q - dmin*m_j; Q6_K d*sc*(q6 - 32); F16 exact.
// Returns false for a type it does not decode.
bool dequantize_rows(int type, const void *src, float *dst, int64_t nrows, int64_t k) {
    const int64_t bs = blck_size(type);
    if (!src || !dst || nrows < 0 || k <= 0 || bs == 0 || k % bs != 0) return false;
    const size_t rs = row_size(type, k);
    for (int64_t r = 0; r < nrows; r++) {
        const uint8_t *x = (const uint8_t *)src + r * rs;
        float *y = dst + r * k;
        switch (type) {
            case MQ_TYPE_F32: std::memcpy(y, x, (size_t)k * 4); break;
            case MQ_TYPE_F16: {
                const uint16_t *h = (const uint16_t *)x;
                for (int64_t i = 0; i < k; i++) y[i] = fp16_to_fp32(h[i]);
                break;
            }
            case MQ_TYPE_Q8_0:
                for (int64_t b = 0; b < k / QK8_0; b++) {
                    const block_q8_0 &q = ((const block_q8_0 *)x)[b];
                    const float d = fp16_to_fp32(q.d);
                    for (int i = 0; i < QK8_0; i++) y[b * QK8_0 + i] = d * (float)q.qs[i];
                }
                break;
            case MQ_TYPE_Q4_K:
                for (int64_t b = 0; b < k / QK_K; b++) {
                    const block_q4_K &q = ((const block_q4_K *)x)[b];
                    const float d = fp16_to_fp32(q.d), dmin = fp16_to_fp32(q.dmin);
                    float *yb = y + b * QK_K;
                    for (int c = 0; c < 4; c++) {
                        int sc0, m0, sc1, m1;
                        unpack_scale_min(2 * c, q.scales, sc0, m0);
                        unpack_scale_min(2 * c + 1, q.scales, sc1, m1);
                        const float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
                        const float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
                        for (int l = 0; l < 32; l++) {
                            yb[64 * c + l] = d1 * (float)(q.qs[32 * c + l] & 0xF) - mm1;
                            yb[64 * c + 32 + l] = d2 * (float)(q.qs[32 * c + l] >> 4) - mm2;
                        }
                    }
                }
                break;
            case MQ_TYPE_Q6_K:
                for (int64_t b = 0; b < k / QK_K; b++) {
                    const block_q6_K &q = ((const block_q6_K *)x)[b];
                    const float d = fp16_to_fp32(q.d);
                    float *yb = y + b * QK_K;
                    for (int h = 0; h < 2; h++) {
                        const uint8_t *ql = q.ql + 64 * h, *qh = q.qh + 32 * h;
                        const int8_t *sc = q.scales + 8 * h;
                        for (int l = 0; l < 32; l++) {
                            const int is = l / 16;
                            const int q1 = (int)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                            const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                            const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                            const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                            yb[128 * h + l] = d * (float)sc[is] * (float)q1;
                            yb[128 * h + l + 32] = d * (float)sc[is + 2] * (float)q2;
                            yb[128 * h + l + 64] = d * (float)sc[is + 4] * (float)q3;
                            yb[128 * h + l + 96] = d * (float)sc[is + 6] * (float)q4;
                        }
                    }
                }
                break;
            default: return false;
        }
    }
    return true;
}

}  // namespace host
}  // namespace mq
