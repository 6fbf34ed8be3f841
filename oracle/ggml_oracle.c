/*
 * ggml_oracle.c -- CPU restatement of ggml's block-quantized MUL_MAT semantics.
 *
 * TEST INFRASTRUCTURE ONLY (the checker; see ggml_oracle.h for the parity
 * status of each function and the reference call sites it stands in for).
 * Compiled with -ffp-contract=off: each multiply and add rounds separately.
 */
#include "ggml_oracle.h"

#include <math.h>
#include <pthread.h>
#include <unistd.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* IEEE binary16 <-> binary32, written from the IEEE 754 definition.          */
/* ggml converts with F16C (_cvtss_sh, round-to-nearest-even) on x86 and with  */
/* an equivalent bit routine elsewhere; both are RNE with subnormals kept.     */
/* ------------------------------------------------------------------------- */
uint16_t or_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu)); /* NaN stays NaN */
    if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    const int32_t e = (int32_t)(ax >> 23); /* biased fp32 exponent */
    if (e >= 113) {
        /* normal in fp16 unless it overflows */
        const int32_t he = e - 127 + 15;
        if (he >= 31) return (uint16_t)(sign | 0x7c00u);
        uint32_t h = ((uint32_t)he << 10) | ((ax >> 13) & 0x3ffu);
        const uint32_t rem = ax & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++; /* carry may reach inf: correct */
        return (uint16_t)(sign | h);
    }
    /* fp16 subnormal range: result = round(|f| / 2^-24) */
    const uint32_t full = (e == 0) ? (ax & 0x7fffffu) : ((ax & 0x7fffffu) | 0x800000u);
    const int32_t shift = (e == 0) ? 126 : 126 - e; /* value = full * 2^(e-150) */
    if (shift > 24) return (uint16_t)sign;
    uint32_t m = full >> shift;
    const uint32_t rem = full & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (m & 1u))) m++;
    return (uint16_t)(sign | m);
}

float or_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    const uint32_t m = (uint32_t)h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {
            /* subnormal: m * 2^-24, normalise */
            int32_t ee = -1;
            uint32_t mm = m;
            do {
                ee++;
                mm <<= 1;
            } while ((mm & 0x400u) == 0);
            x = sign | ((uint32_t)(127 - 15 - ee) << 23) | ((mm & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e - 15 + 127) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ggml's nearest_int: adding 1.5*2^23 leaves round-half-even(f) in the low
 * mantissa bits; valid for |f| < 2^22. */
int or_nearest_int(float fval) {
    const float val = fval + 12582912.f;
    int32_t i;
    memcpy(&i, &val, 4);
    return (i & 0x007fffff) - 0x00400000;
}

/* Q4_K 6-bit scale/min unpacking from the 12-byte scales field. */
void or_get_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* ------------------------------------------------------------------------- */
/* type traits                                                                */
/* ------------------------------------------------------------------------- */
int64_t or_blck_size(int type) {
    switch (type) {
        case OR_TYPE_F32:
        case OR_TYPE_F16: return 1;
        case OR_TYPE_Q8_0: return OR_QK8_0;
        case OR_TYPE_Q4_K:
        case OR_TYPE_Q6_K:
        case OR_TYPE_Q8_K: return OR_QK_K;
        default: return 0;
    }
}

size_t or_type_size(int type) {
    switch (type) {
        case OR_TYPE_F32: return 4;
        case OR_TYPE_F16: return 2;
        case OR_TYPE_Q8_0: return sizeof(or_block_q8_0);
        case OR_TYPE_Q4_K: return sizeof(or_block_q4_K);
        case OR_TYPE_Q6_K: return sizeof(or_block_q6_K);
        case OR_TYPE_Q8_K: return sizeof(or_block_q8_K);
        default: return 0;
    }
}

size_t or_row_size(int type, int64_t k) {
    const int64_t b = or_blck_size(type);
    return b ? (size_t)(k / b) * or_type_size(type) : 0;
}

int or_vec_dot_type(int type) {
    switch (type) {
        case OR_TYPE_Q8_0: return OR_TYPE_Q8_0;
        case OR_TYPE_Q4_K:
        case OR_TYPE_Q6_K: return OR_TYPE_Q8_K;
        case OR_TYPE_F16: return OR_TYPE_F16;
        default: return -1;
    }
}

/* ------------------------------------------------------------------------- */
/* quantizers                                                                 */
/* ------------------------------------------------------------------------- */

/* quantize_row_q8_0_ref: d = amax/127, id = 1/d, q = roundf(x*id). */
void or_quantize_row_q8_0_ref(const float *x, void *vy, int64_t k) {
    or_quantize_row_q8_0_act(x, vy, k, OR_Q8_0_REF);
}

void or_quantize_row_q8_0_act(const float *x, void *vy, int64_t k, int variant) {
    or_block_q8_0 *y = (or_block_q8_0 *)vy;
    const int64_t nb = k / OR_QK8_0;
    for (int64_t i = 0; i < nb; i++) {
        const float *xb = x + i * OR_QK8_0;
        float amax = 0.0f;
        for (int j = 0; j < OR_QK8_0; j++) {
            const float a = fabsf(xb[j]);
            if (a > amax) amax = a;
        }
        const float d = amax / 127.f;
        float id;
        if (variant == OR_Q8_0_X86) {
            id = (amax != 0.0f) ? 127.f / amax : 0.0f;
        } else {
            id = d != 0.0f ? 1.0f / d : 0.0f;
        }
        y[i].d = or_fp32_to_fp16(d);
        for (int j = 0; j < OR_QK8_0; j++) {
            const float v = xb[j] * id;
            float r = (variant == OR_Q8_0_REF) ? roundf(v) : rintf(v);
            if (r > 127.f) r = 127.f; /* x86 packs saturate; never reached for finite input */
            if (r < -128.f) r = -128.f;
            y[i].qs[j] = (int8_t)r;
        }
    }
}

/* quantize_row_q8_K (ggml-cpu uses the _ref body on x86):
 * max = the first value of largest magnitude; iscale = -127/max;
 * q = min(127, nearest_int(iscale*x)); d = 1/iscale; bsums = sums of 16. */
void or_quantize_row_q8_K(const float *x, void *vy, int64_t k) {
    or_block_q8_K *y = (or_block_q8_K *)vy;
    const int64_t nb = k / OR_QK_K;
    for (int64_t i = 0; i < nb; i++) {
        const float *xb = x + i * OR_QK_K;
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < OR_QK_K; j++) {
            const float ax = fabsf(xb[j]);
            if (ax > amax) {
                amax = ax;
                max = xb[j];
            }
        }
        if (amax == 0.0f) {
            /* ggml writes d = 0 and zero quants and leaves bsums untouched;
             * this restatement defines them as 0 (they are only ever
             * multiplied by d = 0). */
            y[i].d = 0.0f;
            memset(y[i].qs, 0, sizeof(y[i].qs));
            memset(y[i].bsums, 0, sizeof(y[i].bsums));
            continue;
        }
        const float iscale = -127.f / max;
        for (int j = 0; j < OR_QK_K; j++) {
            const int v = or_nearest_int(iscale * xb[j]);
            y[i].qs[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < OR_QK_K / 16; j++) {
            int s = 0;
            for (int l = 0; l < 16; l++) s += y[i].qs[16 * j + l];
            y[i].bsums[j] = (int16_t)s;
        }
        y[i].d = 1.0f / iscale;
    }
}

void or_quantize_row_f16(const float *x, void *vy, int64_t k) {
    uint16_t *y = (uint16_t *)vy;
    for (int64_t i = 0; i < k; i++) y[i] = or_fp32_to_fp16(x[i]);
}

/* A planted mistake (tests only, set through or_set_mutation): the tests that pin the weight
 * quantizers show that each of these makes them fail.  0 = none (the published algorithm). */
static int g_mutation = 0;
void or_set_mutation(int m) { g_mutation = m; }

/* make_qkx2_quants: asymmetric (scale, min) search for one sub-block with
 * weighted least squares refits over nstep+1 candidate inverse scales. */
static float make_qkx2_quants(int n, int nmax, const float *x, const float *weights, uint8_t *L, float *the_min,
                              uint8_t *Laux, float rmin, float rdelta, int nstep, int use_mad) {
    if (g_mutation == OR_MUT_Q4K_NO_SEARCH) nstep = 0;
    if (g_mutation == OR_MUT_Q4K_RDELTA) rdelta = 0.2f;
    float min = x[0], max = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        const float w = weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -min;
        return 0.f;
    }
    float iscale = nmax / (max - min);
    float scale = 1 / iscale;
    float best_error = 0;
    for (int i = 0; i < n; ++i) {
        const int l = or_nearest_int(iscale * (x[i] - min));
        L[i] = (uint8_t)(l < 0 ? 0 : (l > nmax ? nmax : l));
        float diff = scale * L[i] + min - x[i];
        diff = use_mad ? fabsf(diff) : diff * diff;
        best_error += weights[i] * diff;
    }
    if (nstep < 1) {
        *the_min = -min;
        return scale;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = or_nearest_int(iscale * (x[i] - min));
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            Laux[i] = (uint8_t)l;
            const float w = weights[i];
            sum_l += w * l;
            sum_l2 += w * l * l;
            sum_xl += w * l * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float cur_error = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                diff = use_mad ? fabsf(diff) : diff * diff;
                cur_error += weights[i] * diff;
            }
            if (cur_error < best_error) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_error = cur_error;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

float or_make_qkx2_quants(int n, int nmax, const float *x, const float *weights, uint8_t *L, float *the_min,
                          float rmin, float rdelta, int nstep) {
    uint8_t Laux[256];
    if (n > 256) return 0.f;
    return make_qkx2_quants(n, nmax, x, weights, L, the_min, Laux, rmin, rdelta, nstep, 0);
}

void or_quantize_row_q4_K_ref(const float *x, void *vy, int64_t k) {
    or_block_q4_K *y = (or_block_q4_K *)vy;
    const int64_t nb = k / OR_QK_K;
    uint8_t L[OR_QK_K];
    uint8_t Laux[32];
    float weights[32];
    float mins[OR_QK_K / 32];
    float scales[OR_QK_K / 32];
    for (int64_t i = 0; i < nb; i++) {
        float max_scale = 0, max_min = 0;
        for (int j = 0; j < OR_QK_K / 32; ++j) {
            float sum_x2 = 0;
            for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
            const float av_x = sqrtf(sum_x2 / 32);
            for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(x[32 * j + l]);
            if (g_mutation == OR_MUT_Q4K_CALL_UNIT_WEIGHTS)
                for (int l = 0; l < 32; ++l) weights[l] = 1.f;
            scales[j] = make_qkx2_quants(32, 15, x + 32 * j, weights, L + 32 * j, &mins[j], Laux,
                                         g_mutation == OR_MUT_Q4K_CALL_RMIN ? -0.5f : -1.f, 0.1f,
                                         g_mutation == OR_MUT_Q4K_CALL_NSTEP0 ? 0 : 20, 0);
            if (scales[j] > max_scale) max_scale = scales[j];
            if (mins[j] > max_min) max_min = mins[j];
        }
        const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
        const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
        memset(y[i].scales, 0, 12);
        for (int j = 0; j < OR_QK_K / 32; ++j) {
            uint8_t ls = (uint8_t)or_nearest_int(inv_scale * scales[j]);
            uint8_t lm = (uint8_t)or_nearest_int(inv_min * mins[j]);
            if (ls > 63) ls = 63;
            if (lm > 63) lm = 63;
            if (j < 4) {
                y[i].scales[j] = ls;
                y[i].scales[j + 4] = lm;
            } else {
                y[i].scales[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
                if (g_mutation == OR_MUT_Q4K_PACK) {  /* the high bits of scale and min swapped */
                    y[i].scales[j - 4] |= (uint8_t)((lm >> 4) << 6);
                    y[i].scales[j - 0] |= (uint8_t)((ls >> 4) << 6);
                } else {
                    y[i].scales[j - 4] |= (uint8_t)((ls >> 4) << 6);
                    y[i].scales[j - 0] |= (uint8_t)((lm >> 4) << 6);
                }
            }
        }
        y[i].d = or_fp32_to_fp16(max_scale / 63.f);
        y[i].dmin = or_fp32_to_fp16(max_min / 63.f);
        for (int j = 0; j < OR_QK_K / 32; ++j) {
            uint8_t sc, m;
            or_get_scale_min_k4(j, y[i].scales, &sc, &m);
            const float d = or_fp16_to_fp32(y[i].d) * sc;
            if (!d) continue;
            const float dm = or_fp16_to_fp32(y[i].dmin) * m;
            for (int ii = 0; ii < 32; ++ii) {
                int l = or_nearest_int((x[32 * j + ii] + dm) / d);
                l = l < 0 ? 0 : (l > 15 ? 15 : l);
                L[32 * j + ii] = (uint8_t)l;
            }
        }
        uint8_t *q = y[i].qs;
        for (int j = 0; j < OR_QK_K; j += 64) {
            for (int l = 0; l < 32; ++l) q[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
            q += 32;
        }
        x += OR_QK_K;
    }
}

#define GROUP_MAX_EPS 1e-15f

/* make_qx_quants with rmse_type 1 (weights x^2), no importance matrix. */
static float make_qx_quants(int n, int nmax, const float *x, int8_t *L) {
    float max = 0, amax = 0;
    for (int i = 0; i < n; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    if (amax < GROUP_MAX_EPS) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = -nmax / max;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = or_nearest_int(iscale * x[i]);
        l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
        L[i] = (int8_t)(l + nmax);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    float scale = suml2 ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    const float step = g_mutation == OR_MUT_Q6K_STEP ? 0.2f : 0.1f;
    for (int is = -9; is <= 9 && g_mutation != OR_MUT_Q6K_NO_SEARCH; ++is) {
        if (is == 0) continue;
        iscale = -(nmax + step * is) / max;
        sumlx = suml2 = 0;
        for (int i = 0; i < n; ++i) {
            int l = or_nearest_int(iscale * x[i]);
            l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
            const float w = x[i] * x[i];
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                int l = or_nearest_int(iscale * x[i]);
                l = l < -nmax ? -nmax : (l > nmax - 1 ? nmax - 1 : l);
                L[i] = (int8_t)(nmax + l);
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

float or_make_qx_quants(int n, int nmax, const float *x, int8_t *L) { return make_qx_quants(n, nmax, x, L); }

void or_quantize_row_q6_K_ref(const float *x, void *vy, int64_t k) {
    or_block_q6_K *y = (or_block_q6_K *)vy;
    const int64_t nb = k / OR_QK_K;
    int8_t L[OR_QK_K];
    float scales[OR_QK_K / 16];
    for (int64_t i = 0; i < nb; i++) {
        float max_scale = 0, max_abs_scale = 0;
        for (int ib = 0; ib < OR_QK_K / 16; ++ib) {
            const float scale = make_qx_quants(16, 32, x + 16 * ib, L + 16 * ib);
            scales[ib] = scale;
            const float abs_scale = fabsf(scale);
            if (abs_scale > max_abs_scale) {
                max_abs_scale = abs_scale;
                max_scale = scale;
            }
        }
        if (max_abs_scale < GROUP_MAX_EPS) {
            memset(&y[i], 0, sizeof(or_block_q6_K));
            y[i].d = or_fp32_to_fp16(0.f);
            x += OR_QK_K;
            continue;
        }
        const float iscale = (g_mutation == OR_MUT_Q6K_ISCALE ? -127.f : -128.f) / max_scale;
        y[i].d = or_fp32_to_fp16(1 / iscale);
        for (int ib = 0; ib < OR_QK_K / 16; ++ib) {
            const int v = or_nearest_int(iscale * scales[ib]);
            y[i].scales[ib] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < OR_QK_K / 16; ++j) {
            const float d = or_fp16_to_fp32(y[i].d) * y[i].scales[j];
            if (!d) continue;
            for (int ii = 0; ii < 16; ++ii) {
                int l = or_nearest_int(x[16 * j + ii] / d);
                l = l < -32 ? -32 : (l > 31 ? 31 : l);
                L[16 * j + ii] = (int8_t)(l + 32);
            }
        }
        uint8_t *ql = y[i].ql;
        uint8_t *qh = y[i].qh;
        for (int j = 0; j < OR_QK_K; j += 128) {
            for (int l = 0; l < 32; ++l) {
                const uint8_t q1 = L[j + l + 0] & 0xF;
                const uint8_t q2 = L[j + l + 32] & 0xF;
                const uint8_t q3 = L[j + l + 64] & 0xF;
                const uint8_t q4 = L[j + l + 96] & 0xF;
                ql[l + 0] = (uint8_t)(q1 | (q3 << 4));
                ql[l + 32] = (uint8_t)(q2 | (q4 << 4));
                qh[l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4) |
                                  ((L[j + l + 96] >> 4) << 6));
            }
            ql += 64;
            qh += 32;
        }
        x += OR_QK_K;
    }
}

size_t or_quantize_chunk(int type, const float *src, void *dst, int64_t nrows, int64_t k) {
    const size_t rs = or_row_size(type, k);
    for (int64_t r = 0; r < nrows; r++) {
        const float *x = src + r * k;
        void *y = (char *)dst + r * rs;
        switch (type) {
            case OR_TYPE_Q8_0: or_quantize_row_q8_0_ref(x, y, k); break;
            case OR_TYPE_Q4_K: or_quantize_row_q4_K_ref(x, y, k); break;
            case OR_TYPE_Q6_K: or_quantize_row_q6_K_ref(x, y, k); break;
            case OR_TYPE_Q8_K: or_quantize_row_q8_K(x, y, k); break;
            case OR_TYPE_F16: or_quantize_row_f16(x, y, k); break;
            case OR_TYPE_F32: memcpy(y, x, (size_t)k * 4); break;
            default: return 0;
        }
    }
    return rs * (size_t)nrows;
}

/* ------------------------------------------------------------------------- */
/* dequantizers                                                               */
/* ------------------------------------------------------------------------- */
void or_dequantize_row(int type, const void *vx, float *y, int64_t k, int fused) {
    switch (type) {
        case OR_TYPE_F32: memcpy(y, vx, (size_t)k * 4); return;
        case OR_TYPE_F16: {
            const uint16_t *x = (const uint16_t *)vx;
            for (int64_t i = 0; i < k; i++) y[i] = or_fp16_to_fp32(x[i]);
            return;
        }
        case OR_TYPE_Q8_0: {
            const or_block_q8_0 *x = (const or_block_q8_0 *)vx;
            for (int64_t i = 0; i < k / OR_QK8_0; i++) {
                const float d = or_fp16_to_fp32(x[i].d);
                for (int j = 0; j < OR_QK8_0; j++) y[i * OR_QK8_0 + j] = x[i].qs[j] * d;
            }
            return;
        }
        case OR_TYPE_Q4_K: {
            const or_block_q4_K *x = (const or_block_q4_K *)vx;
            for (int64_t i = 0; i < k / OR_QK_K; i++) {
                const uint8_t *q = x[i].qs;
                const float d = or_fp16_to_fp32(x[i].d);
                const float min = or_fp16_to_fp32(x[i].dmin);
                int is = 0;
                for (int j = 0; j < OR_QK_K; j += 64) {
                    uint8_t sc, m;
                    or_get_scale_min_k4(is + 0, x[i].scales, &sc, &m);
                    const float d1 = d * sc, m1 = min * m;
                    or_get_scale_min_k4(is + 1, x[i].scales, &sc, &m);
                    const float d2 = d * sc, m2 = min * m;
                    for (int l = 0; l < 32; ++l)
                        *y++ = fused ? fmaf(d1, (float)(q[l] & 0xF), -m1) : d1 * (q[l] & 0xF) - m1;
                    for (int l = 0; l < 32; ++l)
                        *y++ = fused ? fmaf(d2, (float)(q[l] >> 4), -m2) : d2 * (q[l] >> 4) - m2;
                    q += 32;
                    is += 2;
                }
            }
            return;
        }
        case OR_TYPE_Q6_K: {
            const or_block_q6_K *x = (const or_block_q6_K *)vx;
            for (int64_t i = 0; i < k / OR_QK_K; i++) {
                const float d = or_fp16_to_fp32(x[i].d);
                const uint8_t *ql = x[i].ql;
                const uint8_t *qh = x[i].qh;
                const int8_t *sc = x[i].scales;
                for (int n = 0; n < OR_QK_K; n += 128) {
                    for (int l = 0; l < 32; ++l) {
                        const int is = l / 16;
                        const int8_t q1 = (int8_t)((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                        const int8_t q2 = (int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                        const int8_t q3 = (int8_t)((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                        const int8_t q4 = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                        y[l + 0] = d * sc[is + 0] * q1;
                        y[l + 32] = d * sc[is + 2] * q2;
                        y[l + 64] = d * sc[is + 4] * q3;
                        y[l + 96] = d * sc[is + 6] * q4;
                    }
                    y += 128;
                    ql += 64;
                    qh += 32;
                    sc += 8;
                }
            }
            return;
        }
        case OR_TYPE_Q8_K: {
            const or_block_q8_K *x = (const or_block_q8_K *)vx;
            for (int64_t i = 0; i < k / OR_QK_K; i++)
                for (int j = 0; j < OR_QK_K; j++) y[i * OR_QK_K + j] = x[i].d * x[i].qs[j];
            return;
        }
        default: return;
    }
}

/* ------------------------------------------------------------------------- */
/* activation requantization                                                  */
/* ------------------------------------------------------------------------- */
void or_quantize_act_rows(int wtype, const float *x, int64_t ldx, void *xq, int64_t m, int64_t k,
                          int q8_0_variant) {
    const int vt = or_vec_dot_type(wtype);
    const size_t rs = or_row_size(vt, k);
    for (int64_t r = 0; r < m; r++) {
        const float *xr = x + r * ldx;
        void *yr = (char *)xq + r * rs;
        if (vt == OR_TYPE_Q8_0) or_quantize_row_q8_0_act(xr, yr, k, q8_0_variant);
        else if (vt == OR_TYPE_Q8_K) or_quantize_row_q8_K(xr, yr, k);
        else if (vt == OR_TYPE_F16) or_quantize_row_f16(xr, yr, k);
    }
}

/* ------------------------------------------------------------------------- */
/* block dots, ggml's portable C accumulation order                           */
/* ------------------------------------------------------------------------- */
static float vec_dot_q8_0_q8_0(int64_t n, const or_block_q8_0 *x, const or_block_q8_0 *y) {
    float sumf = 0;
    for (int64_t ib = 0; ib < n / OR_QK8_0; ++ib) {
        int sumi = 0;
        for (int j = 0; j < OR_QK8_0; j++) sumi += x[ib].qs[j] * y[ib].qs[j];
        sumf += sumi * (or_fp16_to_fp32(x[ib].d) * or_fp16_to_fp32(y[ib].d));
    }
    return sumf;
}

static float vec_dot_q4_K_q8_K(int64_t n, const or_block_q4_K *x, const or_block_q8_K *y) {
    float sums[8] = {0};
    float sumf = 0;
    for (int64_t i = 0; i < n / OR_QK_K; ++i) {
        int8_t a[OR_QK_K];
        const uint8_t *q4 = x[i].qs;
        for (int j = 0; j < OR_QK_K / 64; ++j) {
            for (int l = 0; l < 32; ++l) a[64 * j + l] = (int8_t)(q4[l] & 0xF);
            for (int l = 0; l < 32; ++l) a[64 * j + 32 + l] = (int8_t)(q4[l] >> 4);
            q4 += 32;
        }
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; j++) or_get_scale_min_k4(j, x[i].scales, &sc[j], &mn[j]);
        int sumi = 0;
        for (int j = 0; j < OR_QK_K / 16; ++j) sumi += y[i].bsums[j] * mn[j / 2];
        int32_t aux32[8] = {0};
        const int8_t *q8 = y[i].qs;
        const int8_t *ap = a;
        for (int j = 0; j < OR_QK_K / 32; ++j) {
            const int32_t scale = sc[j];
            for (int g = 0; g < 4; g++) {
                for (int l = 0; l < 8; ++l) aux32[l] += scale * (int16_t)(q8[l] * ap[l]);
                q8 += 8;
                ap += 8;
            }
        }
        const float d = or_fp16_to_fp32(x[i].d) * y[i].d;
        for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
        const float dmin = or_fp16_to_fp32(x[i].dmin) * y[i].d;
        sumf -= dmin * sumi;
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

static void unpack_q6_K(const or_block_q6_K *x, int8_t *a) {
    const uint8_t *ql = x->ql;
    const uint8_t *qh = x->qh;
    for (int j = 0; j < OR_QK_K; j += 128) {
        for (int l = 0; l < 32; ++l) {
            a[j + l + 0] = (int8_t)((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
            a[j + l + 32] = (int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            a[j + l + 64] = (int8_t)((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            a[j + l + 96] = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
        }
        ql += 64;
        qh += 32;
    }
}

static float vec_dot_q6_K_q8_K(int64_t n, const or_block_q6_K *x, const or_block_q8_K *y) {
    float sums[8] = {0};
    float sumf = 0;
    for (int64_t i = 0; i < n / OR_QK_K; ++i) {
        int8_t a[OR_QK_K];
        unpack_q6_K(&x[i], a);
        int32_t aux32[8] = {0};
        const int8_t *q8 = y[i].qs;
        const int8_t *ap = a;
        for (int j = 0; j < OR_QK_K / 16; ++j) {
            const int scale = x[i].scales[j];
            for (int g = 0; g < 2; g++) {
                for (int l = 0; l < 8; ++l) aux32[l] += scale * (int16_t)(q8[l] * ap[l]);
                q8 += 8;
                ap += 8;
            }
        }
        const float d = or_fp16_to_fp32(x[i].d) * y[i].d;
        for (int l = 0; l < 8; ++l) sums[l] += d * aux32[l];
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

static float vec_dot_f16(int64_t n, const uint16_t *x, const uint16_t *y) {
    double sumf = 0.0; /* ggml_float */
    for (int64_t i = 0; i < n; ++i) sumf += (double)(or_fp16_to_fp32(x[i]) * or_fp16_to_fp32(y[i]));
    return (float)sumf;
}

float or_vec_dot(int wtype, int64_t k, const void *w, const void *xq) {
    switch (wtype) {
        case OR_TYPE_Q8_0: return vec_dot_q8_0_q8_0(k, (const or_block_q8_0 *)w, (const or_block_q8_0 *)xq);
        case OR_TYPE_Q4_K: return vec_dot_q4_K_q8_K(k, (const or_block_q4_K *)w, (const or_block_q8_K *)xq);
        case OR_TYPE_Q6_K: return vec_dot_q6_K_q8_K(k, (const or_block_q6_K *)w, (const or_block_q8_K *)xq);
        case OR_TYPE_F16: return vec_dot_f16(k, (const uint16_t *)w, (const uint16_t *)xq);
        default: return 0.0f;
    }
}

/* ------------------------------------------------------------------------- */
/* mul_mat                                                                    */
/* ------------------------------------------------------------------------- */
typedef struct {
    int wtype;
    const char *w;
    int64_t n, k, m, ldy;
    const char *xq;
    float *y;
    size_t wrs, xrs;
    int64_t n0, n1;
} mm_job;

static void *mm_worker(void *arg) {
    const mm_job *j = (const mm_job *)arg;
    for (int64_t r = 0; r < j->m; r++) {
        const char *xr = j->xq + r * j->xrs;
        for (int64_t c = j->n0; c < j->n1; c++)
            j->y[r * j->ldy + c] = or_vec_dot(j->wtype, j->k, j->w + c * j->wrs, xr);
    }
    return NULL;
}

void or_mul_mat_q(int wtype, const void *w, int64_t n, int64_t k, const void *xq, int64_t m, float *y, int64_t ldy,
                  int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    if (nthreads > n) nthreads = (int)n;
    if (nthreads < 1) return;
    pthread_t tid[256];
    mm_job jobs[256];
    const size_t wrs = or_row_size(wtype, k);
    const size_t xrs = or_row_size(or_vec_dot_type(wtype), k);
    for (int t = 0; t < nthreads; t++) {
        jobs[t] = (mm_job){wtype, (const char *)w, n, k, m, ldy, (const char *)xq, y, wrs, xrs,
                           n * t / nthreads, n * (t + 1) / nthreads};
        if (nthreads > 1) pthread_create(&tid[t], NULL, mm_worker, &jobs[t]);
        else mm_worker(&jobs[t]);
    }
    if (nthreads > 1)
        for (int t = 0; t < nthreads; t++) pthread_join(tid[t], NULL);
}

void or_mul_mat(int wtype, const void *w, int64_t n, int64_t k, const float *x, int64_t ldx, int64_t m, float *y,
                int64_t ldy, int nthreads, int q8_0_variant) {
    const size_t xrs = or_row_size(or_vec_dot_type(wtype), k);
    void *xq = malloc(xrs * (size_t)(m > 0 ? m : 1));
    or_quantize_act_rows(wtype, x, ldx, xq, m, k, q8_0_variant);
    or_mul_mat_q(wtype, w, n, k, xq, m, y, ldy, nthreads);
    free(xq);
}

/* One output of the exact product: integer block sums, the scale products in fp64. */
static double exact_dot(int wtype, const char *wr, const char *xr, int64_t k) {
    double acc = 0.0;
    if (wtype == OR_TYPE_Q8_0) {
        const or_block_q8_0 *a = (const or_block_q8_0 *)wr;
        const or_block_q8_0 *b = (const or_block_q8_0 *)xr;
        for (int64_t ib = 0; ib < k / OR_QK8_0; ib++) {
            int64_t s = 0;
            for (int j = 0; j < OR_QK8_0; j++) s += (int64_t)a[ib].qs[j] * b[ib].qs[j];
            acc += (double)or_fp16_to_fp32(a[ib].d) * (double)or_fp16_to_fp32(b[ib].d) * (double)s;
        }
    } else if (wtype == OR_TYPE_Q4_K) {
        const or_block_q4_K *a = (const or_block_q4_K *)wr;
        const or_block_q8_K *b = (const or_block_q8_K *)xr;
        for (int64_t ib = 0; ib < k / OR_QK_K; ib++) {
            int64_t smain = 0, smin = 0;
            for (int j = 0; j < 8; j++) {
                uint8_t sc, mn;
                or_get_scale_min_k4(j, a[ib].scales, &sc, &mn);
                int64_t s = 0, bs = 0;
                for (int l = 0; l < 32; l++) {
                    const int e = 32 * j + l;          /* element index in the superblock */
                    const int c64 = e / 64, w64 = e % 64;
                    const uint8_t byte = a[ib].qs[32 * c64 + (w64 % 32)];
                    const int q = (w64 < 32) ? (byte & 0xF) : (byte >> 4);
                    s += (int64_t)q * b[ib].qs[e];
                    bs += b[ib].qs[e];
                }
                smain += (int64_t)sc * s;
                smin += (int64_t)mn * bs;
            }
            const double dx = (double)b[ib].d;
            acc += dx * (double)or_fp16_to_fp32(a[ib].d) * (double)smain -
                   dx * (double)or_fp16_to_fp32(a[ib].dmin) * (double)smin;
        }
    } else if (wtype == OR_TYPE_Q6_K) {
        const or_block_q6_K *a = (const or_block_q6_K *)wr;
        const or_block_q8_K *b = (const or_block_q8_K *)xr;
        for (int64_t ib = 0; ib < k / OR_QK_K; ib++) {
            int8_t q6[OR_QK_K];
            unpack_q6_K(&a[ib], q6);
            int64_t s = 0;
            for (int e = 0; e < OR_QK_K; e++) s += (int64_t)a[ib].scales[e / 16] * q6[e] * b[ib].qs[e];
            acc += (double)b[ib].d * (double)or_fp16_to_fp32(a[ib].d) * (double)s;
        }
    } else if (wtype == OR_TYPE_F16) {
        const uint16_t *a = (const uint16_t *)wr;
        const uint16_t *b = (const uint16_t *)xr;
        for (int64_t e = 0; e < k; e++) acc += (double)or_fp16_to_fp32(a[e]) * (double)or_fp16_to_fp32(b[e]);
    }
    return acc;
}

typedef struct {
    int wtype;
    const char *w, *xq;
    int64_t n, k, m;
    size_t wrs, xrs;
    double *y;
    int64_t n0, n1;
} exact_job;

static void *exact_worker(void *arg) {
    const exact_job *j = (const exact_job *)arg;
    for (int64_t r = 0; r < j->m; r++)
        for (int64_t c = j->n0; c < j->n1; c++)
            j->y[r * j->n + c] = exact_dot(j->wtype, j->w + c * j->wrs, j->xq + r * j->xrs, j->k);
    return NULL;
}

/* Threads split the output columns only: every output is computed the same way whatever the
 * thread count, so the result does not depend on it. */
void or_mul_mat_exact(int wtype, const void *w, int64_t n, int64_t k, const void *xq, int64_t m, double *y) {
    long nt = sysconf(_SC_NPROCESSORS_ONLN);
    if (nt < 1) nt = 1;
    if (nt > 16) nt = 16;
    if ((int64_t)nt > n) nt = (long)(n > 0 ? n : 1);
    if (m * n * k < ((int64_t)1 << 22)) nt = 1;
    pthread_t tid[16];
    exact_job jobs[16];
    const size_t wrs = or_row_size(wtype, k), xrs = or_row_size(or_vec_dot_type(wtype), k);
    for (long t = 0; t < nt; t++) {
        jobs[t] = (exact_job){wtype, (const char *)w, (const char *)xq, n, k, m, wrs, xrs, y, n * t / nt,
                              n * (t + 1) / nt};
        if (nt > 1) pthread_create(&tid[t], NULL, exact_worker, &jobs[t]);
        else exact_worker(&jobs[t]);
    }
    if (nt > 1)
        for (long t = 0; t < nt; t++) pthread_join(tid[t], NULL);
}
