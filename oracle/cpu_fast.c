/*
 * cpu_fast.c -- the CPU baseline: ggml-cpu's mul_mat algorithm restated with x86 SIMD and
 * threads, the way ggml's x86 backend runs it (activation rows requantized to the weight's
 * vec_dot_type, integer block dots, fp32 scale accumulation, output tiles spread over
 * threads).
 *
 * TEST INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg times it and tests/ check it against
 * the scalar oracle.  Nothing in the shipped path links it.
 *
 * Restated algorithms (ggml-cpu, not vendored in the reference; call sites
 * src/crispembed.cpp:1168-1170,1300,1410,1416):
 *   Q8_0 x Q8_0 : per 32-block, sum(qw * qx) in int32, times fp16(dw) * fp16(dx), fp32 fma
 *                 across blocks (ggml_vec_dot_q8_0_q8_0).  The SIMD form multiplies |qw| by
 *                 qx * sign(qw) (u8 x s8 byte products, pairwise int16 sums, int32 sums).
 *   Q4_K x Q8_K : per superblock, sumi = sum_j sc_j * sum(q4 * q8) and summ = sum_j m_j *
 *                 (bsum_2j + bsum_2j+1); acc += dx * d * sumi - dx * dmin * summ
 *                 (ggml_vec_dot_q4_K_q8_K).
 *   Q6_K x Q8_K : per superblock, isum = sum_i sc_i * sum((q6 - 32) * q8), computed as
 *                 sum(q6 * q8) - 32 * bsum_i; acc += d * dx * isum (ggml_vec_dot_q6_K_q8_K).
 * The activation quantizers are the oracle's (bit-exact ggml semantics).
 *
 * Two SIMD forms, chosen at run time from the host's CPUID (the library is built here and
 * runs on another host, so it is never compiled for the build host's own ISA):
 *   AVX-512 VNNI (+BW/VL): 64-byte vectors, two 32-value blocks (Q8_0) or two sub-blocks
 *     (K-quants) per instruction; the int8 dots by vpdpbusd (Q8_0) and the scale-weighted
 *     pair sums of the K-quants by vpmaddubsw + vpdpwssd;
 *   AVX2 + FMA + F16C: every x86-64 host of this decade.
 * Both produce the same integer sums; the fp32 accumulation order differs (as ggml's own
 * AVX2 and AVX-512 builds differ), within the mul_mat bar of the exact product.
 */
#include <immintrin.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "ggml_oracle.h"

#define FAST_TARGET __attribute__((target("avx2,fma,f16c")))

FAST_TARGET static inline float hsum8(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_movehdup_ps(s));
    return _mm_cvtss_f32(s);
}

/* pairwise u8 x s8 products summed to int32 lanes (8 lanes of 4 products each) */
FAST_TARGET static inline __m256i dot_u8s8(__m256i u, __m256i s) {
    return _mm256_madd_epi16(_mm256_maddubs_epi16(u, s), _mm256_set1_epi16(1));
}

FAST_TARGET static float dot_q8_0(int64_t nb, const or_block_q8_0 *w, const or_block_q8_0 *x) {
    __m256 acc = _mm256_setzero_ps();
    for (int64_t b = 0; b < nb; b++) {
        const __m256i qw = _mm256_loadu_si256((const __m256i *)w[b].qs);
        const __m256i qx = _mm256_loadu_si256((const __m256i *)x[b].qs);
        const __m256i s = dot_u8s8(_mm256_sign_epi8(qw, qw), _mm256_sign_epi8(qx, qw));
        const float d = _cvtsh_ss(w[b].d) * _cvtsh_ss(x[b].d);
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(s), acc);
    }
    return hsum8(acc);
}

FAST_TARGET static float dot_q4_K(int64_t nb, const or_block_q4_K *w, const or_block_q8_K *x) {
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    __m256 acc = _mm256_setzero_ps();
    float accm = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; j++) or_get_scale_min_k4(j, w[b].scales, &sc[j], &mn[j]);
        int summ = 0;
        for (int j = 0; j < 8; j++) summ += mn[j] * (x[b].bsums[2 * j] + x[b].bsums[2 * j + 1]);
        __m256i sumi = _mm256_setzero_si256();
        for (int c = 0; c < 4; c++) {
            const __m256i q4 = _mm256_loadu_si256((const __m256i *)(w[b].qs + 32 * c));
            const __m256i lo = _mm256_and_si256(q4, m4);
            const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q4, 4), m4);
            const __m256i xa = _mm256_loadu_si256((const __m256i *)(x[b].qs + 64 * c));
            const __m256i xb = _mm256_loadu_si256((const __m256i *)(x[b].qs + 64 * c + 32));
            const __m256i pa = _mm256_madd_epi16(_mm256_maddubs_epi16(lo, xa), _mm256_set1_epi16(sc[2 * c]));
            const __m256i pb = _mm256_madd_epi16(_mm256_maddubs_epi16(hi, xb), _mm256_set1_epi16(sc[2 * c + 1]));
            sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(pa, pb));
        }
        const float d = x[b].d * _cvtsh_ss(w[b].d);
        const float dmin = x[b].d * _cvtsh_ss(w[b].dmin);
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
        accm += dmin * (float)summ;
    }
    return hsum8(acc) - accm;
}

FAST_TARGET static float dot_q6_K(int64_t nb, const or_block_q6_K *w, const or_block_q8_K *x) {
    const __m256i m4 = _mm256_set1_epi8(0x0F), m2 = _mm256_set1_epi8(0x03);
    float acc = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *ql = w[b].ql, *qh = w[b].qh;
        const int8_t *sc = w[b].scales;
        int corr = 0;
        for (int i = 0; i < 16; i++) corr += sc[i] * x[b].bsums[i];
        __m256i sumi = _mm256_setzero_si256();
        for (int h = 0; h < 2; h++) {
            const __m256i l0 = _mm256_loadu_si256((const __m256i *)(ql + 64 * h));
            const __m256i l1 = _mm256_loadu_si256((const __m256i *)(ql + 64 * h + 32));
            const __m256i hb = _mm256_loadu_si256((const __m256i *)(qh + 32 * h));
            __m256i q[4];
            q[0] = _mm256_or_si256(_mm256_and_si256(l0, m4), _mm256_slli_epi16(_mm256_and_si256(hb, m2), 4));
            q[1] = _mm256_or_si256(_mm256_and_si256(l1, m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hb, 2), m2), 4));
            q[2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l0, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hb, 4), m2), 4));
            q[3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l1, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hb, 6), m2), 4));
            for (int j = 0; j < 4; j++) {
                const int e0 = 128 * h + 32 * j;  /* first of the 32 values: sub-blocks e0/16, e0/16 + 1 */
                const __m256i xv = _mm256_loadu_si256((const __m256i *)(x[b].qs + e0));
                const __m256i s16 = _mm256_setr_m128i(_mm_set1_epi16(sc[e0 / 16]), _mm_set1_epi16(sc[e0 / 16 + 1]));
                sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(_mm256_maddubs_epi16(q[j], xv), s16));
            }
        }
        const float d = _cvtsh_ss(w[b].d) * x[b].d;
        /* hsum of the int32 lanes, then the -32 offset through the block sums */
        __m128i s4 = _mm_add_epi32(_mm256_castsi256_si128(sumi), _mm256_extracti128_si256(sumi, 1));
        s4 = _mm_add_epi32(s4, _mm_unpackhi_epi64(s4, s4));
        s4 = _mm_add_epi32(s4, _mm_shuffle_epi32(s4, 1));
        const int isum = _mm_cvtsi128_si32(s4) - 32 * corr;
        acc += d * (float)isum;
    }
    return acc;
}

/* ---- AVX-512 VNNI forms ---- */
#define VNNI_TARGET __attribute__((target("avx512f,avx512bw,avx512vl,avx512vnni,avx2,fma,f16c")))

VNNI_TARGET static inline __m512i cat256(__m256i lo, __m256i hi) {
    return _mm512_inserti64x4(_mm512_castsi256_si512(lo), hi, 1);
}

VNNI_TARGET static float dot_q8_0_vnni(int64_t nb, const or_block_q8_0 *w, const or_block_q8_0 *x) {
    __m512 acc = _mm512_setzero_ps();
    int64_t b = 0;
    for (; b + 1 < nb; b += 2) {  /* two blocks: int32 lanes 0-7 block b, 8-15 block b + 1 */
        const __m512i qw = cat256(_mm256_loadu_si256((const __m256i *)w[b].qs),
                                  _mm256_loadu_si256((const __m256i *)w[b + 1].qs));
        const __m512i qx = cat256(_mm256_loadu_si256((const __m256i *)x[b].qs),
                                  _mm256_loadu_si256((const __m256i *)x[b + 1].qs));
        /* |qw| (unsigned) times qx with qw's sign */
        const __mmask64 neg = _mm512_movepi8_mask(qw);
        const __m512i sx = _mm512_mask_sub_epi8(qx, neg, _mm512_setzero_si512(), qx);
        const __m512i s = _mm512_dpbusd_epi32(_mm512_setzero_si512(), _mm512_abs_epi8(qw), sx);
        const __m256 d0 = _mm256_set1_ps(_cvtsh_ss(w[b].d) * _cvtsh_ss(x[b].d));
        const __m256 d1 = _mm256_set1_ps(_cvtsh_ss(w[b + 1].d) * _cvtsh_ss(x[b + 1].d));
        const __m512 d = _mm512_castpd_ps(
            _mm512_insertf64x4(_mm512_castpd256_pd512(_mm256_castps_pd(d0)), _mm256_castps_pd(d1), 1));
        acc = _mm512_fmadd_ps(d, _mm512_cvtepi32_ps(s), acc);
    }
    float r = _mm512_reduce_add_ps(acc);
    if (b < nb) r += dot_q8_0(nb - b, w + b, x + b);
    return r;
}

VNNI_TARGET static float dot_q4_K_vnni(int64_t nb, const or_block_q4_K *w, const or_block_q8_K *x) {
    const __m512i m4 = _mm512_set1_epi8(0x0F);
    __m512 acc = _mm512_setzero_ps();
    float accm = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; j++) or_get_scale_min_k4(j, w[b].scales, &sc[j], &mn[j]);
        int summ = 0;
        for (int j = 0; j < 8; j++) summ += mn[j] * (x[b].bsums[2 * j] + x[b].bsums[2 * j + 1]);
        __m512i sumi = _mm512_setzero_si512();
        for (int h = 0; h < 2; h++) {
            /* qs bytes 64h..64h+63: 64-value chunks 2h and 2h+1; low nibbles are sub-blocks 4h and 4h+2,
             * high nibbles 4h+1 and 4h+3 */
            const __m512i q4 = _mm512_loadu_si512((const void *)(w[b].qs + 64 * h));
            const __m512i lo = _mm512_and_si512(q4, m4);
            const __m512i hi = _mm512_and_si512(_mm512_srli_epi16(q4, 4), m4);
            const int8_t *xs = x[b].qs + 128 * h;
            const __m512i xlo = cat256(_mm256_loadu_si256((const __m256i *)xs), _mm256_loadu_si256((const __m256i *)(xs + 64)));
            const __m512i xhi =
                cat256(_mm256_loadu_si256((const __m256i *)(xs + 32)), _mm256_loadu_si256((const __m256i *)(xs + 96)));
            const __m512i slo = cat256(_mm256_set1_epi16(sc[4 * h]), _mm256_set1_epi16(sc[4 * h + 2]));
            const __m512i shi = cat256(_mm256_set1_epi16(sc[4 * h + 1]), _mm256_set1_epi16(sc[4 * h + 3]));
            sumi = _mm512_dpwssd_epi32(sumi, _mm512_maddubs_epi16(lo, xlo), slo);
            sumi = _mm512_dpwssd_epi32(sumi, _mm512_maddubs_epi16(hi, xhi), shi);
        }
        const float d = x[b].d * _cvtsh_ss(w[b].d);
        const float dmin = x[b].d * _cvtsh_ss(w[b].dmin);
        acc = _mm512_fmadd_ps(_mm512_set1_ps(d), _mm512_cvtepi32_ps(sumi), acc);
        accm += dmin * (float)summ;
    }
    return _mm512_reduce_add_ps(acc) - accm;
}

VNNI_TARGET static float dot_q6_K_vnni(int64_t nb, const or_block_q6_K *w, const or_block_q8_K *x) {
    const __m512i m4 = _mm512_set1_epi8(0x0F), m2 = _mm512_set1_epi8(0x03);
    /* qh shifts: the lower 32 bytes of a pair take bits (0, 4), the upper (2, 6) */
    const __m512i sh01 = cat256(_mm256_set1_epi16(0), _mm256_set1_epi16(2));
    const __m512i sh23 = cat256(_mm256_set1_epi16(4), _mm256_set1_epi16(6));
    /* int16 lane i of a 64-value pair belongs to 16-value sub-block i / 8 of the pair */
    int16_t ix[32];
    for (int i = 0; i < 32; i++) ix[i] = (int16_t)(i / 8);
    const __m512i idx = _mm512_loadu_si512((const void *)ix);
    float acc = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *ql = w[b].ql, *qh = w[b].qh;
        const int8_t *sc = w[b].scales;
        int corr = 0;
        for (int i = 0; i < 16; i++) corr += sc[i] * x[b].bsums[i];
        const __m512i sc16 = _mm512_cvtepi8_epi16(_mm256_castsi128_si256(_mm_loadu_si128((const __m128i *)sc)));
        __m512i sumi = _mm512_setzero_si512();
        for (int h = 0; h < 2; h++) {
            const __m512i l = _mm512_loadu_si512((const void *)(ql + 64 * h));  /* ql halves l0 | l1 */
            const __m512i hb = _mm512_broadcast_i64x4(_mm256_loadu_si256((const __m256i *)(qh + 32 * h)));
            /* values 128h + 0..63 and 128h + 64..127 */
            const __m512i q01 = _mm512_or_si512(_mm512_and_si512(l, m4),
                                                _mm512_slli_epi16(_mm512_and_si512(_mm512_srlv_epi16(hb, sh01), m2), 4));
            const __m512i q23 = _mm512_or_si512(_mm512_and_si512(_mm512_srli_epi16(l, 4), m4),
                                                _mm512_slli_epi16(_mm512_and_si512(_mm512_srlv_epi16(hb, sh23), m2), 4));
            const __m512i x01 = _mm512_loadu_si512((const void *)(x[b].qs + 128 * h));
            const __m512i x23 = _mm512_loadu_si512((const void *)(x[b].qs + 128 * h + 64));
            const __m512i s01 = _mm512_permutexvar_epi16(_mm512_add_epi16(idx, _mm512_set1_epi16((short)(8 * h))), sc16);
            const __m512i s23 =
                _mm512_permutexvar_epi16(_mm512_add_epi16(idx, _mm512_set1_epi16((short)(8 * h + 4))), sc16);
            sumi = _mm512_dpwssd_epi32(sumi, _mm512_maddubs_epi16(q01, x01), s01);
            sumi = _mm512_dpwssd_epi32(sumi, _mm512_maddubs_epi16(q23, x23), s23);
        }
        const float d = _cvtsh_ss(w[b].d) * x[b].d;
        acc += d * (float)(_mm512_reduce_add_epi32(sumi) - 32 * corr);
    }
    return acc;
}

static int host_vnni(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("avx512vnni");
}

/* The SIMD form or_fast_mul_mat uses on this host ("avx512vnni", "avx2" or "none"); OR_FAST_ISA=avx2
 * forces the AVX2 form (for comparing the two). */
const char *or_fast_isa(void) {
    __builtin_cpu_init();
    if (!(__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") && __builtin_cpu_supports("f16c")))
        return "none";
    const char *f = getenv("OR_FAST_ISA");
    if (f && strcmp(f, "avx2") == 0) return "avx2";
    return host_vnni() ? "avx512vnni" : "avx2";
}

typedef struct {
    int wtype;
    const uint8_t *w, *xq;
    const float *x;
    int64_t n, k, m, ldx, ldy;
    size_t wrow, xrow;
    uint8_t *xq_out;
    float *y;
    int64_t ntn, ntiles;
    int64_t next;  /* work counter (atomic) */
    int vnni;
} fast_job;

enum { TILE_M = 16, TILE_N = 16 };

static void *quant_worker(void *arg) {
    fast_job *j = (fast_job *)arg;
    for (;;) {
        const int64_t r0 = __atomic_fetch_add(&j->next, 64, __ATOMIC_RELAXED);
        if (r0 >= j->m) break;
        const int64_t r1 = r0 + 64 < j->m ? r0 + 64 : j->m;
        or_quantize_act_rows(j->wtype, j->x + r0 * j->ldx, j->ldx, j->xq_out + r0 * j->xrow, r1 - r0, j->k,
                             OR_Q8_0_X86);
    }
    return NULL;
}

FAST_TARGET static void *dot_worker(void *arg) {
    fast_job *j = (fast_job *)arg;
    for (;;) {
        const int64_t t = __atomic_fetch_add(&j->next, 1, __ATOMIC_RELAXED);
        if (t >= j->ntiles) break;
        const int64_t m0 = (t / j->ntn) * TILE_M, n0 = (t % j->ntn) * TILE_N;
        const int64_t m1 = m0 + TILE_M < j->m ? m0 + TILE_M : j->m, n1 = n0 + TILE_N < j->n ? n0 + TILE_N : j->n;
        for (int64_t mi = m0; mi < m1; mi++) {
            const void *xr = j->xq + mi * j->xrow;
            for (int64_t ni = n0; ni < n1; ni++) {
                const void *wr = j->w + ni * j->wrow;
                float v;
                if (j->vnni) {
                    switch (j->wtype) {
                        case OR_TYPE_Q8_0: v = dot_q8_0_vnni(j->k / OR_QK8_0, wr, xr); break;
                        case OR_TYPE_Q4_K: v = dot_q4_K_vnni(j->k / OR_QK_K, wr, xr); break;
                        default: v = dot_q6_K_vnni(j->k / OR_QK_K, wr, xr); break;
                    }
                } else {
                    switch (j->wtype) {
                        case OR_TYPE_Q8_0: v = dot_q8_0(j->k / OR_QK8_0, wr, xr); break;
                        case OR_TYPE_Q4_K: v = dot_q4_K(j->k / OR_QK_K, wr, xr); break;
                        default: v = dot_q6_K(j->k / OR_QK_K, wr, xr); break;
                    }
                }
                j->y[mi * j->ldy + ni] = v;
            }
        }
    }
    return NULL;
}

/* A persistent worker pool, as ggml-cpu keeps one (its threadpool spins between ops instead of
 * creating threads per op): workers wait for a new job generation, spinning for a while and then
 * sleeping on a condition variable; the caller runs the job too and waits for the workers it
 * used.  Creating and joining threads per call cost ~20 us a thread, which at decode sizes (one
 * activation row, a 1-5 MB weight) was most of the call. */
static struct {
    pthread_mutex_t mu;
    pthread_cond_t wake, done;
    pthread_t th[256];
    int size;                  /* workers created */
    unsigned gen;              /* job generation (atomic) */
    int active;                /* workers taking part in the current job */
    int pending;               /* of those, still running */
    void *(*fn)(void *);
    fast_job *job;
} pool = {.mu = PTHREAD_MUTEX_INITIALIZER, .wake = PTHREAD_COND_INITIALIZER, .done = PTHREAD_COND_INITIALIZER};

static void *pool_worker(void *arg) {
    const int idx = (int)(intptr_t)arg;
    unsigned seen = 0;
    for (;;) {
        unsigned g = __atomic_load_n(&pool.gen, __ATOMIC_ACQUIRE);
        for (int spin = 0; g == seen && spin < 200000; spin++) {
            __builtin_ia32_pause();
            g = __atomic_load_n(&pool.gen, __ATOMIC_ACQUIRE);
        }
        if (g == seen) {
            pthread_mutex_lock(&pool.mu);
            while ((g = __atomic_load_n(&pool.gen, __ATOMIC_ACQUIRE)) == seen) pthread_cond_wait(&pool.wake, &pool.mu);
            pthread_mutex_unlock(&pool.mu);
        }
        seen = g;
        if (idx >= pool.active) continue;
        pool.fn(pool.job);
        if (__atomic_sub_fetch(&pool.pending, 1, __ATOMIC_ACQ_REL) == 0) {
            pthread_mutex_lock(&pool.mu);
            pthread_cond_signal(&pool.done);
            pthread_mutex_unlock(&pool.mu);
        }
    }
    return NULL;
}

static void run_threads(void *(*fn)(void *), fast_job *j, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 257) nthreads = 257;
    j->next = 0;
    const int workers = nthreads - 1;
    if (workers == 0) {
        fn(j);
        return;
    }
    pthread_mutex_lock(&pool.mu);
    while (pool.size < workers) {
        if (pthread_create(&pool.th[pool.size], NULL, pool_worker, (void *)(intptr_t)pool.size) != 0) break;
        pthread_detach(pool.th[pool.size]);
        pool.size++;
    }
    pool.fn = fn, pool.job = j;
    pool.active = workers < pool.size ? workers : pool.size;
    __atomic_store_n(&pool.pending, pool.active, __ATOMIC_RELEASE);
    __atomic_add_fetch(&pool.gen, 1, __ATOMIC_RELEASE);
    pthread_cond_broadcast(&pool.wake);
    pthread_mutex_unlock(&pool.mu);
    fn(j);
    for (int spin = 0; __atomic_load_n(&pool.pending, __ATOMIC_ACQUIRE) != 0 && spin < 2000000; spin++)
        __builtin_ia32_pause();
    pthread_mutex_lock(&pool.mu);
    while (__atomic_load_n(&pool.pending, __ATOMIC_ACQUIRE) != 0) pthread_cond_wait(&pool.done, &pool.mu);
    pthread_mutex_unlock(&pool.mu);
}

int or_fast_supported(int wtype) {
    if (wtype != OR_TYPE_Q8_0 && wtype != OR_TYPE_Q4_K && wtype != OR_TYPE_Q6_K) return 0;
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") && __builtin_cpu_supports("f16c");
}

/* y[m*ldy + n] = sum_k W[n,k] X[m,k]; returns 0, or -1 for an unsupported type / host ISA. */
int or_fast_mul_mat(int wtype, const void *w, int64_t n, int64_t k, const float *x, int64_t ldx, int64_t m, float *y,
                    int64_t ldy, int nthreads) {
    if (!or_fast_supported(wtype)) return -1;
    const int vt = or_vec_dot_type(wtype);
    fast_job j;
    memset(&j, 0, sizeof j);
    j.wtype = wtype;
    j.vnni = strcmp(or_fast_isa(), "avx512vnni") == 0;
    j.w = (const uint8_t *)w;
    j.x = x;
    j.n = n;
    j.k = k;
    j.m = m;
    j.ldx = ldx;
    j.ldy = ldy;
    j.y = y;
    j.wrow = or_row_size(wtype, k);
    j.xrow = or_row_size(vt, k);
    j.xq_out = (uint8_t *)malloc((size_t)m * j.xrow + 64);
    if (!j.xq_out) return -1;
    run_threads(quant_worker, &j, nthreads);
    j.xq = j.xq_out;
    j.ntn = (n + TILE_N - 1) / TILE_N;
    j.ntiles = ((m + TILE_M - 1) / TILE_M) * j.ntn;
    run_threads(dot_worker, &j, nthreads);
    free(j.xq_out);
    return 0;
}
