/*
 * m27q_cpu_simd.c -- AVX2 build of the CPU baseline (ggml's q8_K / q8_0
 * activation path: q4_K x q8_K, q6_K x q8_K, q8_0 x q8_0 dots).
 *
 * TEST INFRASTRUCTURE ONLY: bench.py's cpu_baseline leg times it beside the
 * scalar restatement in m27q_oracle.c; tests/test_oracle.py pins it against
 * the same fp64 brute force.  Written from the mathematics of the formats:
 *   q4_K: per 32-group j of a block, sc_j sum(q4 q8) (exact in int32), then
 *         d d8 sum_j(...) - dmin d8 sum_j m_j (bsum_2j + bsum_2j+1);
 *   q6_K: per 16-group j, sc_j sum(q6 q8) with the unsigned 6-bit codes, less
 *         32 sc_j bsum_j for the code offset, then d d8 (...);
 *   q8_0: d_x d_y sum(q_x q_y) per 32-block.
 * Unsigned x signed byte products go through vpmaddubsw (pairs summed in
 * int16: at most 2 x 63 x 127, exact), then vpmaddwd against the group scales
 * into int32.  Only the fp32 combine differs from the scalar form (a vector
 * of 8 partial sums per row, added at the end).
 */
#include <immintrin.h>
#include <pthread.h>
#include <stdint.h>
#include <string.h>

#include "m27q_oracle.h"

static inline int hsum_i32(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4e));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xb1));
    return _mm_cvtsi128_si32(s);
}

static inline float hsum_f32(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_movehdup_ps(s));
    return _mm_cvtss_f32(s);
}

float ora_simd_vec_dot_q4_K_q8_K(int n, const void *vx, const void *vy) {
    const ora_block_q4_K *x = (const ora_block_q4_K *)vx;
    const ora_block_q8_K *y = (const ora_block_q8_K *)vy;
    const __m256i m4 = _mm256_set1_epi8(0x0f);
    __m256 acc = _mm256_setzero_ps();
    float accm = 0.f;
    for (int i = 0; i < n / 256; ++i) {
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; ++j) ora_get_scale_min_k4(j, x[i].scales, &sc[j], &mn[j]);
        /* min term: sum_j m_j (bsum_2j + bsum_2j+1) */
        const __m128i b = _mm_loadu_si128((const __m128i *)y[i].bsums);
        const __m128i b2 = _mm_loadu_si128((const __m128i *)(y[i].bsums + 8));
        const __m128i pair = _mm_hadd_epi16(b, b2); /* bsum_2j + bsum_2j+1, j = 0..7 (|.| <= 8128) */
        const __m128i mv = _mm_cvtepu8_epi16(_mm_loadl_epi64((const __m128i *)mn));
        const __m128i mm = _mm_madd_epi16(pair, mv);
        __m128i ms = _mm_add_epi32(mm, _mm_shuffle_epi32(mm, 0x4e));
        ms = _mm_add_epi32(ms, _mm_shuffle_epi32(ms, 0xb1));
        const int summ = _mm_cvtsi128_si32(ms);
        __m256i sumi = _mm256_setzero_si256();
        for (int g = 0; g < 4; ++g) {
            const __m256i q = _mm256_loadu_si256((const __m256i *)(x[i].qs + 32 * g));
            const __m256i lo = _mm256_and_si256(q, m4);
            const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q, 4), m4);
            const __m256i ylo = _mm256_loadu_si256((const __m256i *)(y[i].qs + 64 * g));
            const __m256i yhi = _mm256_loadu_si256((const __m256i *)(y[i].qs + 64 * g + 32));
            const __m256i plo = _mm256_madd_epi16(_mm256_maddubs_epi16(lo, ylo), _mm256_set1_epi16(sc[2 * g]));
            const __m256i phi = _mm256_madd_epi16(_mm256_maddubs_epi16(hi, yhi), _mm256_set1_epi16(sc[2 * g + 1]));
            sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(plo, phi));
        }
        const float d = ora_fp16_to_fp32(x[i].d) * y[i].d;
        const float dmin = ora_fp16_to_fp32(x[i].dmin) * y[i].d;
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
        accm += dmin * (float)summ;
    }
    return hsum_f32(acc) - accm;
}

float ora_simd_vec_dot_q6_K_q8_K(int n, const void *vx, const void *vy) {
    const ora_block_q6_K *x = (const ora_block_q6_K *)vx;
    const ora_block_q8_K *y = (const ora_block_q8_K *)vy;
    const __m256i m4 = _mm256_set1_epi8(0x0f), m3 = _mm256_set1_epi8(0x03);
    __m256 acc = _mm256_setzero_ps();
    for (int i = 0; i < n / 256; ++i) {
        /* code offset: 32 sum_j sc_j bsum_j over the 16 sub-blocks */
        const __m256i sc16 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)x[i].scales));
        const __m256i bs = _mm256_loadu_si256((const __m256i *)y[i].bsums);
        const int off = 32 * hsum_i32(_mm256_madd_epi16(sc16, bs));
        __m256i sumi = _mm256_setzero_si256();
        for (int h = 0; h < 2; ++h) {
            const __m256i l0 = _mm256_loadu_si256((const __m256i *)(x[i].ql + 64 * h));
            const __m256i l1 = _mm256_loadu_si256((const __m256i *)(x[i].ql + 64 * h + 32));
            const __m256i qh = _mm256_loadu_si256((const __m256i *)(x[i].qh + 32 * h));
            __m256i q[4];
            q[0] = _mm256_or_si256(_mm256_and_si256(l0, m4), _mm256_slli_epi16(_mm256_and_si256(qh, m3), 4));
            q[1] = _mm256_or_si256(_mm256_and_si256(l1, m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 2), m3), 4));
            q[2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l0, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 4), m3), 4));
            q[3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l1, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 6), m3), 4));
            for (int k = 0; k < 4; ++k) {
                /* values 128 h + 32 k + [0, 32): sub-blocks 8 h + 2 k (low 16) and 8 h + 2 k + 1 */
                const int j = 8 * h + 2 * k;
                const __m256i yv = _mm256_loadu_si256((const __m256i *)(y[i].qs + 128 * h + 32 * k));
                const __m256i s = _mm256_setr_m128i(_mm_set1_epi16((int16_t)x[i].scales[j]),
                                                    _mm_set1_epi16((int16_t)x[i].scales[j + 1]));
                sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(_mm256_maddubs_epi16(q[k], yv), s));
            }
        }
        const float d = ora_fp16_to_fp32(x[i].d) * y[i].d;
        const __m256i tot = _mm256_sub_epi32(sumi, _mm256_setr_epi32(off, 0, 0, 0, 0, 0, 0, 0));
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(tot), acc);
    }
    return hsum_f32(acc);
}

float ora_simd_vec_dot_q8_0_q8_0(int n, const void *vx, const void *vy) {
    const ora_block_q8_0 *x = (const ora_block_q8_0 *)vx, *y = (const ora_block_q8_0 *)vy;
    const __m256i ones = _mm256_set1_epi16(1);
    __m256 acc = _mm256_setzero_ps();
    for (int i = 0; i < n / 32; ++i) {
        const __m256i a = _mm256_loadu_si256((const __m256i *)x[i].qs);
        const __m256i b = _mm256_loadu_si256((const __m256i *)y[i].qs);
        /* signed x signed as |a| x (b with a's sign): exact in int16 pairs */
        const __m256i p = _mm256_maddubs_epi16(_mm256_sign_epi8(a, a), _mm256_sign_epi8(b, a));
        const __m256i s = _mm256_madd_epi16(p, ones);
        const float d = ora_fp16_to_fp32(x[i].d) * ora_fp16_to_fp32(y[i].d);
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(s), acc);
    }
    return hsum_f32(acc);
}

typedef struct {
    int type, rb, r0, r1;
    const uint8_t *w;
    const void *xq;
    float *y;
} simd_job;

static void *simd_worker(void *p) {
    const simd_job *j = (const simd_job *)p;
    const size_t rs = (size_t)j->rb * ora_type_size(j->type);
    const int n = j->rb * ora_block_elems(j->type);
    for (int r = j->r0; r < j->r1; ++r) {
        const uint8_t *row = j->w + (size_t)r * rs;
        if (j->type == ORA_Q4_K) j->y[r] = ora_simd_vec_dot_q4_K_q8_K(n, row, j->xq);
        else if (j->type == ORA_Q6_K) j->y[r] = ora_simd_vec_dot_q6_K_q8_K(n, row, j->xq);
        else j->y[r] = ora_simd_vec_dot_q8_0_q8_0(n, row, j->xq);
    }
    return NULL;
}

int ora_gemv_cpu_simd(int type, const void *w, int rb, int rc, const void *xq, float *y, int nthreads) {
    if (type != ORA_Q4_K && type != ORA_Q6_K && type != ORA_Q8_0) return -1;
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    pthread_t th[256];
    simd_job jobs[256];
    for (int t = 0; t < nthreads; ++t) {
        jobs[t].type = type; jobs[t].rb = rb; jobs[t].w = (const uint8_t *)w; jobs[t].xq = xq; jobs[t].y = y;
        jobs[t].r0 = (int)((int64_t)rc * t / nthreads);
        jobs[t].r1 = (int)((int64_t)rc * (t + 1) / nthreads);
    }
    if (nthreads == 1) { simd_worker(&jobs[0]); return 0; }
    for (int t = 0; t < nthreads; ++t) pthread_create(&th[t], NULL, simd_worker, &jobs[t]);
    for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
    return 0;
}
