/*
 * cpu_baseline.c — TEST/BENCH INFRASTRUCTURE ONLY. A C restatement of the
 * reference's CPU scoring path, the `compute_score` runtime dispatch
 * (scirust/src/attention/slha_v2/simd.rs:23-84): AVX-512 kernels when the host
 * has avx512f (int4 :465-499, nf4 :600-633), else AVX2 int4 (:94-157), else
 * the scalar path; other codecs use the scalar path (tile.rs:267-281).
 * Hamming uses POPCNT (simd.rs:1253-1259). Every (query, tile) pair is scored
 * independently, as slha_score_tiles does (slha-c/src/lib.rs:563-581).
 *
 * Only bench.py's cpu_baseline leg and tests load this library; it is the
 * reported CPU baseline, never part of the product path.
 */
#include <immintrin.h>
#include <pthread.h>
#include <stdint.h>
#include <string.h>

#include "slha_oracle.h"

static const float NF4_CB[16] = {
    -1.0f,   -0.7075f, -0.5421f, -0.4165f, -0.3108f, -0.2158f, -0.1272f, -0.0421f,
    0.0421f, 0.1272f,  0.2158f,  0.3108f,  0.4165f,  0.5421f,  0.7075f,  1.0f,
};

__attribute__((target("popcnt"))) static uint32_t ham_popcnt(const uint64_t* a, const uint64_t* b) {
    return (uint32_t)(__builtin_popcountll(a[0] ^ b[0]) + __builtin_popcountll(a[1] ^ b[1]) +
                      __builtin_popcountll(a[2] ^ b[2]) + __builtin_popcountll(a[3] ^ b[3]));
}

/* simd.rs:465-499 (int4) and :600-633 (nf4): one 16-wide FMA per group. */
__attribute__((target("avx512f,popcnt"))) static float score_avx512(const orc_tile* t,
                                                                   const float* q,
                                                                   const uint64_t* qs) {
    const float inv255 = 1.0f / 255.0f;
    const int nf4 = (t->flags & ORC_FLAG_NF4) != 0;
    const __m512 eight = _mm512_set1_ps(8.0f);
    const __m512 cb = _mm512_loadu_ps(NF4_CB);
    const __m128i mask = _mm_set1_epi8(0x0F);
    __m512 acc = _mm512_setzero_ps();
    for (int g = 0; g < 8; ++g) {
        const __m512 gs = _mm512_set1_ps(t->scale * ((float)t->group_scales[g] * inv255));
        const __m128i packed = _mm_loadl_epi64((const __m128i*)(t->latent_kv + 8 * g));
        const __m128i lo = _mm_and_si128(packed, mask);
        const __m128i hi = _mm_and_si128(_mm_srli_epi16(packed, 4), mask);
        const __m512i idx = _mm512_cvtepu8_epi32(_mm_unpacklo_epi8(lo, hi));
        const __m512 level = nf4 ? _mm512_permutexvar_ps(idx, cb)
                                 : _mm512_sub_ps(_mm512_cvtepi32_ps(idx), eight);
        acc = _mm512_fmadd_ps(_mm512_mul_ps(gs, level), _mm512_loadu_ps(q + 16 * g), acc);
    }
    const float coarse = _mm512_reduce_add_ps(acc);
    if (t->flags & ORC_FLAG_WARM) return coarse;
    return coarse + t->dynamic_lambda * (256.0f - 2.0f * (float)ham_popcnt(qs, t->residual_bitmap));
}

/* simd.rs:94-157: AVX2 int4, two 8-wide FMAs per group. */
__attribute__((target("avx2,fma,popcnt"))) static float score_avx2(const orc_tile* t,
                                                                  const float* q,
                                                                  const uint64_t* qs) {
    const float inv255 = 1.0f / 255.0f;
    const __m256 eight = _mm256_set1_ps(8.0f);
    const __m128i mask = _mm_set1_epi8(0x0F);
    __m256 acc = _mm256_setzero_ps();
    for (int g = 0; g < 8; ++g) {
        const __m256 gs = _mm256_set1_ps(t->scale * ((float)t->group_scales[g] * inv255));
        const __m128i packed = _mm_loadl_epi64((const __m128i*)(t->latent_kv + 8 * g));
        const __m128i lo = _mm_and_si128(packed, mask);
        const __m128i hi = _mm_and_si128(_mm_srli_epi16(packed, 4), mask);
        const __m128i d16 = _mm_unpacklo_epi8(lo, hi);
        const __m256 n0 = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(d16));
        const __m256 n1 = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_srli_si128(d16, 8)));
        acc = _mm256_fmadd_ps(_mm256_mul_ps(gs, _mm256_sub_ps(n0, eight)),
                              _mm256_loadu_ps(q + 16 * g), acc);
        acc = _mm256_fmadd_ps(_mm256_mul_ps(gs, _mm256_sub_ps(n1, eight)),
                              _mm256_loadu_ps(q + 16 * g + 8), acc);
    }
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    s = _mm_hadd_ps(s, s);
    s = _mm_hadd_ps(s, s);
    const float coarse = _mm_cvtss_f32(s);
    if (t->flags & ORC_FLAG_WARM) return coarse;
    return coarse + t->dynamic_lambda * (256.0f - 2.0f * (float)ham_popcnt(qs, t->residual_bitmap));
}

static int g_isa = -1; /* 2 = avx512f, 1 = avx2, 0 = scalar */

int cpu_baseline_isa(void) {
    if (g_isa < 0) {
        __builtin_cpu_init();
        g_isa = __builtin_cpu_supports("avx512f") ? 2 : (__builtin_cpu_supports("avx2") ? 1 : 0);
    }
    return g_isa;
}

static float compute_score(const orc_tile* t, const float* q, const uint64_t* qs, int isa) {
    const uint16_t other = ORC_FLAG_MIXED | ORC_FLAG_TQ3 | ORC_FLAG_MIX3;
    if (!(t->flags & other)) {
        if (isa == 2) return score_avx512(t, q, qs);
        if (isa == 1 && !(t->flags & ORC_FLAG_NF4)) return score_avx2(t, q, qs);
    }
    return orc_compute_score_scalar(t, q, qs);
}

typedef struct {
    const orc_tile* tiles;
    size_t n_tok, group;
    const float* qc;
    const uint64_t* qs;
    float* scores;
    size_t begin, end; /* range over flat (row, query, token) pairs */
    int isa;
} job;

static void* worker(void* arg) {
    job* j = (job*)arg;
    for (size_t p = j->begin; p < j->end; ++p) {
        const size_t t = p % j->n_tok;
        const size_t qrow = p / j->n_tok;
        const size_t row = qrow / j->group;
        j->scores[p] = compute_score(j->tiles + row * j->n_tok + t, j->qc + qrow * 128,
                                     j->qs + qrow * 4, j->isa);
    }
    return NULL;
}

/* Score tiles[n_rows][n_tok] against group queries per row (GQA layout of
 * slha_gpu_score), pairs split statically over n_threads threads. */
void cpu_score_rows(const orc_tile* tiles, size_t n_rows, size_t n_tok, const float* qc,
                    const uint64_t* qs, size_t group, float* scores, int n_threads) {
    const int isa = cpu_baseline_isa();
    const size_t total = n_rows * group * n_tok;
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 256) n_threads = 256;
    pthread_t th[256];
    job jobs[256];
    for (int i = 0; i < n_threads; ++i) {
        jobs[i] = (job){tiles, n_tok, group, qc, qs, scores, total * (size_t)i / (size_t)n_threads,
                        total * (size_t)(i + 1) / (size_t)n_threads, isa};
        if (n_threads > 1)
            pthread_create(&th[i], NULL, worker, &jobs[i]);
        else
            worker(&jobs[i]);
    }
    if (n_threads > 1)
        for (int i = 0; i < n_threads; ++i) pthread_join(th[i], NULL);
}
