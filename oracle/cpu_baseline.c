/*
 * cpu_baseline.c — TEST/BENCH INFRASTRUCTURE ONLY. A C restatement of the
 * reference's CPU scoring path, the `compute_score` runtime dispatch
 * (scirust/src/attention/slha_v2/simd.rs:23-84): with avx512f the AVX-512
 * kernel of the tile's codec, else with avx2 the AVX2 kernel, else the scalar
 * path (tile.rs:267-281), codecs checked in dequant_at's precedence (mixed,
 * tq3, mix3, nf4, int4). Kernels, each in the reference's own operation
 * order (the AVX2 ones multiply then add and sum the 8 lanes in order; the
 * AVX-512 ones fuse the multiply-add and reduce with _mm512_reduce_add_ps):
 *   AVX2    int4 simd.rs:94-157, tq3 :158-238, nf4 :239-309, mixed :310-380,
 *           mix3 :381-463
 *   AVX-512 int4 :464-514, tq3 :515-598, nf4 :599-649, mixed :650-709,
 *           mix3 :710-800
 * Hamming (simd.rs:1240-1282): one vpopcntq over the 256-bit XOR when the host
 * has avx512vpopcntdq and avx512vl, else four POPCNTs. Every (query, tile)
 * pair is scored on its own, as slha_score_tiles does
 * (slha-c/src/lib.rs:563-581).
 *
 * Only bench.py's cpu_baseline leg and tests load this library; it is the
 * reported CPU baseline, never part of the product path.
 */
#include <immintrin.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "slha_oracle.h"

#define CB_TQ3_CODE_BYTES 48 /* constants.rs:102 */
#define CB_MIX3_CODES_OFF 8  /* constants.rs:124 */
#define CB_MIX3_CORR_OFF 50  /* constants.rs:128 */
#define CB_MIXED_HI_DIMS 8   /* constants.rs:59 */

static const float NF4_CB[16] = {
    -1.0f,   -0.7075f, -0.5421f, -0.4165f, -0.3108f, -0.2158f, -0.1272f, -0.0421f,
    0.0421f, 0.1272f,  0.2158f,  0.3108f,  0.4165f,  0.5421f,  0.7075f,  1.0f,
};

static float group_scale(const orc_tile* t, int g) {
    return t->scale * ((float)t->group_scales[g] * (1.0f / 255.0f));
}

static int is_tq3_nocorr(const orc_tile* t) { return (t->flags & ORC_FLAG_TQ3_NOCORR) != 0; }

/* little-endian u32 at byte o of the latent (o + 3 < 64 for every use) */
static uint32_t latent_u32(const orc_tile* t, int o) {
    return (uint32_t)t->latent_kv[o] | ((uint32_t)t->latent_kv[o + 1] << 8) |
           ((uint32_t)t->latent_kv[o + 2] << 16) | ((uint32_t)t->latent_kv[o + 3] << 24);
}

/* ---------------------------------------------------------------- Hamming */

__attribute__((target("popcnt"))) static uint32_t ham_popcnt(const uint64_t* a, const uint64_t* b) {
    uint32_t h = 0;
    for (int w = 0; w < 4; ++w) h += (uint32_t)__builtin_popcountll(a[w] ^ b[w]);
    return h;
}

__attribute__((target("avx512vpopcntdq,avx512vl"))) static uint32_t ham_vpopcntdq(const uint64_t* a,
                                                                                  const uint64_t* b) {
    const __m256i x = _mm256_xor_si256(_mm256_loadu_si256((const __m256i*)a),
                                       _mm256_loadu_si256((const __m256i*)b));
    uint64_t lanes[4];
    _mm256_storeu_si256((__m256i*)lanes, _mm256_popcnt_epi64(x));
    return (uint32_t)(lanes[0] + lanes[1] + lanes[2] + lanes[3]);
}

static int g_vpop = -1;

static uint32_t hamming(const uint64_t* a, const uint64_t* b) {
    if (g_vpop < 0) {
        __builtin_cpu_init();
        g_vpop = __builtin_cpu_supports("avx512vpopcntdq") && __builtin_cpu_supports("avx512vl");
    }
    return g_vpop ? ham_vpopcntdq(a, b) : ham_popcnt(a, b);
}

/* tile.rs:261-264; the coarse sum is returned alone for WARM tiles */
static float finish(const orc_tile* t, float coarse, const uint64_t* qs) {
    if (t->flags & ORC_FLAG_WARM) return coarse;
    return coarse + t->dynamic_lambda * (256.0f - 2.0f * (float)hamming(qs, t->residual_bitmap));
}

/* -------------------------------------------------------------------- AVX2 */

/* 16 nibbles of 8 latent bytes in dimension order (low nibble first) */
__attribute__((target("avx2"))) static __m128i nibbles16(const uint8_t* p) {
    const __m128i packed = _mm_loadl_epi64((const __m128i*)p);
    const __m128i m = _mm_set1_epi8(0x0F);
    return _mm_unpacklo_epi8(_mm_and_si128(packed, m), _mm_and_si128(_mm_srli_epi16(packed, 4), m));
}

__attribute__((target("avx2"))) static float hsum8_in_order(__m256 acc) {
    float lane[8];
    _mm256_storeu_ps(lane, acc);
    float s = 0.0f;
    for (int i = 0; i < 8; ++i) s += lane[i];
    return s;
}

/* (nibble - 8) * gs for 8 dims, times q, added to acc */
__attribute__((target("avx2"))) static __m256 avx2_int4_half(__m128i bytes, __m256 gs, const float* q,
                                                             __m256 acc) {
    const __m256 n = _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(bytes));
    const __m256 v = _mm256_mul_ps(gs, _mm256_sub_ps(n, _mm256_set1_ps(8.0f)));
    return _mm256_add_ps(acc, _mm256_mul_ps(v, _mm256_loadu_ps(q)));
}

__attribute__((target("avx2"))) static float avx2_int4(const orc_tile* t, const float* q,
                                                       const uint64_t* qs) {
    __m256 acc = _mm256_setzero_ps();
    for (int g = 0; g < 8; ++g) {
        const __m256 gs = _mm256_set1_ps(group_scale(t, g));
        const __m128i d16 = nibbles16(t->latent_kv + 8 * g);
        acc = avx2_int4_half(d16, gs, q + 16 * g, acc);
        acc = avx2_int4_half(_mm_srli_si128(d16, 8), gs, q + 16 * g + 8, acc);
    }
    return finish(t, hsum8_in_order(acc), qs);
}

/* NF4 levels of 8 nibbles: one permute per codebook half, blended on bit 3 */
__attribute__((target("avx2"))) static __m256 avx2_nf4_half(__m128i bytes, __m256 gs, const float* q,
                                                            __m256 acc) {
    const __m256i nib = _mm256_cvtepu8_epi32(bytes);
    const __m256 lo = _mm256_permutevar8x32_ps(_mm256_loadu_ps(NF4_CB), nib);
    const __m256 hi = _mm256_permutevar8x32_ps(_mm256_loadu_ps(NF4_CB + 8), nib);
    const __m256 pick = _mm256_castsi256_ps(_mm256_cmpgt_epi32(nib, _mm256_set1_epi32(7)));
    const __m256 v = _mm256_mul_ps(gs, _mm256_blendv_ps(lo, hi, pick));
    return _mm256_add_ps(acc, _mm256_mul_ps(v, _mm256_loadu_ps(q)));
}

__attribute__((target("avx2"))) static float avx2_nf4(const orc_tile* t, const float* q,
                                                      const uint64_t* qs) {
    __m256 acc = _mm256_setzero_ps();
    for (int g = 0; g < 8; ++g) {
        const __m256 gs = _mm256_set1_ps(group_scale(t, g));
        const __m128i d16 = nibbles16(t->latent_kv + 8 * g);
        acc = avx2_nf4_half(d16, gs, q + 16 * g, acc);
        acc = avx2_nf4_half(_mm_srli_si128(d16, 8), gs, q + 16 * g + 8, acc);
    }
    return finish(t, hsum8_in_order(acc), qs);
}

/* 8-bit head of the mixed layouts: (byte - 128) * gs[0] times q[0..8] */
__attribute__((target("avx2"))) static __m256 avx2_head(const orc_tile* t, const float* q) {
    const __m256 hs = _mm256_set1_ps(group_scale(t, 0));
    const __m256 head =
        _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i*)t->latent_kv)));
    const __m256 hv = _mm256_mul_ps(hs, _mm256_sub_ps(head, _mm256_set1_ps(128.0f)));
    return _mm256_mul_ps(hv, _mm256_loadu_ps(q));
}

__attribute__((target("avx2"))) static float avx2_mixed(const orc_tile* t, const float* q,
                                                        const uint64_t* qs) {
    __m256 acc = avx2_head(t, q);
    for (int g = 0; g < 7; ++g) {
        const int base = CB_MIXED_HI_DIMS + 16 * g;
        const __m256 gs = _mm256_set1_ps(group_scale(t, 1 + g));
        const __m128i d16 = nibbles16(t->latent_kv + CB_MIXED_HI_DIMS + 8 * g);
        acc = avx2_int4_half(d16, gs, q + base, acc);
        acc = avx2_int4_half(_mm_srli_si128(d16, 8), gs, q + base + 8, acc);
    }
    return finish(t, hsum8_in_order(acc), qs);
}

/* TQ3 block of 8 dims: codes at bits 3l of the 4-byte window at `codes_off`,
 * correction bits in the byte at `corr_off`; level = code - 3.75 + 0.5 corr
 * (code - 3.5 without the plane), times gs, times q, added to acc */
__attribute__((target("avx2"))) static __m256 avx2_tq3_block(const orc_tile* t, int codes_off,
                                                             int corr_off, __m256 gs,
                                                             const float* q, __m256 acc) {
    const int nocorr = is_tq3_nocorr(t);
    const __m256i codes = _mm256_and_si256(
        _mm256_srlv_epi32(_mm256_set1_epi32((int)latent_u32(t, codes_off)),
                          _mm256_setr_epi32(0, 3, 6, 9, 12, 15, 18, 21)),
        _mm256_set1_epi32(7));
    __m256 level = _mm256_sub_ps(_mm256_cvtepi32_ps(codes), _mm256_set1_ps(nocorr ? 3.5f : 3.75f));
    if (!nocorr) {
        const __m256i corr = _mm256_and_si256(
            _mm256_srlv_epi32(_mm256_set1_epi32((int)t->latent_kv[corr_off]),
                              _mm256_setr_epi32(0, 1, 2, 3, 4, 5, 6, 7)),
            _mm256_set1_epi32(1));
        level = _mm256_add_ps(level, _mm256_mul_ps(_mm256_cvtepi32_ps(corr), _mm256_set1_ps(0.5f)));
    }
    const __m256 v = _mm256_mul_ps(level, gs);
    return _mm256_add_ps(acc, _mm256_mul_ps(v, _mm256_loadu_ps(q)));
}

__attribute__((target("avx2"))) static float avx2_tq3(const orc_tile* t, const float* q,
                                                      const uint64_t* qs) {
    __m256 acc = _mm256_setzero_ps();
    for (int b = 0; b < 16; ++b)
        acc = avx2_tq3_block(t, 3 * b, CB_TQ3_CODE_BYTES + b, _mm256_set1_ps(group_scale(t, b / 2)),
                             q + 8 * b, acc);
    return finish(t, hsum8_in_order(acc), qs);
}

__attribute__((target("avx2"))) static float avx2_mix3(const orc_tile* t, const float* q,
                                                       const uint64_t* qs) {
    __m256 acc = avx2_head(t, q);
    for (int b = 0; b < 14; ++b)
        acc = avx2_tq3_block(t, CB_MIX3_CODES_OFF + 3 * b, CB_MIX3_CORR_OFF + b,
                             _mm256_set1_ps(group_scale(t, 1 + b / 2)), q + CB_MIXED_HI_DIMS + 8 * b,
                             acc);
    return finish(t, hsum8_in_order(acc), qs);
}

/* ----------------------------------------------------------------- AVX-512 */

__attribute__((target("avx512f"))) static float avx512_int4(const orc_tile* t, const float* q,
                                                            const uint64_t* qs) {
    __m512 acc = _mm512_setzero_ps();
    for (int g = 0; g < 8; ++g) {
        const __m512 n = _mm512_cvtepi32_ps(_mm512_cvtepu8_epi32(nibbles16(t->latent_kv + 8 * g)));
        const __m512 v = _mm512_mul_ps(_mm512_set1_ps(group_scale(t, g)),
                                       _mm512_sub_ps(n, _mm512_set1_ps(8.0f)));
        acc = _mm512_fmadd_ps(v, _mm512_loadu_ps(q + 16 * g), acc);
    }
    return finish(t, _mm512_reduce_add_ps(acc), qs);
}

__attribute__((target("avx512f"))) static float avx512_nf4(const orc_tile* t, const float* q,
                                                           const uint64_t* qs) {
    const __m512 cb = _mm512_loadu_ps(NF4_CB);
    __m512 acc = _mm512_setzero_ps();
    for (int g = 0; g < 8; ++g) {
        const __m512 level =
            _mm512_permutexvar_ps(_mm512_cvtepu8_epi32(nibbles16(t->latent_kv + 8 * g)), cb);
        const __m512 v = _mm512_mul_ps(_mm512_set1_ps(group_scale(t, g)), level);
        acc = _mm512_fmadd_ps(v, _mm512_loadu_ps(q + 16 * g), acc);
    }
    return finish(t, _mm512_reduce_add_ps(acc), qs);
}

/* the 8-lane head, zero-extended into a 16-wide accumulator */
__attribute__((target("avx512f"))) static __m512 avx512_head(const orc_tile* t, const float* q) {
    const __m256 hs = _mm256_set1_ps(group_scale(t, 0));
    const __m256 head =
        _mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i*)t->latent_kv)));
    const __m256 hv = _mm256_mul_ps(hs, _mm256_sub_ps(head, _mm256_set1_ps(128.0f)));
    return _mm512_zextps256_ps512(_mm256_mul_ps(hv, _mm256_loadu_ps(q)));
}

__attribute__((target("avx512f"))) static float avx512_mixed(const orc_tile* t, const float* q,
                                                             const uint64_t* qs) {
    __m512 acc = avx512_head(t, q);
    for (int g = 0; g < 7; ++g) {
        const __m512 n = _mm512_cvtepi32_ps(
            _mm512_cvtepu8_epi32(nibbles16(t->latent_kv + CB_MIXED_HI_DIMS + 8 * g)));
        const __m512 v = _mm512_mul_ps(_mm512_set1_ps(group_scale(t, 1 + g)),
                                       _mm512_sub_ps(n, _mm512_set1_ps(8.0f)));
        acc = _mm512_fmadd_ps(v, _mm512_loadu_ps(q + CB_MIXED_HI_DIMS + 16 * g), acc);
    }
    return finish(t, _mm512_reduce_add_ps(acc), qs);
}

/* TQ3 group of 16 dims: two 4-byte windows (bytes codes_off, codes_off + 3),
 * 16 correction bits at corr_off; the correction enters with one FMA */
__attribute__((target("avx512f"))) static __m512 avx512_tq3_group(const orc_tile* t, int codes_off,
                                                                  int corr_off, float gs,
                                                                  const float* q, __m512 acc) {
    const int nocorr = is_tq3_nocorr(t);
    const __m512i windows = _mm512_inserti64x4(
        _mm512_castsi256_si512(_mm256_set1_epi32((int)latent_u32(t, codes_off))),
        _mm256_set1_epi32((int)latent_u32(t, codes_off + 3)), 1);
    const __m512i codes = _mm512_and_epi32(
        _mm512_srlv_epi32(windows, _mm512_setr_epi32(0, 3, 6, 9, 12, 15, 18, 21, 0, 3, 6, 9, 12, 15,
                                                     18, 21)),
        _mm512_set1_epi32(7));
    __m512 level = _mm512_sub_ps(_mm512_cvtepi32_ps(codes), _mm512_set1_ps(nocorr ? 3.5f : 3.75f));
    if (!nocorr) {
        const int c16 = (int)t->latent_kv[corr_off] | ((int)t->latent_kv[corr_off + 1] << 8);
        const __m512i corr = _mm512_and_epi32(
            _mm512_srlv_epi32(_mm512_set1_epi32(c16), _mm512_setr_epi32(0, 1, 2, 3, 4, 5, 6, 7, 8, 9,
                                                                         10, 11, 12, 13, 14, 15)),
            _mm512_set1_epi32(1));
        level = _mm512_fmadd_ps(_mm512_cvtepi32_ps(corr), _mm512_set1_ps(0.5f), level);
    }
    const __m512 v = _mm512_mul_ps(level, _mm512_set1_ps(gs));
    return _mm512_fmadd_ps(v, _mm512_loadu_ps(q), acc);
}

__attribute__((target("avx512f"))) static float avx512_tq3(const orc_tile* t, const float* q,
                                                           const uint64_t* qs) {
    __m512 acc = _mm512_setzero_ps();
    for (int g = 0; g < 8; ++g)
        acc = avx512_tq3_group(t, 6 * g, CB_TQ3_CODE_BYTES + 2 * g, group_scale(t, g), q + 16 * g, acc);
    return finish(t, _mm512_reduce_add_ps(acc), qs);
}

__attribute__((target("avx512f"))) static float avx512_mix3(const orc_tile* t, const float* q,
                                                            const uint64_t* qs) {
    __m512 acc = avx512_head(t, q);
    for (int g = 0; g < 7; ++g)
        acc = avx512_tq3_group(t, CB_MIX3_CODES_OFF + 6 * g, CB_MIX3_CORR_OFF + 2 * g,
                               group_scale(t, 1 + g), q + CB_MIXED_HI_DIMS + 16 * g, acc);
    return finish(t, _mm512_reduce_add_ps(acc), qs);
}

/* ---------------------------------------------------------------- dispatch */

static int g_isa = -1; /* 2 = avx512f, 1 = avx2, 0 = scalar */

int cpu_baseline_isa(void) {
    if (g_isa < 0) {
        __builtin_cpu_init();
        g_isa = __builtin_cpu_supports("avx512f") ? 2 : (__builtin_cpu_supports("avx2") ? 1 : 0);
    }
    return g_isa;
}

/* 1 when Hamming runs on vpopcntq (avx512vpopcntdq + avx512vl), else 0 */
int cpu_baseline_vpopcntdq(void) {
    const uint64_t z[4] = {0, 0, 0, 0};
    (void)hamming(z, z);
    return g_vpop;
}

static float compute_score(const orc_tile* t, const float* q, const uint64_t* qs, int isa) {
    const uint16_t f = t->flags;
    if (isa == 2) {
        if (f & ORC_FLAG_MIXED) return avx512_mixed(t, q, qs);
        if (f & ORC_FLAG_TQ3) return avx512_tq3(t, q, qs);
        if (f & ORC_FLAG_MIX3) return avx512_mix3(t, q, qs);
        if (f & ORC_FLAG_NF4) return avx512_nf4(t, q, qs);
        return avx512_int4(t, q, qs);
    }
    if (isa == 1) {
        if (f & ORC_FLAG_MIXED) return avx2_mixed(t, q, qs);
        if (f & ORC_FLAG_TQ3) return avx2_tq3(t, q, qs);
        if (f & ORC_FLAG_MIX3) return avx2_mix3(t, q, qs);
        if (f & ORC_FLAG_NF4) return avx2_nf4(t, q, qs);
        return avx2_int4(t, q, qs);
    }
    return orc_compute_score_scalar(t, q, qs);
}

/* Score n tiles against one query with an explicit ISA level (tests): returns
 * -1 when the host lacks it. */
int cpu_score_tiles_isa(const orc_tile* tiles, size_t n, const float* q, const uint64_t* qs,
                        float* out, int isa) {
    if (isa < 0 || isa > cpu_baseline_isa()) return -1;
    for (size_t i = 0; i < n; ++i) out[i] = compute_score(tiles + i, q, qs, isa);
    return 0;
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
    (void)hamming(qs, qs); /* resolve the Hamming dispatch before the threads start */
    if (n_threads < 1) n_threads = 1;
    if (n_threads > 1024) n_threads = 1024;
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)n_threads);
    job* jobs = (job*)malloc(sizeof(job) * (size_t)n_threads);
    if (!th || !jobs) { /* cannot spread the work: score on this thread */
        free(th);
        free(jobs);
        job one = {tiles, n_tok, group, qc, qs, scores, 0, total, isa};
        worker(&one);
        return;
    }
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
    free(th);
    free(jobs);
}
