// slha_kernels.hip — gfx950 kernels of the SLHA v2 tile path.
//
// Compiled with -ffp-contract=off: every "exact" routine below performs the
// reference's f32 operations in the reference's order (Rust never contracts
// a*b+c). Fast routines contract explicitly with fmaf().
//
// Kernels:
//   score_rows_kernel      eq. 2.3 over tile rows, GQA fan-out (tile.rs:267-281)
//   encode_kernel<CODEC>   key -> tile, mode R/Z (codec/*.rs, scenario.rs:95-114)
//   prepare_query_kernel   q -> (q_coarse, q_sign) (scenario.rs:70-83)
//   decode_kernel          tile -> latent (+ sign-sketch residual) (learned.rs:283-321)
//   validate_kernel        slha-c/src/lib.rs:244-286 on device
//   ccos_apply_kernel      page_out / drop_correction (ccos.rs:369-397)
//   learned_*_kernel       d > 128 LearnedModel encode / query / decode (learned.rs:257-408)
//   attn_*_kernel          decode attention softmax(s * scale) . V (benchmark_decode.rs:29-90)
//   eventlog_*_kernel      EventLog records of evicted tiles, and rehydrate (eventlog.rs:9-36)
//   observe_*_kernel       CCOS H2O importance from the arena's scores (ccos.rs:257-300)
#include "slha_device.h"
#include "slha_launch.h"
#include "slha_tile_io.h"

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <utility>

namespace slha {

// ---------------------------------------------------------------------------
// Tile loads

__device__ __forceinline__ void load_tile(const uint4* __restrict__ p, uint32_t* w) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint4 v = p[j];
        w[4 * j + 0] = v.x;
        w[4 * j + 1] = v.y;
        w[4 * j + 2] = v.z;
        w[4 * j + 3] = v.w;
    }
}

// ---------------------------------------------------------------------------
// Scoring.
//
// One lane scores one tile against all `group` queries of its row: the tile
// (128 B) is read from HBM once into 32 VGPRs; queries are wave-uniform, so
// the compiler reads them through the scalar cache and every MAC is a single
// v_fma_f32 with an SGPR operand. The tile is decoded one 16-dim group at a
// time for a chunk of kQC queries, which keeps the register footprint small
// enough for several waves per SIMD.
//
// Fast mode factors the per-group scale out of the group sum:
//     sum_{d in g} q_d * (a_g * m_d - b_g) = a_g * (sum q_d m_d - b_g/a_g-free offset * Q_g)
// with m_d a small integer decoded by integer ops (INT4 nibble, TQ3 2*code+corr),
// Q_g = sum_{d in g} q_d computed once per workgroup into LDS. Mixed/MIX3
// tiles, whose sections do not align to 16-dim groups, decode to scaled
// values. EXACT mode evaluates tile.rs:267-281 verbatim (sequential f32, no
// FMA) and is bit-identical to the scalar reference.
//
// A wave whose lanes hold different codecs runs each codec's path with only
// the matching lanes active; a codec-uniform wave runs exactly one path.


enum : int { kClsInt4 = 0, kClsNF4 = 1, kClsMixed = 2, kClsTQ3 = 3, kClsMix3 = 4 };

__device__ __forceinline__ int codec_class(uint32_t flags) {  // tile.rs:142-157 precedence
    if (flags & kFlagMixed) return kClsMixed;
    if (flags & kFlagTQ3) return kClsTQ3;
    if (flags & kFlagMix3) return kClsMix3;
    if (flags & kFlagNF4) return kClsNF4;
    return kClsInt4;
}

// Fast decode of dims [16g, 16g+16) into m[16]; returns the group factor a
// and offset b such that the group's dequantised values are a*(m - b).
template <int CLS>
__device__ __forceinline__ void decode_group_fast(const uint32_t* w, int g, float s255,
                                                  const float* cb, float* m, float& a, float& b) {
    const uint32_t* lw = w;
    const float gsf = gs_at(w + 30, g);
    const uint32_t flags = w[29] >> 16;
    if constexpr (CLS == kClsInt4 || CLS == kClsNF4) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint32_t x = lw[2 * g + k];
            const uint32_t lo = x & 0x0F0F0F0Fu;
            const uint32_t hi = (x >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t n0 = (lo >> (8 * j)) & 0xFFu, n1 = (hi >> (8 * j)) & 0xFFu;
                if constexpr (CLS == kClsInt4) {
                    m[8 * k + 2 * j] = (float)n0;
                    m[8 * k + 2 * j + 1] = (float)n1;
                } else {
                    m[8 * k + 2 * j] = cb[n0];
                    m[8 * k + 2 * j + 1] = cb[n1];
                }
            }
        }
        a = gsf * s255;
        b = CLS == kClsInt4 ? 8.0f : 0.0f;
    } else if constexpr (CLS == kClsTQ3) {
        const bool nocorr = (flags & kFlagNoCorr) != 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int d = 16 * g + i;
            const uint32_t code = bits3_at(lw, 3 * d);
            const uint32_t corr = nocorr ? 0u : bit_at(lw, 384 + d);
            m[i] = (float)((code << 1) | corr);
        }
        a = 0.5f * gsf * s255;
        b = nocorr ? 7.0f : 7.5f;
    } else {  // mixed / MIX3: scaled values, a = 1, b = 0
        const float s0 = gs_at(w + 30, 0) * s255;
        const bool nocorr = (flags & kFlagNoCorr) != 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int d = 16 * g + i;
            if (d < 8) {
                m[i] = fmaf((float)byte_at(lw, d), s0, -128.0f * s0);
            } else if (d < 120) {
                const int ld = d - 8;
                const float sg = gs_at(w + 30, 1 + ld / 16) * s255;
                if constexpr (CLS == kClsMixed) {
                    m[i] = fmaf((float)nib_at(lw, 16 + ld), sg, -8.0f * sg);
                } else {
                    const uint32_t code = bits3_at(lw, 64 + 3 * ld);
                    const uint32_t corr = nocorr ? 0u : bit_at(lw, 400 + ld);
                    m[i] = fmaf((float)((code << 1) | corr), 0.5f * sg,
                                (nocorr ? -3.5f : -3.75f) * sg);
                }
            } else {
                m[i] = 0.0f;
            }
        }
        a = 1.0f;
        b = 0.0f;
    }
}

// Exact dequant of dims [16g, 16g+16) (tile.rs:141-246, operation order kept).
template <int CLS>
__device__ __forceinline__ void decode_group_exact(const uint32_t* w, int g, const float* cb,
                                                   float* k) {
    const uint32_t* lw = w;
    const uint32_t* gw = w + 30;
    const float scale = __uint_as_float(w[24]);
    const bool nocorr = ((w[29] >> 16) & kFlagNoCorr) != 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int d = 16 * g + i;
        if constexpr (CLS == kClsInt4) {
            k[i] = (float)((int)nib_at(lw, d) - 8) * group_scale_exact(scale, gs_at(gw, g));
        } else if constexpr (CLS == kClsNF4) {
            k[i] = cb[nib_at(lw, d)] * group_scale_exact(scale, gs_at(gw, g));
        } else if constexpr (CLS == kClsTQ3) {
            k[i] = tq3_level_exact(lw, 0, 384, d, nocorr) * group_scale_exact(scale, gs_at(gw, g));
        } else {
            if (d < 8) {
                k[i] = (float)((int)byte_at(lw, d) - 128) * section_scale_exact(scale, gs_at(gw, 0));
            } else if (d < 120) {
                const int ld = d - 8;
                const float sec = section_scale_exact(scale, gs_at(gw, 1 + ld / 16));
                if constexpr (CLS == kClsMixed)
                    k[i] = (float)((int)nib_at(lw, 16 + ld) - 8) * sec;
                else
                    k[i] = tq3_level_exact(lw, 64, 400, ld, nocorr) * sec;
            } else {
                k[i] = 0.0f;
            }
        }
    }
}

// Score one tile (in w) against queries qrow0 .. qrow0+group-1, writing
// query j's score to out[j * stride + t]. This per-lane path serves EXACT
// mode and waves whose lanes hold different codecs. It decodes one 16-dim
// group at a time for one query at a time; the empty asm makes the tile words
// opaque per query so the compiler cannot hoist all 128 decoded values out of
// the query loop (which would cost 128 VGPRs and most of the occupancy).
template <int CLS, bool EXACT, bool HAM>
__device__ __forceinline__ void score_lane(const uint32_t* w_in, uint32_t group, size_t qrow0,
                                           const float* __restrict__ qc,
                                           const uint32_t* __restrict__ qs, const float* cb,
                                           float* __restrict__ out, uint32_t* __restrict__ ham,
                                           size_t stride, uint32_t t) {
#pragma unroll 1
    for (uint32_t j = 0; j < group; ++j) {
        uint32_t w[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            w[i] = w_in[i];
            asm volatile("" : "+v"(w[i]));
        }
        const float scale = __uint_as_float(w[24]);
        const float lambda = __uint_as_float(w[25]);
        const bool warm = ((w[29] >> 16) & kFlagWarm) != 0;
        const float s255 = scale * (1.0f / 255.0f);
        const size_t qrow = qrow0 + j;
        const float* qrowp = qc + qrow * kDC;
        float acc = 0.0f;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            float m[16];
            const float* q = qrowp + 16 * g;
            if constexpr (EXACT) {
                decode_group_exact<CLS>(w, g, cb, m);
#pragma unroll
                for (int i = 0; i < 16; ++i) acc += q[i] * m[i];
            } else {
                float a, b;
                decode_group_fast<CLS>(w, g, s255, cb, m, a, b);
                float p = 0.0f;
#pragma unroll
                for (int i = 0; i < 16; ++i) p = fmaf(q[i], m[i] - b, p);
                acc = fmaf(a, p, acc);
            }
        }
        const uint32_t h = hamming_words(w + 16, qs + qrow * 8);
        float score = acc;
        if (!warm) {
            if constexpr (EXACT)
                score = score + lambda * (256.0f - 2.0f * (float)h);
            else
                score = fmaf(lambda, 256.0f - 2.0f * (float)h, score);
        }
        store_out(out + (size_t)j * stride + t, score);
        if constexpr (HAM) store_out(ham + (size_t)j * stride + t, h);
    }
}

// ---------------------------------------------------------------------------
// Fast path on the matrix cores (v_mfma_f32_4x4x1_16b_f32).
//
// One wave scores its 64 tiles against a chunk of 4 queries. In the 16-block
// 4x4x1 layout lane l supplies B column l and receives C column l in its four
// result registers, while row r of block l/4 takes A from lane 4*(l/4) + r.
// So lane l feeds dim d of ITS tile as B and q_{l%4}[d] as A, and after 128
// MFMAs (one per dim) holds the four query dot products of its own tile: no
// cross-lane traffic. B is the dequantised value a_g*(m - b_g) of
// decode_group_fast (one FMA per dim); products and sums are f32.

typedef float v4f __attribute__((ext_vector_type(4)));


constexpr uint32_t kQStride = 132;      // LDS row stride of a staged query (floats)
constexpr uint32_t kQStrideH = 264;     // u16 words per staged f16 query (512 B + 16 B pad)
constexpr uint32_t kMfmaMaxGroup = 64;  // queries staged in LDS per workgroup

// Dynamic LDS of the fast kernels: f32 staged queries (MFMA f32 paths), f16
// hi/lo staged queries and their 2^e factors (INT4 f16 path).
struct StagedQueries {
    float* q32;
    uint16_t* q16;
    float* qexp;
};

// rows_alloc: staged query rows the launch allocated (staging_bytes(rows_alloc)).
__device__ __forceinline__ StagedQueries carve_staging(float* smem, uint32_t rows_alloc) {
    const uint32_t rows = rows_alloc;
    StagedQueries sq;
    sq.q32 = smem;
    sq.q16 = reinterpret_cast<uint16_t*>(smem + rows * kQStride);
    sq.qexp = reinterpret_cast<float*>(sq.q16 + rows * kQStrideH);
    return sq;
}

__host__ __device__ constexpr uint32_t staging_rows(uint32_t group) { return (group + 3u) & ~3u; }
__host__ __device__ constexpr size_t staging_bytes(uint32_t rows_alloc) {
    return (size_t)rows_alloc * (kQStride * 4u + kQStrideH * 2u + 4u);
}

template <int CLS>
__device__ __forceinline__ void score_wave_mfma(const uint32_t* w_in, bool valid, uint32_t group,
                                                size_t qrow0, const float* qlds, const float* cb,
                                                const uint32_t* __restrict__ qs,
                                                float* __restrict__ out, size_t stride,
                                                uint32_t t) {
    const uint32_t r = threadIdx.x & 3u;
#pragma unroll 1
    for (uint32_t c0 = 0; c0 < group; c0 += 4) {
        // Opaque per chunk: keeps the decode inside the loop (see score_lane).
        uint32_t w[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            w[i] = w_in[i];
            asm volatile("" : "+v"(w[i]));
        }
        const float lambda = __uint_as_float(w[25]);
        const bool warm = ((w[29] >> 16) & kFlagWarm) != 0;
        const float s255 = __uint_as_float(w[24]) * (1.0f / 255.0f);
        const float* qa = qlds + (c0 + r) * kQStride;
        v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            float m[16], ga, gb;
            decode_group_fast<CLS>(w, g, s255, cb, m, ga, gb);
            const float off = -ga * gb;
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                const float4 x = *reinterpret_cast<const float4*>(qa + 16 * g + i);
                const float qv[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    // dequantised value a_g * (m - b_g), then one MFMA step
                    const float v = (CLS == kClsMixed || CLS == kClsMix3) ? m[i + k]
                                                                          : fmaf(m[i + k], ga, off);
                    acc = __builtin_amdgcn_mfma_f32_4x4x1f32(qv[k], v, acc, 0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            if (c0 + rr < group) {
                float sc = acc[rr];
                const uint32_t h = hamming_words(w + 16, qs + (qrow0 + c0 + rr) * 8);
                if (!warm) sc = fmaf(lambda, 256.0f - 2.0f * (float)h, sc);
                if (valid) store_out(out + (size_t)(c0 + rr) * stride + t, sc);
            }
        }
    }
}

// INT4 fast path on v_mfma_f32_4x4x4_16b_f16 (same lane = tile layout,
// four dims per MFMA). B is the exact integer n - 8 in f16, built from
// magic-number halves: for a latent dword x holding nibbles n0..n7,
// (x & 0x000F000F) | 0x64006400 is the f16 pair (1024 + n0, 1024 + n4) and
// (x & 0x00F000F0) | 0x64006400 is (1024 + 16 n1, 1024 + 16 n5); one
// v_and_or_b32 plus one packed add / fma per pair gives n - 8 exactly. The
// dims of a dword therefore enter the MFMA in the order
// (d0, d4, d1, d5 | d2, d6, d3, d7), and the staged queries use the same
// order. Each 16-dim group is accumulated on its own and then added in with
// its group scale gs, once per (tile, query, group) instead of once per
// element. Each query is prescaled by an exact power of
// two 2^-e (|q 2^-e| <= 1) and split into f16 hi + lo halves, so q is carried
// to ~2^-20 relative and every product is exact in the f32 accumulator. The
// tile's scale/255 and 2^e are applied once per (tile, query) at the end.

typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v2h as_v2h(uint32_t u) { return __builtin_bit_cast(v2h, u); }

// ONE_CHUNK: group <= 4, a single pass with no loop-carried copy of the tile.
template <bool ONE_CHUNK>
__device__ __forceinline__ void score_wave_int4_f16(const uint32_t* w_in, bool valid,
                                                    uint32_t group, size_t qrow0,
                                                    const uint16_t* qh, const float* qexp,
                                                    const uint32_t* __restrict__ qs,
                                                    float* __restrict__ out, size_t stride,
                                                    uint32_t t) {
    const uint32_t r = threadIdx.x & 3u;
    const v2h k_lo = v2h{(_Float16)-1032.0f, (_Float16)-1032.0f};
    const v2h k_sixteenth = v2h{(_Float16)0.0625f, (_Float16)0.0625f};
    const v2h k_hi = v2h{(_Float16)-72.0f, (_Float16)-72.0f};
    // Held in a VGPR: a VOP3 op reads at most one SGPR or literal here, and
    // the masks take that slot in v_and_or_b32.
    uint32_t magic = 0x64006400u;
    asm volatile("" : "+v"(magic));
    uint32_t w[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) w[i] = w_in[i];
#pragma unroll 1
    for (uint32_t c0 = 0; c0 < group; c0 += 4) {
        // Opaque per chunk: keeps the decode inside the loop (see score_lane).
        if constexpr (!ONE_CHUNK) {
#pragma unroll
            for (int i = 0; i < 32; ++i) asm volatile("" : "+v"(w[i]));
        }
        const uint16_t* qa = qh + (c0 + r) * kQStrideH;
        v4f dot = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int p = 2 * g; p < 2 * g + 2; ++p) {
                const uint32_t x = w[p];
                const uint32_t x8 = x >> 8;
                const v2h l0 = as_v2h((x & 0x000F000Fu) | magic) + k_lo;
                const v2h l1 = __builtin_elementwise_fma(as_v2h((x & 0x00F000F0u) | magic),
                                                         k_sixteenth, k_hi);
                const v2h l2 = as_v2h((x8 & 0x000F000Fu) | magic) + k_lo;
                const v2h l3 = __builtin_elementwise_fma(as_v2h((x8 & 0x00F000F0u) | magic),
                                                         k_sixteenth, k_hi);
                const v4h b01 = v4h{l0.x, l0.y, l1.x, l1.y};
                const v4h b23 = v4h{l2.x, l2.y, l3.x, l3.y};
                const uint4 hq = *reinterpret_cast<const uint4*>(qa + 16 * p);      // hi halves
                const uint4 lq = *reinterpret_cast<const uint4*>(qa + 16 * p + 8);  // lo halves
                const v4h a_hi01 = __builtin_bit_cast(v4h, make_uint2(hq.x, hq.y));
                const v4h a_hi23 = __builtin_bit_cast(v4h, make_uint2(hq.z, hq.w));
                const v4h a_lo01 = __builtin_bit_cast(v4h, make_uint2(lq.x, lq.y));
                const v4h a_lo23 = __builtin_bit_cast(v4h, make_uint2(lq.z, lq.w));
                acc = __builtin_amdgcn_mfma_f32_4x4x4f16(a_hi01, b01, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_4x4x4f16(a_lo01, b01, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_4x4x4f16(a_hi23, b23, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_4x4x4f16(a_lo23, b23, acc, 0, 0, 0);
            }
            const float gsf = gs_at(w + 30, g);
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) dot[rr] = fmaf(acc[rr], gsf, dot[rr]);
        }
        const float s255 = __uint_as_float(w[24]) * (1.0f / 255.0f);
        const float lambda = __uint_as_float(w[25]);
        const bool warm = ((w[29] >> 16) & kFlagWarm) != 0;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            if (c0 + rr < group) {
                float sc = dot[rr] * (s255 * qexp[c0 + rr]);
                const uint32_t h = hamming_words(w + 16, qs + (qrow0 + c0 + rr) * 8);
                if (!warm) sc = fmaf(lambda, 256.0f - 2.0f * (float)h, sc);
                if (valid) store_out(out + (size_t)(c0 + rr) * stride + t, sc);
            }
        }
        if constexpr (ONE_CHUNK) break;
    }
}

// Stage queries for the f16 INT4 path: per query, dword position p (8 dims)
// holds 8 hi halves then 8 lo halves in the (d0, d4, d1, d5, d2, d6, d3, d7)
// order; qexp[j] = 2^e with |q_j| <= 2^e. One wave per query; rows past
// `group` up to a multiple of 4 are zero.
// Runs the MFMA path when every valid lane of the wave holds the same codec
// (always true for arrays written by one encoder call); returns false when
// the wave must fall back to the per-lane path.
__device__ __forceinline__ bool score_wave_try_mfma(const uint32_t* w, bool valid, uint32_t group,
                                                    size_t qrow0, const float* qlds, const float* cb,
                                                    const uint16_t* qh, const float* qexp,
                                                    const uint32_t* __restrict__ qs,
                                                    float* __restrict__ out, size_t stride,
                                                    uint32_t t) {
    const int cls = valid ? codec_class(w[29] >> 16) : -1;
    const int c0 = __builtin_amdgcn_readfirstlane(cls);
    if (c0 < 0 || !__all(cls == c0 || cls < 0)) return false;
    if (c0 == kClsInt4 && qh) {
        if (group <= 4)
            score_wave_int4_f16<true>(w, valid, group, qrow0, qh, qexp, qs, out, stride, t);
        else
            score_wave_int4_f16<false>(w, valid, group, qrow0, qh, qexp, qs, out, stride, t);
        return true;
    }
#define SLHA_WAVE(C) score_wave_mfma<C>(w, valid, group, qrow0, qlds, cb, qs, out, stride, t)
    switch (c0) {
        case kClsInt4: SLHA_WAVE(kClsInt4); break;
        case kClsNF4: SLHA_WAVE(kClsNF4); break;
        case kClsTQ3: SLHA_WAVE(kClsTQ3); break;
        case kClsMixed: SLHA_WAVE(kClsMixed); break;
        default: SLHA_WAVE(kClsMix3); break;
    }
#undef SLHA_WAVE
    return true;
}

// Queries of one row staged in LDS for the MFMA A operand.
// Rows group..round_up(group, 4) are zero so the MFMA A operand needs no mask.
__device__ __forceinline__ uint32_t staged_rows(uint32_t group) { return (group + 3u) & ~3u; }

__device__ __forceinline__ void stage_queries(const float* __restrict__ qc, size_t qrow0,
                                              uint32_t group, float* qlds) {
    const uint32_t n = staged_rows(group) * 32u;  // float4s
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const uint32_t q = i >> 5, d4 = i & 31u;
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (q < group) v = reinterpret_cast<const float4*>(qc + (qrow0 + q) * kDC)[d4];
        *reinterpret_cast<float4*>(qlds + q * kQStride + 4 * d4) = v;
    }
}

// Max over the wave of non-negative floats (their IEEE order is their bit
// order): DPP quad, half-row and row mirrors, then row broadcasts 15 and 31
// leave the maximum in lane 63.
__device__ __forceinline__ float wave_max_nonneg(float m) {
    int v = (int)__float_as_uint(m);
    // Full-row patterns read a valid lane everywhere; the broadcasts leave
    // lanes outside their row mask at 0, the identity of this max.
#define SLHA_DPP_MAX(ctrl, rows) \
    v = max(v, __builtin_amdgcn_update_dpp(0, v, ctrl, rows, 0xF, false))
    SLHA_DPP_MAX(0xB1, 0xF);   // quad_perm [1,0,3,2]
    SLHA_DPP_MAX(0x4E, 0xF);   // quad_perm [2,3,0,1]
    SLHA_DPP_MAX(0x141, 0xF);  // row_half_mirror
    SLHA_DPP_MAX(0x140, 0xF);  // row_mirror
    SLHA_DPP_MAX(0x142, 0xA);  // row_bcast:15 into rows 1 and 3
    SLHA_DPP_MAX(0x143, 0xC);  // row_bcast:31 into rows 2 and 3
#undef SLHA_DPP_MAX
    return __uint_as_float((uint32_t)__builtin_amdgcn_readlane(v, 63));
}

// Dims a lane stages for the f16 path: (d, d + 4) with d = 8 (lane/4) + lane%4,
// which sit next to each other in the (d0, d4, d1, d5, d2, d6, d3, d7) order.
__device__ __forceinline__ uint32_t f16_stage_dim(uint32_t lane) {
    return 8u * (lane >> 2) + (lane & 3u);
}

// Two-phase query staging for group <= kRegStageMaxGroup: stage_issue() only
// issues the global loads into registers, so the kernel can issue its tile
// loads right after them; stage_commit() then waits for the (older) query
// loads alone and fills both LDS copies. Together with lds_barrier(), which
// waits for LDS traffic only, the tile loads stay in flight across the
// workgroup barrier.
constexpr uint32_t kRegStageMaxGroup = 16;

// ROWS = staged query rows (4 or 16); the launch allocates staging_bytes(ROWS).
template <uint32_t ROWS>
struct QueryRegs {
    float4 a[ROWS * 32 / 256 > 0 ? ROWS * 32 / 256 : 1];  // f32 copy, float4 (threadIdx.x + 256 k) mod 32*ROWS
    float2 b[ROWS / 4];  // f16 copy: row wave + 4 k, dims (d, d + 4), d = f16_stage_dim(lane)
};

// NATURAL: the f16 copy holds dims (d, d + 1), d = 8 (lane / 4) + 2 (lane % 4),
// i.e. K order (d0, d1, d2, d3 | d4, d5, d6, d7) per latent dword.
template <uint32_t ROWS, bool NATURAL = false>
__device__ __forceinline__ void stage_issue(const float* __restrict__ qc, size_t qrow0,
                                            uint32_t group, QueryRegs<ROWS>& r) {
    // Buffer loads over exactly the row's `group` queries: rows past `group`
    // fall outside the range and read as zero, with no branch or clamp. The
    // whole offset goes in the VGPR operand: the range check of a raw buffer
    // load does not cover the SGPR offset.
    constexpr uint32_t NA = ROWS * 32 / 256 > 0 ? ROWS * 32 / 256 : 1;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t bytes =
        __builtin_amdgcn_readfirstlane((group < ROWS ? group : ROWS) * kDC * 4u);
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(qc + qrow0 * kDC), 0, bytes, 0x00020000);
#pragma unroll
    for (uint32_t k = 0; k < NA; ++k) {
        const uint32_t i = (threadIdx.x + 256u * k) & (ROWS * 32u - 1u);  // float4 index
        r.a[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, 16u * i, 0, 0));
    }
    const uint32_t voff = 4u * (NATURAL ? 8u * (lane >> 2) + 2u * (lane & 3u) : f16_stage_dim(lane));
    constexpr uint32_t second = NATURAL ? 4u : 16u;  // byte offset of the pair's second dim
#pragma unroll
    for (uint32_t k = 0; k < ROWS / 4; ++k) {
        const uint32_t soff = (wv + 4u * k) * kDC * 4u;
        r.b[k] = make_float2(
            __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, soff + voff, 0, 0)),
            __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, soff + voff + second, 0, 0)));
    }
}

// Exponent e of the smallest power of two >= max |q| over the wave's query
// (m = 0 -> e = 0); v0, v1 are this lane's two values.
__device__ __forceinline__ int stage_exponent(float v0, float v1) {
    const float m = wave_max_nonneg(fmaxf(fabsf(v0), fabsf(v1)));
    // m = 2^e' * mant, mant in [0.5, 1); a power of two (mant = 0.5) is its
    // own bound. Zero gives exponent 0 and mantissa 0.
    return __builtin_amdgcn_frexp_exp(m) - (__builtin_amdgcn_frexp_mant(m) == 0.5f ? 1 : 0);
}

// v0 = q_j[d], v1 = q_j[d + 4] with d = f16_stage_dim(lane); one wave per query.
__device__ __forceinline__ void stage_f16_row_e(float v0, float v1, int e, uint32_t j,
                                                uint16_t* qh, float* qexp) {
    const uint32_t lane = threadIdx.x & 63u;
    const float inv = ldexpf(1.0f, -e);
    const float d0 = v0 * inv, d1 = v1 * inv;
    // Truncating f16 split: x - hi is exact in f32 and lo keeps 11 more bits.
    const auto hi = __builtin_amdgcn_cvt_pkrtz(d0, d1);
    const auto lo = __builtin_amdgcn_cvt_pkrtz(d0 - (float)hi.x, d1 - (float)hi.y);
    const uint32_t n = lane & 3u, pword = lane >> 2;
    // Stored from inline asm: the compiler would merge two plain stores into
    // one ds_write2_b32, which loses the information that they do not alias
    // the tile regions the DMA loads fill, and then wait for those loads.
    const uint32_t addr = lds_byte_addr(qh + j * kQStrideH + 16 * pword + 2 * n);
    asm volatile("ds_write_b32 %0, %1\n\tds_write_b32 %0, %2 offset:16" ::"v"(addr),
                 "v"(__builtin_bit_cast(uint32_t, hi)), "v"(__builtin_bit_cast(uint32_t, lo))
                 : "memory");
    if (lane == 0) qexp[j] = ldexpf(1.0f, e);
}

__device__ __forceinline__ void stage_f16_row(float v0, float v1, uint32_t j, uint16_t* qh,
                                              float* qexp) {
    stage_f16_row_e(v0, v1, stage_exponent(v0, v1), j, qh, qexp);
}

__device__ __forceinline__ void stage_queries_f16(const float* __restrict__ qc, size_t qrow0,
                                                  uint32_t group, uint16_t* qh, float* qexp) {
    const uint32_t lane = threadIdx.x & 63u, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const uint32_t rows = (group + 3u) & ~3u;
    for (uint32_t j = wv; j < rows; j += nw) {
        float v0 = 0.0f, v1 = 0.0f;
        if (j < group) {
            const float* q = qc + (qrow0 + j) * kDC + f16_stage_dim(lane);
            v0 = q[0];
            v1 = q[4];
        }
        stage_f16_row(v0, v1, j, qh, qexp);
    }
}

// Writes all ROWS staged rows (rows past `group` were read as zero; threads
// past 32*ROWS float4s rewrite identical values), with no branch.
template <uint32_t ROWS>
__device__ __forceinline__ void stage_commit(const QueryRegs<ROWS>& r, uint32_t group,
                                             const StagedQueries& sq) {
    constexpr uint32_t NA = ROWS * 32 / 256 > 0 ? ROWS * 32 / 256 : 1;
    const uint32_t wv = threadIdx.x >> 6;
#pragma unroll
    for (uint32_t k = 0; k < NA; ++k) {
        const uint32_t i = (threadIdx.x + 256u * k) & (ROWS * 32u - 1u), q = i >> 5;
        *reinterpret_cast<float4*>(sq.q32 + q * kQStride + 4 * (i & 31u)) = r.a[k];
    }
#pragma unroll
    for (uint32_t k = 0; k < ROWS / 4; ++k)
        stage_f16_row(r.b[k].x, r.b[k].y, wv + 4u * k, sq.q16, sq.qexp);
}

__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// NF4 codebook (constants.rs:138-141) staged in LDS.
__device__ __forceinline__ void stage_codebook(float* cb) {
    if (threadIdx.x < 16) cb[threadIdx.x] = nf4_level(threadIdx.x);
}
// The same by the first 16 lanes of the calling wave.
__device__ __forceinline__ void stage_codebook_wave(float* cb) {
    const uint32_t lane = threadIdx.x & 63u;
    if (lane < 16) cb[lane] = nf4_level(lane);
}

template <bool EXACT, bool HAM>
__device__ __forceinline__ void score_dispatch(const uint32_t* w, uint32_t group, size_t qrow0,
                                               const float* __restrict__ qc,
                                               const uint32_t* __restrict__ qs, const float* cb,
                                               float* __restrict__ out, uint32_t* __restrict__ ham,
                                               size_t stride, uint32_t t) {
    const int cls = codec_class(w[29] >> 16);
#define SLHA_LANE(C) score_lane<C, EXACT, HAM>(w, group, qrow0, qc, qs, cb, out, ham, stride, t)
    if (cls == kClsInt4) SLHA_LANE(kClsInt4);
    if (cls == kClsNF4) SLHA_LANE(kClsNF4);
    if (cls == kClsTQ3) SLHA_LANE(kClsTQ3);
    if (cls == kClsMixed) SLHA_LANE(kClsMixed);
    if (cls == kClsMix3) SLHA_LANE(kClsMix3);
#undef SLHA_LANE
}


// Per-lane scoring of tile rows: EXACT mode, Hamming output, or groups too
// large for the staged MFMA path.
template <bool EXACT, bool HAM>
__global__ __launch_bounds__(256) void score_rows_kernel(
    const uint4* __restrict__ tiles, uint32_t n_tok, uint32_t group,
    const float* __restrict__ qc, const uint32_t* __restrict__ qs,
    float* __restrict__ scores, uint32_t* __restrict__ ham) {
    __shared__ float cb[16];
    const uint32_t row = blockIdx.y;
    const size_t qrow0 = (size_t)row * group;
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    const bool valid = t < n_tok;
    uint32_t w[32];
    if (valid) load_tile(tiles + ((size_t)row * n_tok + t) * 8, w);
    stage_codebook(cb);
    __syncthreads();
    if (!valid) return;
    score_dispatch<EXACT, HAM>(w, group, qrow0, qc, qs, cb, scores + qrow0 * n_tok,
                               HAM ? ham + qrow0 * n_tok : nullptr, n_tok, t);
}

// ---------------------------------------------------------------------------
// INT4 on the integer matrix cores, pipelined with the tile DMA (group <= 4).
//
// v_mfma_i32_16x16x64_i8: lane L supplies A row / B column L % 16 for the 16
// K slots 16 (L / 16) .. +15 and receives C[4 (L / 16) + r][L % 16], r < 4.
//  * Columns are 16 tiles (a "block"; a wave's 64 tiles are 4 blocks).
//  * Rows are (query j, limb l) = 4 j + l: each query, prescaled by 2^-e
//    (|q 2^-e| <= 1) and rounded to q30 = q 2^(30 - e), is split into four
//    signed bytes l0 + 2^8 l1 + 2^16 l2 + 2^24 l3. So lane L's accumulators
//    are the four limb sums of query L / 16 for its tile.
//  * B is the nibble n itself (0..15): latent dword x gives the bytes
//    x & 0x0F0F0F0F (dims 0, 2, 4, 6) and (x >> 4) & 0x0F0F0F0F (dims 1, 3,
//    5, 7); the staged query bytes use the same K order. K-block kb covers
//    dims 64 kb .. +63, lane group h the latent dwords 8 kb + 2 h, +1.
//  * The -8 of n - 8 is exact in integers: the accumulator starts at
//    -sum_d 8 limb(q_d), one tile-independent product with B = 8 per wave.
// The limb sums are exact; q is carried to 2^-31 of max |q| (about f32's
// own rounding). The tile scale applies once per (tile, query); the path serves
// INT4 tiles whose 8 group scales are equal (every codec-0 tile; eff =
// scale * gs / 255), other blocks send the wave to the per-codec MFMA paths.
//
// The wave's tiles are dealt into four blocks (block k holds tiles 4c + k,
// fetch_tiles_lds_dealt), so after the last block a lane holds four
// consecutive tokens and stores them as one 16-byte write.
// Each block's two 1 KiB DMA loads land in its own 2 KiB of the wave's region;
// the block is scored as soon as they are in (s_waitcnt vmcnt(2 (3 - cb)):
// loads complete in issue order, so this counts only the later tile loads),
// while the later blocks are still in flight. The reads of the region are
// inline asm, invisible to the compiler's LDS-DMA tracking, which would
// otherwise wait for every tile load before the first read. Scores are stored
// after the last block: a store before a partial vmcnt wait would make the
// wait cover it too.

typedef int v4i __attribute__((ext_vector_type(4)));

struct I8Staging {
    uint4 a8[2][4][16];  // A operand [kb][lane group][row]
    uint32_t qsw[4][8];  // the 4 queries' sign words
    float qf[4];         // 2^(e - 30) / 255, NaN for a non-finite query
};

// Tile c of a block: the dwords lane group h reads.
struct I8BlockWords {
    uint2 x0, x1;  // latent dwords (2h, 2h+1) and (8+2h, 9+2h)
    uint4 r0, r1;  // residual words 0..7
    uint2 m6;      // scale, lambda
    uint4 m7;      // position, head | flags << 16, gs[0..7]
};

// LDS byte addresses of tile c's words in block 0 of a wave region filled by
// fetch_tiles_lds (block cb sits 2048 cb bytes further).
struct I8BlockAddr {
    uint32_t x0, x1, r0, r1, m6, m7;
};

__device__ __forceinline__ I8BlockAddr i8_block_addr(const uint4* region, uint32_t c, uint32_t h) {
    const uint32_t base = lds_byte_addr(region) + 128u * c, sx = c & 7u;  // local tile c, swizzled by c & 7
    I8BlockAddr a;
    a.x0 = base + 16u * ((h >> 1) ^ sx) + 8u * (h & 1u);
    a.x1 = base + 16u * ((2u + (h >> 1)) ^ sx) + 8u * (h & 1u);
    a.r0 = base + 16u * (4u ^ sx);
    a.r1 = base + 16u * (5u ^ sx);
    a.m6 = base + 16u * (6u ^ sx);
    a.m7 = base + 16u * (7u ^ sx);
    return a;
}

// Waits until at most VMCNT tile loads are outstanding, then reads block OFF/2048.
template <int VMCNT, int OFF>
__device__ __forceinline__ I8BlockWords i8_read_block(const I8BlockAddr& a) {
    I8BlockWords b;
    asm volatile(
        "s_waitcnt vmcnt(%12)\n\t"
        "ds_read_b64 %0, %6 offset:%13\n\t"
        "ds_read_b64 %1, %7 offset:%13\n\t"
        "ds_read_b128 %2, %8 offset:%13\n\t"
        "ds_read_b128 %3, %9 offset:%13\n\t"
        "ds_read_b64 %4, %10 offset:%13\n\t"
        "ds_read_b128 %5, %11 offset:%13\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(b.x0), "=&v"(b.x1), "=&v"(b.r0), "=&v"(b.r1), "=&v"(b.m6), "=&v"(b.m7)
        : "v"(a.x0), "v"(a.x1), "v"(a.r0), "v"(a.r1), "v"(a.m6), "v"(a.m7), "n"(VMCNT), "n"(OFF)
        : "memory");
    return b;
}

// The block takes the integer path: INT4 (no codec flag) with equal group scales.
__device__ __forceinline__ bool i8_block_ok(const I8BlockWords& b) {
    const uint32_t g = b.m7.z;  // all 8 bytes equal: the word equals its byte rotation and m7.w
    return ((b.m7.y >> 16) & kCodecFlags) == 0u && b.m7.w == g &&
           __builtin_amdgcn_alignbit(g, g, 8) == g;
}

struct I8Query {
    v4i a0, a1, neg;  // A per K-block; -8 sum limb(q) per limb row
    uint32_t qw[8];   // sign words of query h
    float qf;
};

__device__ __forceinline__ I8Query i8_load_query(const I8Staging& st, uint32_t c, uint32_t h) {
    I8Query q;
    q.a0 = __builtin_bit_cast(v4i, st.a8[0][h][c]);
    q.a1 = __builtin_bit_cast(v4i, st.a8[1][h][c]);
    const v4i b8 = v4i{0x08080808, 0x08080808, 0x08080808, 0x08080808};
    v4i off = __builtin_amdgcn_mfma_i32_16x16x64_i8(q.a0, b8, v4i{0, 0, 0, 0}, 0, 0, 0);
    off = __builtin_amdgcn_mfma_i32_16x16x64_i8(q.a1, b8, off, 0, 0, 0);
    q.neg = -off;
    const uint4 x = *reinterpret_cast<const uint4*>(&st.qsw[h][0]);
    const uint4 y = *reinterpret_cast<const uint4*>(&st.qsw[h][4]);
    q.qw[0] = x.x, q.qw[1] = x.y, q.qw[2] = x.z, q.qw[3] = x.w;
    q.qw[4] = y.x, q.qw[5] = y.y, q.qw[6] = y.z, q.qw[7] = y.w;
    q.qf = st.qf[h];
    return q;
}

// Score of (query h, tile c of the block).
__device__ __forceinline__ float i8_score_block(const I8BlockWords& b, const I8Query& q) {
    constexpr uint32_t M = 0x0F0F0F0Fu;
    const v4i b0 = v4i{(int)(b.x0.x & M), (int)((b.x0.x >> 4) & M), (int)(b.x0.y & M), (int)((b.x0.y >> 4) & M)};
    const v4i b1 = v4i{(int)(b.x1.x & M), (int)((b.x1.x >> 4) & M), (int)(b.x1.y & M), (int)((b.x1.y >> 4) & M)};
    v4i acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(q.a0, b0, q.neg, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(q.a1, b1, acc, 0, 0, 0);
    const uint32_t ham = __popc(b.r0.x ^ q.qw[0]) + __popc(b.r0.y ^ q.qw[1]) + __popc(b.r0.z ^ q.qw[2]) +
                         __popc(b.r0.w ^ q.qw[3]) + __popc(b.r1.x ^ q.qw[4]) + __popc(b.r1.y ^ q.qw[5]) +
                         __popc(b.r1.z ^ q.qw[6]) + __popc(b.r1.w ^ q.qw[7]);
    // sum q30 (n - 8) = (acc3 2^8 + acc2) 2^16 + (acc1 2^8 + acc0), both
    // brackets exact in int32 (|acc| <= 2^17); one rounding each to f32
    const float dot = fmaf((float)((acc[3] << 8) + acc[2]), 65536.0f, (float)((acc[1] << 8) + acc[0]));
    const float eff = __uint_as_float(b.m6.x) * (float)(b.m7.z & 0xFFu);
    const float sc = dot * (eff * q.qf);
    // the residual term always, then a select: no branch around it
    const float with_res = fmaf(__uint_as_float(b.m6.y), 256.0f - 2.0f * (float)ham, sc);
    return ((b.m7.y >> 16) & kFlagWarm) == 0u ? with_res : sc;
}

// Query staging of the integer path, on top of stage_issue<4> /
// stage_commit<4>: each wave also loads its query's 8 sign words (lanes 0..7;
// rows past `group` read as zero) and writes its query's limb bytes, 2^(e-22)
// and sign words to the I8Staging (inline asm stores, as in stage_f16_row).
__device__ __forceinline__ uint32_t stage_issue_signs(const uint32_t* __restrict__ qs, size_t qrow0,
                                                      uint32_t group) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(qs + qrow0 * 8), 0,
        __builtin_amdgcn_readfirstlane((group < 4u ? group : 4u) * 32u), 0x00020000);
    return __builtin_amdgcn_raw_buffer_load_b32(rs, wv * 32u + 4u * (lane & 7u), 0, 0);
}

// Bytes l0 | l1 << 8 | l2 << 16 | l3 << 24 of q30 = l0 + 2^8 l1 + 2^16 l2 +
// 2^24 l3: l0, l1, l2 are the sign-extended low bytes of q30, q1 =
// (q30 - l0) / 2^8 and q2 = (q1 - l1) / 2^8 (each division exact), so they lie
// in [-128, 127]; |q30| <= 2^30 gives |q2| <= 2^14 + 1 and l3 = (q2 - l2) /
// 2^8 in [-64, 64].
__device__ __forceinline__ uint32_t q30_limbs(int32_t q) {
    const int32_t q1 = (q - (int32_t)(int8_t)(q & 0xFF)) >> 8;
    const int32_t q2 = (q1 - (int32_t)(int8_t)(q1 & 0xFF)) >> 8;
    const int32_t l3 = (q2 - (int32_t)(int8_t)(q2 & 0xFF)) >> 8;
    return ((uint32_t)q & 0xFFu) | (((uint32_t)q1 & 0xFFu) << 8) | (((uint32_t)q2 & 0xFFu) << 16) |
           ((uint32_t)l3 << 24);
}

// Wave j's query: v0 = q_j[d], v1 = q_j[d + 4], d = f16_stage_dim(lane) =
// 8 p + o (latent dword p = lane / 4, o = lane % 4); sw = sign word lane (< 8).
__device__ __forceinline__ void stage_i8_row(float v0, float v1, uint32_t sw, uint32_t j,
                                             I8Staging& st) {
    const uint32_t lane = threadIdx.x & 63u;
    // max |q| over the wave as an integer max of the bit patterns, in which
    // NaN sorts above +inf above every finite value; e as in stage_exponent
    const float m = wave_max_nonneg(__uint_as_float(
        max(__float_as_uint(fabsf(v0)), __float_as_uint(fabsf(v1)))));
    const int e = __builtin_amdgcn_frexp_exp(m) - (__builtin_amdgcn_frexp_mant(m) == 0.5f ? 1 : 0);
    const uint32_t b0 = q30_limbs((int32_t)rintf(ldexpf(v0, 30 - e)));
    const uint32_t b1 = q30_limbs((int32_t)rintf(ldexpf(v1, 30 - e)));
    // K slot of dim 8 p + o inside lane group h = (p & 7) / 2 of K-block p / 8:
    // 8 (p & 1) + 4 (o & 1) + o / 2; dim d + 4 sits two slots further.
    const uint32_t p = lane >> 2, o = lane & 3u;
    const uint32_t addr = lds_byte_addr(&st.a8[p >> 3][(p & 7u) >> 1][4u * j]) +
                          8u * (p & 1u) + 4u * (o & 1u) + (o >> 1);
    asm volatile(
        "ds_write_b8 %0, %1\n\tds_write_b8 %0, %2 offset:2\n\t"
        "ds_write_b8 %0, %3 offset:16\n\tds_write_b8 %0, %4 offset:18\n\t"
        "ds_write_b8_d16_hi %0, %1 offset:32\n\tds_write_b8_d16_hi %0, %2 offset:34\n\t"
        "ds_write_b8 %0, %5 offset:48\n\tds_write_b8 %0, %6 offset:50"
        ::"v"(addr), "v"(b0), "v"(b1), "v"(b0 >> 8), "v"(b1 >> 8), "v"(b0 >> 24), "v"(b1 >> 24)
        : "memory");
    // A non-finite query value makes every score of the query NaN (the f16
    // path propagates it through its products; here the limbs would not).
    const float qf = m <= 3.402823466e38f ? ldexpf(1.0f, e - 30) * (1.0f / 255.0f) : __builtin_nanf("");
    // every lane writes (lanes l and l + 8 hold the same sign word): no branch
    asm volatile("ds_write_b32 %0, %1\n\tds_write_b32 %2, %3" ::"v"(lds_byte_addr(&st.qf[j])),
                 "v"(qf), "v"(lds_byte_addr(&st.qsw[j][lane & 7u])), "v"(sw)
                 : "memory");
}

// Fast scoring of tile rows on the matrix cores (group <= kMfmaMaxGroup).
// Each wave fetches its 64 tiles with coalesced loads (fetch_tiles_*). With
// REG_STAGE (group <= kRegStageMaxGroup) the query loads are issued first and
// the tile loads stay in flight across the workgroup barrier.
template <uint32_t REG_ROWS>
__global__ __launch_bounds__(256) void score_rows_fast_kernel(
    const uint4* __restrict__ tiles, uint32_t n_tok, uint32_t group,
    const float* __restrict__ qc, const uint32_t* __restrict__ qs, float* __restrict__ scores) {
    __shared__ float cb[16];
    __shared__ uint4 tile_lds[4][512];  // one 8 KiB region per wave
    // REG_ROWS > 0: staging in a static array, so the compiler can tell that
    // the staging stores do not touch the tile regions the DMA loads write
    // and does not wait for those loads before them. Otherwise dynamic LDS
    // of staging_bytes(staging_rows(group)).
    __shared__ __attribute__((aligned(16))) float qstatic[REG_ROWS ? staging_bytes(REG_ROWS) / 4 : 1];
    extern __shared__ __attribute__((aligned(16))) float qlds[];
    const uint32_t row = blockIdx.y;
    const size_t qrow0 = (size_t)row * group;
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    const StagedQueries sq =
        carve_staging(REG_ROWS ? qstatic : qlds, REG_ROWS ? REG_ROWS : staging_rows(group));
    QueryRegs<REG_ROWS ? REG_ROWS : 4> qr;
    if constexpr (REG_ROWS > 0) stage_issue<REG_ROWS>(qc, qrow0, group, qr);
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t wave0 = blockIdx.x * blockDim.x + 64u * wave;
    const uint32_t n_valid = wave0 < n_tok ? n_tok - wave0 : 0u;
    fetch_tiles_lds(tiles + ((size_t)row * n_tok + wave0) * 8, n_valid, tile_lds[wave]);
    stage_codebook(cb);
    if constexpr (REG_ROWS > 0) {
        stage_commit<REG_ROWS>(qr, group, sq);
        lds_barrier();
    } else {
        stage_queries(qc, qrow0, group, sq.q32);
        stage_queries_f16(qc, qrow0, group, sq.q16, sq.qexp);
        __syncthreads();
    }
    uint32_t w[32];
    fetch_tiles_readback(tile_lds[wave], w);
    const bool valid = t < n_tok;
    float* out = scores + qrow0 * n_tok;
    if (score_wave_try_mfma(w, valid, group, qrow0, sq.q32, cb, sq.q16, sq.qexp, qs, out, n_tok, t))
        return;
    if (valid) score_dispatch<false, false>(w, group, qrow0, qc, qs, cb, out, nullptr, n_tok, t);
}

// NF4 fast path for group <= 4 (the launch takes it when the caller's
// codec hint is NF4) on v_mfma_f32_4x4x4_16b_f16: lane = tile, 4 queries,
// each 16-dim group accumulated on its own and added in with its scale gs.
// Per latent byte (dims d0 = 2i, d1 = 2i + 1, nibbles n0, n1), one MFMA
// K-step of four slots:
//  * B is a 256-entry LDS table indexed by the byte: the f16 hi halves of the
//    two nibbles' NF4 levels (constants.rs:138-141), then their lo halves
//    (hi + lo = level to ~2^-22). One 8-byte read is one B operand.
//  * A is (q_hi[d0], q_hi[d1], q_hi[d0], q_hi[d1]): q_hi (L_hi + L_lo) over
//    the pair.
// and per pair of bytes one more K-step for q_lo, the query's low f16 half:
// A = q_lo of the four dims, B = the two entries' hi halves, so q_lo L_hi.
// The q_lo L_lo term left out is below 2^-22 of each product. All 16 blocks
// multiply the same 4 queries, so every MFMA broadcasts one block's A
// operand to all (CBSZ 4): the 96 A operands (64 bytes' q_hi, then 32 byte
// pairs' q_lo) live as 6 register pairs spread over the lane blocks,
// operand o in pair o / 16 of block o % 16 (ABID), read once per wave.
// Table entries are used as they are read: no VALU builds an operand.
constexpr uint32_t kNF4QStride = 96u * 8u + 16u;  // bytes per staged query
constexpr int kNF4LoOperand = 64;                 // first q_lo operand

template <int O>
__device__ __forceinline__ v4f nf4_mfma(const uint2 (&a)[6], v4h b, v4f acc) {
    return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(v4h, a[O >> 4]), b, acc, 4, O & 15, 0);
}

// Group G (latent bytes 8G .. 8G + 7, dims 16G .. 16G + 15) accumulated on
// its own, added in with gs.
template <int G>
__device__ __forceinline__ void nf4_group(const uint32_t* w, const uint2* lut, const uint2 (&a)[6],
                                          v4f& dot) {
    v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    uint2 e[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) e[j] = lut[(w[2 * G + (j >> 2)] >> (8 * (j & 3))) & 0xFFu];
    // bytes 8G + 2P, 8G + 2P + 1: q_hi operands 8G + 2P, 8G + 2P + 1, then
    // q_lo operand 64 + 4G + P
#define SLHA_NF4_PAIR(P)                                                                   \
    acc = nf4_mfma<8 * G + 2 * (P)>(a, __builtin_bit_cast(v4h, e[2 * (P)]), acc);          \
    acc = nf4_mfma<8 * G + 2 * (P) + 1>(a, __builtin_bit_cast(v4h, e[2 * (P) + 1]), acc);  \
    acc = nf4_mfma<kNF4LoOperand + 4 * G + (P)>(                                           \
        a, __builtin_bit_cast(v4h, make_uint2(e[2 * (P)].x, e[2 * (P) + 1].x)), acc);
    SLHA_NF4_PAIR(0) SLHA_NF4_PAIR(1) SLHA_NF4_PAIR(2) SLHA_NF4_PAIR(3)
#undef SLHA_NF4_PAIR
    const float gsf = gs_at(w + 30, G);
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) dot[rr] = fmaf(acc[rr], gsf, dot[rr]);
}

template <int... G>
__device__ __forceinline__ void nf4_groups(const uint32_t* w, const uint2* lut, const uint2 (&a)[6],
                                           v4f& dot, std::integer_sequence<int, G...>) {
    (nf4_group<G>(w, lut, a, dot), ...);
}

// qdup: per query kNF4QStride bytes, A operand o at byte 8 o.
__device__ __forceinline__ void score_wave_nf4_f16(const uint32_t* w, bool valid, uint32_t group,
                                                   size_t qrow0, const char* qdup,
                                                   const float* qexp, const uint2* lut,
                                                   const uint32_t* __restrict__ qs,
                                                   float* __restrict__ out, size_t stride,
                                                   uint32_t t) {
    const uint32_t lane = threadIdx.x & 63u;
    // lane 4b + r: operands 16k + b of query r, k = 0..5
    const uint2* qa = reinterpret_cast<const uint2*>(qdup + (lane & 3u) * kNF4QStride) + (lane >> 2);
    uint2 a[6];
#pragma unroll
    for (int k = 0; k < 6; ++k) a[k] = qa[16 * k];
    v4f dot = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    nf4_groups(w, lut, a, dot, std::make_integer_sequence<int, 8>{});
    const float s255 = __uint_as_float(w[24]) * (1.0f / 255.0f);
    const float lambda = __uint_as_float(w[25]);
    const bool warm = ((w[29] >> 16) & kFlagWarm) != 0;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
        if ((uint32_t)rr < group) {
            float sc = dot[rr] * (s255 * qexp[rr]);
            const uint32_t h = hamming_words(w + 16, qs + (qrow0 + rr) * 8);
            if (!warm) sc = fmaf(lambda, 256.0f - 2.0f * (float)h, sc);
            if (valid) store_out(out + (size_t)rr * stride + t, sc);
        }
    }
}

// f16 hi/lo bits of an NF4 level: hi | lo << 16.
__device__ __forceinline__ uint32_t nf4_level_pair(float l) {
    const _Float16 hi = (_Float16)l;
    const _Float16 lo = (_Float16)(l - (float)hi);
    return (uint32_t)__builtin_bit_cast(uint16_t, hi) | ((uint32_t)__builtin_bit_cast(uint16_t, lo) << 16);
}

// Scoring of rows of NF4 tiles, group <= 4: the tile fetch of
// score_rows_fast_kernel, the queries staged for score_wave_nf4_f16 (wave j
// stages query j, lane l converts dims 2l, 2l + 1 into q_hi operand l and
// half of q_lo operand 64 + l / 2; rows past `group` are zero), and
// score_wave_nf4_f16 for NF4 waves. Other waves take the per-lane path.
__global__ __launch_bounds__(256) void score_rows_nf4_kernel(
    const uint4* __restrict__ tiles, uint32_t n_tok, uint32_t group,
    const float* __restrict__ qc, const uint32_t* __restrict__ qs, float* __restrict__ scores) {
    __shared__ float cb[16];
    __shared__ uint2 lut[256];
    __shared__ uint4 tile_lds[4][512];
    __shared__ __attribute__((aligned(16))) char qdup[4 * kNF4QStride];
    __shared__ float qexp[4];
    const uint32_t row = blockIdx.y;
    const size_t qrow0 = (size_t)row * group;
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // query `wave`, dims (2 lane, 2 lane + 1), read as zero past `group`
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(qc + qrow0 * kDC), 0, __builtin_amdgcn_readfirstlane(group * kDC * 4u),
        0x00020000);
    const uint2 qv = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                                   rq, wave * kDC * 4u + 8u * lane, 0, 0));
    const uint32_t wave0 = blockIdx.x * blockDim.x + 64u * wave;
    const uint32_t n_valid = wave0 < n_tok ? n_tok - wave0 : 0u;
    fetch_tiles_lds(tiles + ((size_t)row * n_tok + wave0) * 8, n_valid, tile_lds[wave]);
    {
        // byte b = n0 | n1 << 4: (hi(n0), hi(n1), lo(n0), lo(n1)). One level
        // a lane (the select tree runs as branches under a divergent index):
        // lane l holds level l & 15, and the level n1 = b >> 4 comes from
        // lane n1 of the same wave.
        const float lv = nf4_level(lane & 15u);
        const uint32_t p0 = nf4_level_pair(lv);
        const uint32_t p1 = (uint32_t)__shfl((int)p0, (int)(threadIdx.x >> 4));
        lut[threadIdx.x] = make_uint2((p0 & 0xFFFFu) | (p1 << 16), (p0 >> 16) | (p1 & 0xFFFF0000u));
        if (threadIdx.x < 16) cb[threadIdx.x] = lv;
    }
    {
        const float v0 = __uint_as_float(qv.x), v1 = __uint_as_float(qv.y);
        const int e = stage_exponent(v0, v1);
        const float inv = ldexpf(1.0f, -e);
        const float d0 = v0 * inv, d1 = v1 * inv;
        // Truncating f16 split: x - hi is exact in f32 and lo keeps 11 more bits.
        const auto hi = __builtin_amdgcn_cvt_pkrtz(d0, d1);
        const auto lo = __builtin_amdgcn_cvt_pkrtz(d0 - (float)hi.x, d1 - (float)hi.y);
        const uint32_t h2 = __builtin_bit_cast(uint32_t, hi), l2 = __builtin_bit_cast(uint32_t, lo);
        // q_hi operand `lane` (byte 8 lane) and half of q_lo operand
        // 64 + lane / 2 (byte 512 + 4 lane); stored from inline asm, as in
        // stage_f16_row: no wait for the tile DMA
        typedef uint32_t v2u __attribute__((ext_vector_type(2)));
        const uint32_t qa = lds_byte_addr(qdup + wave * kNF4QStride);
        asm volatile("ds_write_b64 %0, %1\n\tds_write_b32 %2, %3" ::"v"(qa + 8u * lane), "v"(v2u{h2, h2}),
                     "v"(qa + 8u * kNF4LoOperand + 4u * lane), "v"(l2)
                     : "memory");
        if (lane == 0) qexp[wave] = ldexpf(1.0f, e);
    }
    lds_barrier();
    uint32_t w[32];
    fetch_tiles_readback(tile_lds[wave], w);
    const bool valid = t < n_tok;
    float* out = scores + qrow0 * n_tok;
    const int cls = valid ? codec_class(w[29] >> 16) : -1;
    if (__all(cls == kClsNF4 || cls < 0) && __builtin_amdgcn_readfirstlane(cls) == kClsNF4) {
        score_wave_nf4_f16(w, valid, group, qrow0, qdup, qexp, lut, qs, out, n_tok, t);
        return;
    }
    if (valid) score_dispatch<false, false>(w, group, qrow0, qc, qs, cb, out, nullptr, n_tok, t);
}

// Scoring of rows of INT4 tiles, group <= 4, on the pipelined integer path
// (the launch takes it when the caller's codec hint is INT4). A wave whose
// block holds another codec, or group scales that differ, scores its 64
// tiles on the per-lane path instead: same results, slower. Registers stay
// within 128 (four waves per SIMD), which a kernel that also carried the
// per-codec MFMA paths could not do.
__global__ __launch_bounds__(256, 4) void score_rows_int4_kernel(
    const uint4* __restrict__ tiles, uint32_t n_tok, uint32_t group,
    const float* __restrict__ qc, const uint32_t* __restrict__ qs, float* __restrict__ scores) {
    __shared__ float cb[16];
    __shared__ uint4 tile_lds[4][512];  // one 8 KiB region per wave
    __shared__ I8Staging st;
    const uint32_t row = blockIdx.y;
    const size_t qrow0 = (size_t)row * group;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // wave w stages query w: its dims (d, d + 4), d = f16_stage_dim(lane), and
    // its sign words; buffer ranges end at the row's `group` queries
    float v0, v1;
    {
        const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(qc + qrow0 * kDC), 0,
            __builtin_amdgcn_readfirstlane(group * kDC * 4u), 0x00020000);
        const uint32_t voff = 4u * f16_stage_dim(lane), soff = wave * kDC * 4u;
        v0 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rq, soff + voff, 0, 0));
        v1 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rq, soff + voff + 16u, 0, 0));
    }
    const uint32_t sw = stage_issue_signs(qs, qrow0, group);
    const uint32_t wave0 = blockIdx.x * blockDim.x + 64u * wave;
    const uint32_t n_valid = wave0 < n_tok ? n_tok - wave0 : 0u;
    fetch_tiles_lds_dealt(tiles + ((size_t)row * n_tok + wave0) * 8, n_valid, tile_lds[wave]);
    // keep the staging arithmetic after the tile loads are issued
    __builtin_amdgcn_sched_barrier(0);
    stage_i8_row(v0, v1, sw, wave, st);
    lds_barrier();
    const uint32_t c = lane & 15u, h = lane >> 4;
    const I8Query q = i8_load_query(st, c, h);
    const I8BlockAddr a = i8_block_addr(tile_lds[wave], c, h);
    // This lane's outputs: query h, tokens wave0 + 4c .. +3 (block k holds
    // token 4c + k), computed while the tiles are in flight.
    const size_t o = (qrow0 + h) * n_tok + wave0 + 4u * c;
    // wave-uniform: every lane stores all four, 16-byte aligned
    const bool whole = group == 4u && wave0 + 64u <= n_tok && (n_tok & 3u) == 0u &&
                       (reinterpret_cast<uintptr_t>(scores) & 15u) == 0u;
    // Every block is scored as it lands; whether the wave's tiles all fit the
    // integer path is decided once, after the last block (a block that does
    // not fit only yields values that are then discarded). The empty asm pins
    // each block's score where it is computed: sunk to the stores, four
    // blocks' accumulators would be live at once.
    float res[4];
    bool ok;
    {
        const I8BlockWords b = i8_read_block<6, 0>(a);
        ok = i8_block_ok(b);
        res[0] = i8_score_block(b, q);
        asm volatile("" : "+v"(res[0]));
    }
    {
        const I8BlockWords b = i8_read_block<4, 2048>(a);
        ok = ok & i8_block_ok(b);
        res[1] = i8_score_block(b, q);
        asm volatile("" : "+v"(res[1]));
    }
    {
        const I8BlockWords b = i8_read_block<2, 4096>(a);
        ok = ok & i8_block_ok(b);
        res[2] = i8_score_block(b, q);
        asm volatile("" : "+v"(res[2]));
    }
    {
        const I8BlockWords b = i8_read_block<0, 6144>(a);
        ok = ok & i8_block_ok(b);
        res[3] = i8_score_block(b, q);
    }
    if (__all(ok)) {
        if (whole) {  // 16 lanes x 16 B: 256 contiguous bytes per query
            typedef float v4f_nt __attribute__((ext_vector_type(4)));
            __builtin_nontemporal_store(v4f_nt{res[0], res[1], res[2], res[3]},
                                        reinterpret_cast<v4f_nt*>(scores + o));
        } else {
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k)
                if (h < group && wave0 + 4u * c + k < n_tok) store_out(scores + o + k, res[k]);
        }
        return;
    }
    // Per-lane path; nothing was stored above. The compiler waits for the
    // tile loads before this read-back. The wave stages the NF4 codebook for
    // itself (waves that reach here write identical values; no barrier).
    stage_codebook_wave(cb);
    uint32_t w[32];
    fetch_tiles_readback_dealt(tile_lds[wave], w);
    const uint32_t t = wave0 + lane;
    if (t < n_tok)
        score_dispatch<false, false>(w, group, qrow0, qc, qs, cb, scores + qrow0 * n_tok, nullptr,
                                     n_tok, t);
}

// Wide-group scoring (16 < group <= 64 queries per tile, e.g. 64) on the
// 32x32 matrix-core shapes: v_mfma_f32_32x32x16_f16 for the codes and
// v_mfma_i32_32x32x32_i8 for the residual term. Rows (A) are queries,
// columns (B) are tiles: lane L holds, for its tile L % 32, the scores of
// queries 8 (i / 4) + 4 (L / 32) + i % 4 in accumulator i, so one register
// store writes two queries' scores for 32 consecutive tiles (whole 128-byte
// lines).
//
// K order, the same on both operands: at f16 K-step ks (16 dims) lane group
// g = L / 32 supplies K slots 8 g .. 8 g + 7, which are dims
// 64 g + 8 ks + (s >> 1) + 4 (s & 1), s = 0..7. B's dword k then holds dims
// (k, k + 4) of an 8-dim window as f16 (lo, hi), which both codecs' bit
// layouts give with one shift and one masked OR per dword; the f16 value is
// a magic-number float (exponent bits OR'd over the field) minus its base.
// Each level enters B exactly:
//  * INT4: (n - 8) * gs, |.| <= 2040, exact in f16.
//  * TQ3: L = 4 code + 2 corr - 15 (NOCORR: 4 code - 14), and L * gs
//    (|.| <= 3825) is split into B_main = f16(L * gs) and its exact rounding
//    error B_err = L * gs - B_main (-1, 0 or 1). The sum is B_main * q_hi +
//    B_main * q_lo + B_err * q_hi; the dropped B_err * q_lo is below 2^-22 of
//    the product.
// Queries enter as f16 hi + lo of q * 2^-e (e: the query's power-of-two
// normalisation, undone in the epilogue), exact to ~2^-22 per element.
// The residual term takes +-1 bytes of both sign sketches on the i8 MFMA:
// their dot product is 256 - 2 * Hamming, exactly.
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef int v16i __attribute__((ext_vector_type(16)));

// +-1 bytes of 8 sign bits: byte j = 1 - 2 * bit j (0x01 or 0xFF).
__device__ __forceinline__ uint2 pm1_bytes(uint32_t b) {
    auto spread = [](uint32_t n) {  // bit j of a nibble to bit 0 of byte j
        return ((n * 0x00204081u) & 0x01010101u) * 0xFEu | 0x01010101u;
    };
    return make_uint2(spread(b & 15u), spread((b >> 4) & 15u));
}

// The wide query image of one row: wide_nq(group) query rows (rows at or
// past `group` are zero), laid out so that every LDS read of the scoring
// kernel is 16 bytes per lane at consecutive addresses:
//   H [ks 0..7][part: 0 hi, 1 lo][g 0..1][q]: 8 f16, the K slots above
//   P [kc 0..7][g][q]: 16 bytes 1 - 2 bit for sign bits 128 g + 16 kc + j
//   E [q]: 2^e
__host__ __device__ constexpr uint32_t wide_nq(uint32_t group) { return group <= 32u ? 32u : 64u; }
__host__ __device__ constexpr uint32_t wide_off_p(uint32_t nq) { return 512u * nq; }
__host__ __device__ constexpr uint32_t wide_off_e(uint32_t nq) { return 768u * nq; }
__host__ __device__ constexpr size_t wide_image_bytes(uint32_t group) {
    return ((size_t)wide_nq(group) * 772u + 1023u) & ~(size_t)1023u;
}

// The row's wide query image, built in LDS by the workgroup: wave w stages
// queries w, w + 8, ... . Lane l converts dims (d, d + 4),
// d = 8 (l / 4) + l % 4 = 64 g + 8 ks + k, which are K slots (2k, 2k + 1)
// of step ks for lane group g: dword k of the 16-byte entry. Buffer loads
// over exactly the row's `group` queries read zero past them, so the rows
// of the last query block past `group` are zero.
template <uint32_t NQB>
__device__ __forceinline__ void wide_stage_lds(const float* __restrict__ qc,
                                               const uint32_t* __restrict__ qs, size_t qrow0,
                                               uint32_t group, char* img) {
    constexpr uint32_t NQ = 32u * NQB, PER = NQ / 8u;
    const uint32_t lane = threadIdx.x & 63u, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t d = f16_stage_dim(lane);
    const uint32_t g = lane >> 5, ks = (lane >> 2) & 7u, k = lane & 3u;
    // P: chunk c = lane / 4 (kc = c & 7, gp = c >> 3), dword k = sign bits
    // 128 gp + 16 kc + 4 k .. + 3
    const uint32_t kc = (lane >> 2) & 7u, gp = lane >> 5;
    const uint32_t bit = 128u * gp + 16u * kc + 4u * k;
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(qc + qrow0 * kDC), 0, __builtin_amdgcn_readfirstlane(group * kDC * 4u),
        0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(qs + qrow0 * 8), 0, __builtin_amdgcn_readfirstlane(group * 32u), 0x00020000);
    float v0[PER], v1[PER];
    uint32_t sw[PER];
#pragma unroll
    for (uint32_t i = 0; i < PER; ++i) {  // all loads first, then the conversions
        const uint32_t j = wv + 8u * i;
        v0[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rq, (j * kDC + d) * 4u, 0, 0));
        v1[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rq, (j * kDC + d + 4u) * 4u, 0, 0));
        sw[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, (j * 8u + (bit >> 5)) * 4u, 0, 0);
    }
#pragma unroll
    for (uint32_t i = 0; i < PER; ++i) {
        const uint32_t j = wv + 8u * i;
        const int e = stage_exponent(v0[i], v1[i]);
        const float inv = ldexpf(1.0f, -e);
        const float d0 = v0[i] * inv, d1 = v1[i] * inv;
        // Truncating f16 split: x - hi is exact in f32 and lo keeps 11 more bits.
        const auto hi = __builtin_amdgcn_cvt_pkrtz(d0, d1);
        const auto lo = __builtin_amdgcn_cvt_pkrtz(d0 - (float)hi.x, d1 - (float)hi.y);
        const uint32_t h_hi = (((ks * 2u + 0u) * 2u + g) * NQ + j) * 16u + 4u * k;
        const uint32_t h_lo = (((ks * 2u + 1u) * 2u + g) * NQ + j) * 16u + 4u * k;
        *reinterpret_cast<uint32_t*>(img + h_hi) = __builtin_bit_cast(uint32_t, hi);
        *reinterpret_cast<uint32_t*>(img + h_lo) = __builtin_bit_cast(uint32_t, lo);
        const uint32_t pm = j < group ? pm1_bytes((sw[i] >> (bit & 31u)) & 15u).x : 0u;
        *reinterpret_cast<uint32_t*>(img + wide_off_p(NQ) + ((kc * 2u + gp) * NQ + j) * 16u + 4u * k) = pm;
        if (lane == 0) *reinterpret_cast<float*>(img + wide_off_e(NQ) + 4u * j) = ldexpf(1.0f, e);
    }
}

// A lane's share of one tile (its tile L % 32 of a 32-tile block, half
// g = L / 32): the 64-byte latent, 16 residual bytes (bits 128 g .. +127),
// scale and lambda, the flags word and its group-scale dword (groups
// 4 g .. 4 g + 3). Loaded before the block's codec is known; the codec's
// half of the latent is picked after.
struct WideTile {
    uint32_t lat[16];
    uint4 res;
    float scale, lambda;
    uint32_t flagw, gsw;
};

__device__ __forceinline__ void wide_load_tile(__amdgpu_buffer_rsrc_t rsrc, uint32_t n, uint32_t g,
                                               WideTile& t) {
    // Default cache policy: the two lane halves read parts of the same tile
    // in separate instructions, and the second must find it in L2.
    const uint32_t o = 128u * n;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint4 v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, o + 16u * j, 0, 0));
        t.lat[4 * j] = v.x, t.lat[4 * j + 1] = v.y, t.lat[4 * j + 2] = v.z, t.lat[4 * j + 3] = v.w;
    }
    t.res = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, o + 64u + 16u * g, 0, 0));
    const uint2 m = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rsrc, o + 96u, 0, 0));
    t.scale = __uint_as_float(m.x);
    t.lambda = __uint_as_float(m.y);
    t.flagw = __builtin_amdgcn_raw_buffer_load_b32(rsrc, o + 116u, 0, 0);
    t.gsw = __builtin_amdgcn_raw_buffer_load_b32(rsrc, o + 120u + 4u * g, 0, 0);
}

// The lane's half of the latent: INT4 dwords 8 g .. 8 g + 7; TQ3 code
// dwords 6 g .. 6 g + 5, then corr dwords 12 + 2 g, 13 + 2 g.
template <int CLS>
__device__ __forceinline__ void wide_pick_half(const uint32_t (&lat)[16], uint32_t g, uint32_t (&h)[8]) {
    // a bit-select in asm: written as a select, the compiler indexes the
    // latent array with g and moves it to scratch memory
    const uint32_t gm = 0u - g;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t a = CLS == kClsInt4 ? lat[j] : lat[j < 6 ? j : 6 + j];
        const uint32_t b = CLS == kClsInt4 ? lat[8 + j] : lat[j < 6 ? 6 + j : 8 + j];
        asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(h[j]) : "v"(gm), "v"(b), "v"(a));
    }
}

// f16 B operands of K-step ks for the lane's tile (see above).
__device__ __forceinline__ v8h wide_b_int4(uint32_t x, uint32_t magic, v2h off, v2h g2) {
    constexpr uint32_t M = 0x00F000F0u;  // nibbles k, k + 4 at bits 4..7 / 20..23
    const uint32_t d[4] = {((x << 4) & M) | magic, (x & M) | magic, ((x >> 4) & M) | magic,
                           ((x >> 8) & M) | magic};
    uint32_t r[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) r[k] = __builtin_bit_cast(uint32_t, (as_v2h(d[k]) + off) * g2);
    return __builtin_bit_cast(v8h, make_uint4(r[0], r[1], r[2], r[3]));
}

// x: the window's 24 code bits (code of dim j at 3 j); cm: the window's
// corr-LUT entry (corr bits placed under the codes, over the magic
// exponents); off: minus (base + 7.5) per half (NOCORR: base + 7).
__device__ __forceinline__ void wide_b_tq3(uint32_t x, uint4 cm, v2h off, v2h g2, v8h& bm, v8h& be) {
    constexpr uint32_t M = 0x001C01C0u;  // code of dim k at bits 6..8, of dim k + 4 at 18..20
    const uint32_t d[4] = {((x << 6) & M) | cm.x, ((x << 3) & M) | cm.y, (x & M) | cm.z,
                           ((x >> 3) & M) | cm.w};
    uint32_t m[4], e[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const v2h lh = as_v2h(d[k]) + off;  // L / 2, exact
        const v2h p = lh * g2;               // f16(L * gs)
        m[k] = __builtin_bit_cast(uint32_t, p);
        e[k] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(lh, g2, -p));  // exact
    }
    bm = __builtin_bit_cast(v8h, make_uint4(m[0], m[1], m[2], m[3]));
    be = __builtin_bit_cast(v8h, make_uint4(e[0], e[1], e[2], e[3]));
}

// 24-bit code window of K-step ks from the lane's six code dwords.
__device__ __forceinline__ uint32_t wide_code_window(const uint32_t* cd, int ks) {
    const int b = 24 * ks, j = b >> 5, sh = b & 31;
    return sh == 0 ? cd[j] : sh <= 8 ? cd[j] >> sh : __builtin_amdgcn_alignbit(cd[j + 1], cd[j], sh);
}

// Where a block's scores go.
struct WideOut {
    float* out;     // the row's scores, [group][n_tok]
    uint32_t n_tok, group;
};

// One codec-uniform INT4 or TQ3 block of 32 tiles against NQ = 32 NQB
// queries.
template <int CLS, uint32_t NQB>
__device__ __forceinline__ void wide_score_block(const char* lds_img, const uint2* pm1_lut,
                                                 const uint4* corr_lut, const WideTile& cur,
                                                 const WideOut& o, uint32_t tile0, uint32_t n_valid) {
    constexpr uint32_t NQ = 32u * NQB;
    const uint32_t lane = threadIdx.x & 63u, g = lane >> 5, col = lane & 31u;
    const uint4* H = reinterpret_cast<const uint4*>(lds_img);
    const uint4* P = reinterpret_cast<const uint4*>(lds_img + wide_off_p(NQ));
    const float* E = reinterpret_cast<const float*>(lds_img + wide_off_e(NQ));
    uint32_t magic = CLS == kClsInt4 ? 0x54005400u : 0u;  // 64.0 in both halves
    asm volatile("" : "+v"(magic));
    const uint32_t flags = cur.flagw >> 16;
    uint32_t h[8];
    wide_pick_half<CLS>(cur.lat, g, h);
    const bool nocorr = (flags & kFlagNoCorr) != 0;
    if constexpr (CLS == kClsTQ3) {
        if (nocorr) h[6] = h[7] = 0u;
    }
    auto b_of = [&](int ks, v8h& bm, v8h& be) {
        // group of K-step ks: 4 g + ks / 2 (byte ks / 2 of gsw)
        const _Float16 gv = (_Float16)(float)((cur.gsw >> (8 * (ks >> 1))) & 0xFFu);
        if constexpr (CLS == kClsInt4) {
            const v2h off = v2h{(_Float16)-72.0f, (_Float16)-72.0f};
            bm = wide_b_int4(h[ks], magic, off, v2h{gv, gv});
            be = bm;
        } else {
            const uint32_t cr = (h[6 + (ks >> 2)] >> (8 * (ks & 3))) & 0xFFu;
            const uint4 cm = corr_lut[cr];
            const v2h off = nocorr ? v2h{(_Float16)-39.0f, (_Float16)-519.0f}
                                   : v2h{(_Float16)-39.5f, (_Float16)-519.5f};
            const _Float16 g2v = gv + gv;
            wide_b_tq3(wide_code_window(h, ks), cm, off, v2h{g2v, g2v}, bm, be);
        }
    };
    auto a_of = [&](int ks, uint32_t qb, v8h& ah, v8h& al) {
        const uint32_t ia = ((uint32_t)ks * 2u * 2u + g) * NQ + 32u * qb + col;
        ah = __builtin_bit_cast(v8h, H[ia]);
        al = __builtin_bit_cast(v8h, H[ia + 2u * NQ]);
    };
    // The A operands of step ks + 1 are read from LDS during step ks; B
    // needs no copy ahead (the MFMAs of step ks run while the decode of
    // step ks + 1 issues). The scheduling barrier at the end of each step
    // keeps the compiler from hoisting later steps' LDS reads (and their
    // registers) above it.
    v16f acc[NQB];
#pragma unroll
    for (uint32_t qb = 0; qb < NQB; ++qb) acc[qb] = v16f{};
    v8h ah[NQB], al[NQB];
#pragma unroll
    for (uint32_t qb = 0; qb < NQB; ++qb) a_of(0, qb, ah[qb], al[qb]);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
        v8h bm, be, ah_n[NQB], al_n[NQB];
        b_of(ks, bm, be);
        if (ks < 7) {
#pragma unroll
            for (uint32_t qb = 0; qb < NQB; ++qb) a_of(ks + 1, qb, ah_n[qb], al_n[qb]);
        }
#pragma unroll
        for (uint32_t qb = 0; qb < NQB; ++qb) {
            acc[qb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[qb], bm, acc[qb], 0, 0, 0);
            acc[qb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[qb], bm, acc[qb], 0, 0, 0);
            if constexpr (CLS == kClsTQ3)
                acc[qb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[qb], be, acc[qb], 0, 0, 0);
        }
        if (ks < 7) {
#pragma unroll
            for (uint32_t qb = 0; qb < NQB; ++qb) ah[qb] = ah_n[qb], al[qb] = al_n[qb];
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    // Residual term: 16 sign bits per K-chunk kc, bits 16 kc .. of the
    // lane's 128, expanded to +-1 bytes once for both query blocks.
    const uint32_t rw[4] = {cur.res.x, cur.res.y, cur.res.z, cur.res.w};
    auto bt_of = [&](int kc) {
        const uint32_t w = rw[kc >> 1] >> (16 * (kc & 1));
        const uint2 lo = pm1_lut[w & 0xFFu], hi = pm1_lut[(w >> 8) & 0xFFu];
        return v4i{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
    };
    auto aq_of = [&](int kc, uint32_t qb) {
        return __builtin_bit_cast(v4i, P[((uint32_t)kc * 2u + g) * NQ + 32u * qb + col]);
    };
    v16i dots[NQB];
#pragma unroll
    for (uint32_t qb = 0; qb < NQB; ++qb) dots[qb] = v16i{};
#pragma unroll
    for (int kc = 0; kc < 8; ++kc) {
        const v4i bt = bt_of(kc);
#pragma unroll
        for (uint32_t qb = 0; qb < NQB; ++qb)
            dots[qb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aq_of(kc, qb), bt, dots[qb], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    }
    const float lvl = CLS == kClsInt4 ? 1.0f : 0.25f;
    const float s = cur.scale * (1.0f / 255.0f) * lvl;
    const float lam = (flags & kFlagWarm) ? 0.0f : cur.lambda;
    const uint32_t t = tile0 + col;
#pragma unroll
    for (uint32_t qb = 0; qb < NQB; ++qb) {
        const v16i dot = dots[qb];
        float sc[16];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float4 qe = *reinterpret_cast<const float4*>(E + 32u * qb + 8u * j + 4u * g);
            const float q4[4] = {qe.x, qe.y, qe.z, qe.w};
#pragma unroll
            for (int r = 0; r < 4; ++r)
                sc[4 * j + r] = fmaf(lam, (float)dot[4 * j + r], acc[qb][4 * j + r] * (s * q4[r]));
        }
        // Accumulator i is query row 32 qb + 4 g + 8 (i / 4) + i % 4. The
        // stores go through a buffer over the block's rows that exist
        // (n_tok < 2^25 keeps every offset below 2^32): with all 32 rows,
        // the row offset rides in the SGPR operand; otherwise in the VGPR
        // operand, where the range check drops rows at or past `group`.
        const uint32_t rows = o.group - 32u * qb < 32u ? o.group - 32u * qb : 32u;
        const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(
            o.out + (size_t)32u * qb * o.n_tok, 0, __builtin_amdgcn_readfirstlane(rows * o.n_tok * 4u),
            0x00020000);
        const uint32_t voff = (4u * g * o.n_tok + t) * 4u;
        if (col < n_valid) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const uint32_t di = (8u * (i >> 2) + (i & 3)) * o.n_tok * 4u;
                if (rows == 32u)
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(sc[i]), ors, voff,
                                                          __builtin_amdgcn_readfirstlane(di), kCachePolicyNT);
                else
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(sc[i]), ors, voff + di, 0,
                                                          kCachePolicyNT);
            }
        }
    }
}

// Scoring of tile rows for 16 < group <= kMfmaMaxGroup. Workgroups of 8
// waves stay resident and loop over the row's 512-tile chunks (chunk
// blockIdx.x + k gridDim.x); wave w takes the chunk's 32-tile blocks 2w and
// 2w + 1. The workgroup builds the row's query image in LDS once
// (wide_stage_lds). A codec-uniform INT4 or TQ3 block runs
// wide_score_block, any other block the per-lane path (lanes 0..31, one
// tile each).
constexpr uint32_t kWideChunk = 512;
constexpr uint32_t kWideMaxTok = 1u << 25;  // longer rows take score_rows_kernel

template <uint32_t NQB>
__global__ __launch_bounds__(512, 4) void score_rows_wide_kernel(
    const uint4* __restrict__ tiles, uint32_t n_tok, uint32_t group,
    const float* __restrict__ qc, const uint32_t* __restrict__ qs, float* __restrict__ scores) {
    __shared__ float cb[16];
    __shared__ uint2 pm1_lut[256];
    __shared__ uint4 corr_lut[256];
    extern __shared__ __attribute__((aligned(16))) float qlds[];  // wide_image_bytes(group)
    const uint32_t row = blockIdx.y;
    const size_t qrow0 = (size_t)row * group;
    const uint32_t lane = threadIdx.x & 63u, g = lane >> 5, col = lane & 31u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t n_chunks = (n_tok + kWideChunk - 1) / kWideChunk;
    wide_stage_lds<NQB>(qc, qs, qrow0, group, reinterpret_cast<char*>(qlds));
    // Block i of this wave: chunk blockIdx.x + (i / 2) gridDim.x, tiles
    // 64 wave + 32 (i % 2) of it. Tiles at or past n_valid read as zero.
    const uint4* row_tiles = tiles + (size_t)row * n_tok * 8;
    auto block_tile0 = [&](uint32_t i) {
        return (blockIdx.x + (i >> 1) * gridDim.x) * kWideChunk + 64u * wave + 32u * (i & 1u);
    };
    auto block_rsrc = [&](uint32_t tile0) {
        const uint32_t nv = tile0 < n_tok ? n_tok - tile0 : 0u;
        return __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint4*>(row_tiles + (size_t)tile0 * 8), 0,
            __builtin_amdgcn_readfirstlane((nv < 32u ? nv : 32u) * 128u), 0x00020000);
    };
    auto block_exists = [&](uint32_t i) {
        return blockIdx.x + (i >> 1) * gridDim.x < n_chunks && block_tile0(i) < n_tok;
    };
    stage_codebook(cb);
    if (threadIdx.x < 256u) {
        const uint32_t b = threadIdx.x;
        pm1_lut[b] = pm1_bytes(b);
        uint32_t e[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            e[k] = (((b >> k) & 1u) << 5) | (((b >> (k + 4)) & 1u) << 17) | 0x60005000u;
        corr_lut[b] = make_uint4(e[0], e[1], e[2], e[3]);
    }
    __syncthreads();
    const char* lds_img = reinterpret_cast<const char*>(qlds);
    const WideOut o{scores + qrow0 * n_tok, n_tok, group};
    // No block is loaded ahead: the 16 resident waves of a CU cover each
    // other's load latency, and a tile held across the loop would cost the
    // registers that keep 4 waves per SIMD.
    for (uint32_t i = 0; block_exists(i); ++i) {
        const uint32_t tile0 = block_tile0(i);
        const uint32_t n_valid = n_tok - tile0;  // > 0
        const __amdgpu_buffer_rsrc_t rs = block_rsrc(tile0);
        WideTile cur;
        wide_load_tile(rs, col, g, cur);
        const int cls = codec_class(cur.flagw >> 16);
        const int c0 = __builtin_amdgcn_readfirstlane(cls);  // lane 0's tile is valid
        const bool uniform = __all(cls == c0 || col >= n_valid);
        if (uniform && c0 == kClsInt4) {
            wide_score_block<kClsInt4, NQB>(lds_img, pm1_lut, corr_lut, cur, o, tile0, n_valid);
        } else if (uniform && c0 == kClsTQ3) {
            wide_score_block<kClsTQ3, NQB>(lds_img, pm1_lut, corr_lut, cur, o, tile0, n_valid);
        } else if (lane < 32u && col < n_valid) {
            // per-lane path: lane L < 32 scores tile tile0 + L
            uint32_t w[32];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint4 v = __builtin_bit_cast(
                    uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, 128u * col + 16u * j, 0, 0));
                w[4 * j] = v.x, w[4 * j + 1] = v.y, w[4 * j + 2] = v.z, w[4 * j + 3] = v.w;
            }
            score_dispatch<false, false>(w, group, qrow0, qc, qs, cb, o.out, nullptr, n_tok, tile0 + col);
        }
    }
}

// CCOS paged scoring on the fast path (pages of at least 64 tiles, group <=
// kMfmaMaxGroup): as score_rows_fast_kernel, with each wave's 64 consecutive
// tokens gathered from one physical page. Block (x, y) covers tokens
// [256x, 256x+256) of row y = s*n_kv + h (sequence s, KV head h); token t
// lives in page page_table[y*max_pages + t/page_tiles] at slot t % page_tiles.
// (Token blocks along x keep a row's pages together in time; with rows along
// x the paged C5 scoring ran 9 % slower.)
template <uint32_t REG_ROWS>
__global__ __launch_bounds__(256) void score_paged_fast_kernel(
    const uint4* __restrict__ arena, uint32_t page_shift, const uint32_t* __restrict__ page_table,
    uint32_t max_pages, const uint32_t* __restrict__ seq_len,
    const unsigned long long* __restrict__ score_base, uint32_t n_kv, uint32_t group,
    const float* __restrict__ qc, const uint32_t* __restrict__ qs, float* __restrict__ scores) {
    __shared__ float cb[16];
    __shared__ uint4 tile_lds[4][512];
    __shared__ __attribute__((aligned(16))) float qstatic[REG_ROWS ? staging_bytes(REG_ROWS) / 4 : 1];
    extern __shared__ __attribute__((aligned(16))) float qlds[];
    const uint32_t y = blockIdx.y, bx = blockIdx.x;
    const uint32_t s = y / n_kv, h = y - s * n_kv;
    const uint32_t len = seq_len[s];
    if (bx * blockDim.x >= len) return;  // whole block past this sequence
    const size_t qrow0 = (size_t)y * group;
    const uint32_t t = bx * blockDim.x + threadIdx.x;
    const StagedQueries sq =
        carve_staging(REG_ROWS ? qstatic : qlds, REG_ROWS ? REG_ROWS : staging_rows(group));
    QueryRegs<REG_ROWS ? REG_ROWS : 4> qr;
    if constexpr (REG_ROWS > 0) stage_issue<REG_ROWS>(qc, qrow0, group, qr);
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t wave0 = bx * blockDim.x + 64u * wave;
    const uint32_t n_valid = wave0 < len ? len - wave0 : 0u;
    const uint4* base = arena;
    if (n_valid) {  // 64 | page_tiles: the wave's tokens share one page
        const uint32_t phys = page_table[(size_t)y * max_pages + (wave0 >> page_shift)];
        base = arena + (((size_t)phys << page_shift) + (wave0 & ((1u << page_shift) - 1u))) * 8;
    }
    fetch_tiles_lds(base, n_valid, tile_lds[wave]);
    stage_codebook(cb);
    if constexpr (REG_ROWS > 0) {
        stage_commit<REG_ROWS>(qr, group, sq);
        lds_barrier();
    } else {
        stage_queries(qc, qrow0, group, sq.q32);
        stage_queries_f16(qc, qrow0, group, sq.q16, sq.qexp);
        __syncthreads();
    }
    uint32_t w[32];
    fetch_tiles_readback(tile_lds[wave], w);
    const bool valid = t < len;
    float* out = scores + score_base[s] + (size_t)h * group * len;
    if (score_wave_try_mfma(w, valid, group, qrow0, sq.q32, cb, sq.q16, sq.qexp, qs, out, len, t))
        return;
    if (valid) score_dispatch<false, false>(w, group, qrow0, qc, qs, cb, out, nullptr, len, t);
}

// CCOS paged scoring, general case (pages of fewer than 64 tiles, or groups
// past kMfmaMaxGroup): one lane per token, tiles gathered per lane. Blocks
// map to (token block, row) as in score_paged_fast_kernel.
__global__ __launch_bounds__(256) void score_paged_kernel(
    const uint4* __restrict__ arena, uint32_t page_shift, const uint32_t* __restrict__ page_table,
    uint32_t max_pages, const uint32_t* __restrict__ seq_len,
    const unsigned long long* __restrict__ score_base, uint32_t n_kv, uint32_t group,
    const float* __restrict__ qc, const uint32_t* __restrict__ qs, float* __restrict__ scores) {
    __shared__ float cb[16];
    extern __shared__ __attribute__((aligned(16))) float qlds[];  // staged_rows * kQStride
    const uint32_t y = blockIdx.y, bx = blockIdx.x;
    const uint32_t s = y / n_kv, h = y - s * n_kv;
    const uint32_t len = seq_len[s];
    if (bx * blockDim.x >= len) return;  // whole block past this sequence
    const size_t qrow0 = (size_t)y * group;
    const uint32_t t = bx * blockDim.x + threadIdx.x;
    const bool valid = t < len;
    uint32_t w[32];
    if (valid) {
        const uint32_t phys = page_table[(size_t)y * max_pages + (t >> page_shift)];
        const size_t slot = ((size_t)phys << page_shift) + (t & ((1u << page_shift) - 1u));
        load_tile(arena + slot * 8, w);
    } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) w[i] = 0u;
    }
    stage_codebook(cb);
    const bool mfma = group <= kMfmaMaxGroup;
    const StagedQueries sq = carve_staging(qlds, staging_rows(group));
    if (mfma) {
        stage_queries(qc, qrow0, group, sq.q32);
        stage_queries_f16(qc, qrow0, group, sq.q16, sq.qexp);
    }
    __syncthreads();
    float* out = scores + score_base[s] + (size_t)h * group * len;
    if (mfma && score_wave_try_mfma(w, valid, group, qrow0, sq.q32, cb, sq.q16, sq.qexp, qs, out,
                                    len, t))
        return;
    if (!valid) return;
    score_dispatch<false, false>(w, group, qrow0, qc, qs, cb, out, nullptr, len, t);
}

// ---------------------------------------------------------------------------
// Top-k per score row: score descending, ties to the lower token index.
//
// Two stages; each reads its input once, with coalesced branch-free loads:
//  1. topk_segment_kernel: one 512-thread workgroup per 16384-score segment
//     of a (sequence, query head) row, 32 scores per thread in registers; its
//     top k go, sorted, to the row's candidate list (k slots per segment).
//  2. topk_merge_kernel: one workgroup per row merges the row's sorted
//     segment lists by rank counting (binary searches).
// The segments use block_topk: scores are order-preserving u32 keys; each wave
// extracts the r-th largest of its 64 per-thread maxima (r rounds of a DPP
// wave maximum), r = ceil(kk / waves); tau = the smallest of those is a lower
// bound of the kk-th largest key (every wave has r threads holding a key
// >= tau), so the keys >= tau contain the whole top kk, ties included.
// They are typically a few times kk: each one's rank in (key desc, index
// asc) order is counted against the others and ranks < kk are written in
// that order. When they do not fit in LDS (heavy ties), an exact 8-bit radix
// select finds the kk-th largest key T and the winners are the keys > T
// plus the first keys == T in index order.

constexpr int kSegThreads = 512;       // 32 scores per thread (kTopkSeg = 16384)
constexpr int kMergeThreads = 256;     // merge workgroup
constexpr uint32_t kTopkCap = 1024;    // candidates ranked in LDS

__device__ __forceinline__ uint32_t order_key(float f) {
    // -0.0 and +0.0 compare equal, so they share a key (ties then go by index).
    const uint32_t u = __float_as_uint(f == 0.0f ? 0.0f : f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key_to_float(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// Inclusive prefix sum of one u32 per lane over the wave (DPP row shifts,
// then row broadcasts).
__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t x) {
#define SLHA_DPP_ADD(ctrl, rows) \
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, ctrl, rows, 0xF, false)
    SLHA_DPP_ADD(0x111, 0xF);  // row_shr:1
    SLHA_DPP_ADD(0x112, 0xF);  // row_shr:2
    SLHA_DPP_ADD(0x114, 0xF);  // row_shr:4
    SLHA_DPP_ADD(0x118, 0xF);  // row_shr:8
    SLHA_DPP_ADD(0x142, 0xA);  // row_bcast:15
    SLHA_DPP_ADD(0x143, 0xC);  // row_bcast:31
#undef SLHA_DPP_ADD
    return x;
}

// Exclusive prefix sum of one u32 per thread over a workgroup of NT threads
// (NT a multiple of 64); `tmp` holds NT/64 words of LDS. Returns the
// exclusive prefix; *total receives the sum. Contains barriers.
template <int NT>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t x, uint32_t* tmp,
                                                         uint32_t* total) {
    const uint32_t lane = threadIdx.x & 63u, wv = threadIdx.x >> 6;
    const uint32_t incl = wave_inclusive_sum(x);
    if (lane == 63) tmp[wv] = incl;
    __syncthreads();
    uint32_t before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) {
        const uint32_t t = tmp[w];
        before += (uint32_t)w < wv ? t : 0u;
        all += t;
    }
    __syncthreads();
    *total = all;
    return before + incl - x;
}

// Max of one u32 per lane across the wave (DPP row steps, then row
// broadcasts 15 and 31 leave it in lane 63).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
#define SLHA_DPP_UMAX(ctrl, rows) \
    x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, ctrl, rows, 0xF, false))
    SLHA_DPP_UMAX(0xB1, 0xF);   // quad_perm [1,0,3,2]
    SLHA_DPP_UMAX(0x4E, 0xF);   // quad_perm [2,3,0,1]
    SLHA_DPP_UMAX(0x141, 0xF);  // row_half_mirror
    SLHA_DPP_UMAX(0x140, 0xF);  // row_mirror
    SLHA_DPP_UMAX(0x142, 0xA);  // row_bcast:15
    SLHA_DPP_UMAX(0x143, 0xC);  // row_bcast:31
#undef SLHA_DPP_UMAX
    return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}

// r-th largest (1-based, 1 <= r <= 64) of one u32 per lane across the wave:
// r rounds of "take the maximum, retire the lowest lane holding it".
__device__ __forceinline__ uint32_t wave_rth_largest(uint32_t x, uint32_t r) {
    const uint32_t lane = threadIdx.x & 63u;
    bool live = true;
    uint32_t m = 0;
    for (uint32_t i = 0; i < r; ++i) {
        m = wave_max_u32(live ? x : 0u);
        const unsigned long long holders = __ballot(live && x == m);
        if (holders == 0ull) break;  // fewer than r live lanes: m is 0 already
        if (lane == (uint32_t)__ffsll((long long)holders) - 1u) live = false;
    }
    return m;
}

// hist[256]: counts of the current 8-bit digit; finds the bin holding the
// need-th largest key and the count of keys above it (threads 0..255 own one
// bin each). Contains barriers.
template <int NT>
__device__ __forceinline__ void select_digit(const uint32_t* hist, uint32_t need, uint32_t* tmp,
                                             uint32_t* sh_bin, uint32_t* sh_above) {
    const uint32_t t = threadIdx.x;
    const uint32_t cnt = t < 256u ? hist[255u - t] : 0u;  // thread t <-> bin 255 - t
    uint32_t total;
    const uint32_t above = block_exclusive_scan<NT>(cnt, tmp, &total);
    if (t < 256u && above < need && above + cnt >= need) {
        *sh_bin = 255u - t;
        *sh_above = above;
    }
    __syncthreads();
}

// Exact radix select over the valid items of the workgroup: the need-th
// largest of value(j) among items with take(j) (8-bit digits, LDS
// histograms). Returns it and sets *need_eq to how many items equal to it
// are among the top `need`. Every thread calls it.
template <int NT, int PER, typename Val, typename Take>
__device__ __forceinline__ uint32_t radix_select(Val value, Take take, uint32_t need,
                                                 uint32_t* hist, uint32_t* tmp, uint32_t* sh,
                                                 uint32_t* need_eq) {
    uint32_t prefix = 0, mask = 0;
#pragma unroll 1
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (uint32_t i = threadIdx.x; i < 256u; i += NT) hist[i] = 0u;
        __syncthreads();
#pragma unroll 4
        for (int j = 0; j < PER; ++j) {
            const uint32_t v = value(j);
            if (take(j) && (v & mask) == prefix) atomicAdd(&hist[(v >> shift) & 255u], 1u);
        }
        __syncthreads();
        select_digit<NT>(hist, need, tmp, &sh[0], &sh[1]);
        need -= sh[1];
        prefix |= sh[0] << shift;
        mask |= 255u << shift;
        __syncthreads();
    }
    *need_eq = need;
    return prefix;
}

// Top kk (<= kMaxTopK, <= number of valid items) of the workgroup's items:
// thread t holds items j = 0..PER-1 with key_at(j), index idx_at(j) (unique)
// and ok_at(j) (valid). key_ld/ok_ld give the same from memory for any j;
// the rare heavy-tie path uses them so that the register copies need not
// stay alive through it. Writes the winners, ranked, to out_key/out_idx[0..kk).
// Shared-memory scratch comes from the caller. Every thread calls it.
template <int NT, int PER, typename KeyAt, typename OkAt, typename KeyLd, typename OkLd,
          typename IdxAt>
__device__ __forceinline__ void block_topk(KeyAt key_at, OkAt ok_at, KeyLd key_ld, OkLd ok_ld,
                                           IdxAt idx_at, uint32_t kk,
                                           uint2* cand, uint32_t* rank, uint32_t* hist,
                                           uint32_t* tmp, uint32_t* sh,
                                           uint32_t* __restrict__ out_key,
                                           uint32_t* __restrict__ out_idx) {
    constexpr uint32_t kWaves = NT / 64;
    const uint32_t wv = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    uint32_t m = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) m = ok_at(j) ? max(m, key_at(j)) : m;
    uint32_t r = (kk + kWaves - 1) / kWaves;
    r = r < 1u ? 1u : (r > 64u ? 64u : r);
    const uint32_t tau_w = wave_rth_largest(m, r);
    if (lane == 0) tmp[wv] = tau_w;
    __syncthreads();
    uint32_t tau = 0xFFFFFFFFu;
#pragma unroll
    for (uint32_t w = 0; w < kWaves; ++w) tau = min(tau, tmp[w]);
    __syncthreads();
    uint32_t c = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) c += (ok_at(j) && key_at(j) >= tau) ? 1u : 0u;
    uint32_t total;
    uint32_t pos = block_exclusive_scan<NT>(c, tmp, &total);
    if (total <= kTopkCap) {
#pragma unroll
        for (int j = 0; j < PER; ++j)
            if (ok_at(j) && key_at(j) >= tau) cand[pos++] = make_uint2(key_at(j), idx_at(j));
    } else {
        // Heavy ties: the kk-th largest key T, then among the keys == T the
        // `need` lowest indices (the largest ~index), both by radix select.
        // This rare path reads the keys again (key_ld) rather than keeping
        // the register copies alive, which keeps the common path's register
        // budget low.
        uint32_t need;
        const uint32_t thr = radix_select<NT, PER>(key_ld, ok_ld, kk, hist, tmp, sh, &need);
        auto is_eq = [&](int j) { return ok_ld(j) && key_ld(j) == thr; };
        auto inv_idx = [&](int j) { return ~idx_at(j); };
        uint32_t one;
        const uint32_t ithr = need ? radix_select<NT, PER>(inv_idx, is_eq, need, hist, tmp, sh, &one)
                                   : 0xFFFFFFFFu;
        auto win = [&](int j) {
            const uint32_t kj = key_ld(j);
            return ok_ld(j) && (kj > thr || (need && kj == thr && ~idx_at(j) >= ithr));
        };
        c = 0;
#pragma unroll 4
        for (int j = 0; j < PER; ++j) c += win(j) ? 1u : 0u;
        pos = block_exclusive_scan<NT>(c, tmp, &total);
#pragma unroll 4
        for (int j = 0; j < PER; ++j)
            if (win(j)) cand[pos++] = make_uint2(key_ld(j), idx_at(j));
    }
    // rank by (key desc, index asc); ranks < kk are the result, in order.
    // Candidate i's rank is summed over `slices` threads, each comparing it
    // with a contiguous slice of the others.
    for (uint32_t i = threadIdx.x; i < total; i += NT) rank[i] = 0u;
    __syncthreads();
    const uint32_t slices = total ? (NT / total > 0 ? NT / total : 1u) : 1u;
    const uint32_t per = (total + slices - 1) / slices;
    for (uint32_t p = threadIdx.x; p < total * slices; p += NT) {
        const uint32_t i = p / slices, q = p - i * slices;
        const uint2 me = cand[i];
        const uint32_t j0 = q * per, j1 = j0 + per < total ? j0 + per : total;
        uint32_t rk = 0;
        uint32_t j = j0;
        for (; j + 4 <= j1; j += 4) {
            const uint2 o0 = cand[j], o1 = cand[j + 1], o2 = cand[j + 2], o3 = cand[j + 3];
            rk += (o0.x > me.x || (o0.x == me.x && o0.y < me.y)) ? 1u : 0u;
            rk += (o1.x > me.x || (o1.x == me.x && o1.y < me.y)) ? 1u : 0u;
            rk += (o2.x > me.x || (o2.x == me.x && o2.y < me.y)) ? 1u : 0u;
            rk += (o3.x > me.x || (o3.x == me.x && o3.y < me.y)) ? 1u : 0u;
        }
        for (; j < j1; ++j) {
            const uint2 o = cand[j];
            rk += (o.x > me.x || (o.x == me.x && o.y < me.y)) ? 1u : 0u;
        }
        if (rk) atomicAdd(&rank[i], rk);
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < total; i += NT) {
        const uint32_t rk = rank[i];
        if (rk < kk) {
            out_key[rk] = cand[i].x;
            out_idx[rk] = cand[i].y;
        }
    }
}

__global__ __launch_bounds__(kSegThreads, 2) void topk_segment_kernel(
    const float* __restrict__ scores, const uint32_t* __restrict__ seq_len,
    const unsigned long long* __restrict__ score_base, uint32_t hq, uint32_t k, uint32_t nseg_max,
    uint32_t* __restrict__ cand_key, uint32_t* __restrict__ cand_idx) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t tmp[kSegThreads / 64];
    __shared__ uint32_t sh[2];
    __shared__ uint2 cand[kTopkCap];
    __shared__ uint32_t rank[kTopkCap];
    const uint32_t row = blockIdx.x, seg = blockIdx.y;
    const uint32_t s = row / hq, qh = row - s * hq;
    const uint32_t len = seq_len[s];
    const unsigned long long sbase = score_base[s];  // issued with seq_len
    const uint32_t start = seg * kTopkSeg;
    if (start >= len) return;  // whole segment past this sequence
    const uint32_t n = len - start < kTopkSeg ? len - start : kTopkSeg;
    const uint32_t kk = k < n ? k : n;
    constexpr int PER = kTopkSeg / kSegThreads;
    // Item j of thread t is score start + j * kSegThreads + t; the buffer
    // range ends at the segment's last score, so the loads past it read zero
    // without a branch and all PER are in flight together.
    const float* sc = scores + sbase + (size_t)qh * len + start;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(sc), 0, __builtin_amdgcn_readfirstlane(n * 4u), 0x00020000);
    // Key 0 marks an item past the segment: order_key never yields 0 for a
    // score (it would take the NaN 0xFFFFFFFF, which is raised to key 1).
    uint32_t key[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const uint32_t kj = max(order_key(__builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, (j * kSegThreads + threadIdx.x) * 4u, 0, 0))), 1u);
        key[j] = (uint32_t)j * kSegThreads + threadIdx.x < n ? kj : 0u;
    }
    const size_t o = ((size_t)row * nseg_max + seg) * k;
    block_topk<kSegThreads, PER>(
        [&](int j) { return key[j]; }, [&](int j) { return key[j] != 0u; },
        [&](int j) {
            return max(order_key(__builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, (j * kSegThreads + threadIdx.x) * 4u, 0, 0))), 1u);
        },
        [&](int j) { return (uint32_t)j * kSegThreads + threadIdx.x < n; },
        [&](int j) { return start + (uint32_t)j * kSegThreads + threadIdx.x; }, kk, cand, rank, hist,
        tmp, sh, cand_key + o, cand_idx + o);
}

// Merge of the sorted per-segment lists of a row. Segment g's list holds its
// top min(k, n_g) scores sorted by (key desc, index asc), and segment g's
// indices all precede segment g+1's. A candidate's final rank is its position
// in its own list plus, for every other list, the number of that list's
// entries that precede it: entries with a larger key, plus entries with an
// equal key from an earlier segment (binary search, the lists being sorted).
// Ranks are unique, so candidates with rank < k write themselves in place.
// The lists live in dynamic LDS (nseg_max * k * 8 bytes, at most 64 KiB).
__global__ __launch_bounds__(kMergeThreads) void topk_merge_kernel(
    const uint32_t* __restrict__ cand_key, const uint32_t* __restrict__ cand_idx,
    const uint32_t* __restrict__ seq_len, uint32_t hq, uint32_t k, uint32_t nseg_max,
    uint32_t* __restrict__ topk_idx, float* __restrict__ topk_val) {
    extern __shared__ uint32_t merge_lds[];
    uint32_t* lkey = merge_lds;                      // [nseg_max * k]
    uint32_t* lidx = merge_lds + (size_t)nseg_max * k;
    const uint32_t row = blockIdx.x;
    const uint32_t s = row / hq;
    const uint32_t len = seq_len[s];
    const uint32_t kk = k < len ? k : len;
    const uint32_t nseg = (len + kTopkSeg - 1) / kTopkSeg;
    const size_t base = (size_t)row * nseg_max * k;
    const uint32_t slots = nseg * k;
    for (uint32_t c = threadIdx.x; c < slots; c += kMergeThreads) {
        lkey[c] = cand_key[base + c];
        lidx[c] = cand_idx[base + c];
    }
    __syncthreads();
    auto list_len = [&](uint32_t g) {
        const uint32_t n = len - g * kTopkSeg;
        return n < k ? n : k;
    };
    for (uint32_t c = threadIdx.x; c < slots; c += kMergeThreads) {
        const uint32_t g = c / k, p = c - g * k;
        if (p >= list_len(g)) continue;
        const uint32_t key = lkey[c];
        uint32_t rank = p;
        for (uint32_t h = 0; h < nseg && rank < kk; ++h) {
            if (h == g) continue;
            // entries of list h before this candidate: key > K, or key == K
            // when h is an earlier segment (first position failing that)
            const uint32_t* lk = lkey + h * k;
            uint32_t lo = 0, hi = list_len(h);
            while (lo < hi) {
                const uint32_t mid = (lo + hi) >> 1;
                const uint32_t e = lk[mid];
                if (e > key || (h < g && e == key))
                    lo = mid + 1;
                else
                    hi = mid;
            }
            rank += lo;
        }
        if (rank < kk) {
            const size_t oo = (size_t)row * k + rank;
            topk_idx[oo] = lidx[c];
            topk_val[oo] = key_to_float(key);
        }
    }
    for (uint32_t i = kk + threadIdx.x; i < k; i += kMergeThreads) {
        const size_t oo = (size_t)row * k + i;
        topk_idx[oo] = 0xFFFFFFFFu;
        topk_val[oo] = -INFINITY;
    }
}

// ---------------------------------------------------------------------------
// Encode: Rust numeric semantics.

// `f as i32`: truncation, saturating at the i32 range, NaN -> 0. That is
// exactly what v_cvt_i32_f32 does, so one instruction replaces the branches.
__device__ __forceinline__ int32_t rs_i32(float f) {
    int32_t r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(f));
    return r;
}
// `f.round() as i32` (half away from zero, then the saturating cast):
// f + copysign(0.5 - 2^-25, f) truncates to round(f) for every f32 (checked
// over all 2^32 inputs against roundf), and v_cvt_i32_f32 truncates and
// saturates as rs_i32 does. Two VALU and the convert instead of roundf's five.
__device__ __forceinline__ int32_t rs_round_i32(float f) {
    return rs_i32(f + copysignf(0x1.fffffep-2f, f));
}
__device__ __forceinline__ uint32_t rs_u8(float f) {  // `f as u8`
    if (isnan(f)) return 0u;
    if (f >= 255.0f) return 255u;
    if (f <= 0.0f) return 0u;
    return (uint32_t)f;
}
__device__ __forceinline__ float rs_clampf(float x, float lo, float hi) {  // f32::clamp
    if (x < lo) x = lo;
    if (x > hi) x = hi;
    return x;
}
__device__ __forceinline__ int32_t clampi(int32_t x, int32_t lo, int32_t hi) {
    return x < lo ? lo : (x > hi ? hi : x);
}

template <int LO, int HI>
__device__ __forceinline__ float absmax(const float* v) {
    float m = 0.0f;
#pragma unroll
    for (int d = LO; d < HI; ++d) m = fmaxf(m, fabsf(v[d]));
    return m;
}

// (global, gs) from the per-section steps: int4.rs:43-50 and its twins.
__device__ __forceinline__ float group_bytes(const float* steps, uint32_t* gsw) {
    float global = 0.0f;
#pragma unroll
    for (int g = 0; g < 8; ++g) global = fmaxf(global, steps[g]);
    if (!(global > 0.0f)) global = 1.0f;
    gsw[0] = gsw[1] = 0u;
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        const float r = roundf(steps[g] / global * 255.0f);
        gsw[g >> 2] |= rs_u8(rs_clampf(r, 1.0f, 255.0f)) << (8 * (g & 3));
    }
    return global;
}

__device__ __forceinline__ void put_bits(uint32_t* lw, int p, uint32_t v) {
    const int wi = p >> 5, sh = p & 31;
    lw[wi] |= v << sh;
    if (sh > 29 && wi + 1 < 16) lw[wi + 1] |= v >> (32 - sh);
}

// nf4.rs:7-18 scans the 16 levels for the first smallest f32 |t - L_i|.
// For t in [-1, 1] (the quantiser clamps it there) level i beats level i - 1
// in that f32 comparison exactly when t >= T_i, and only neighbours can tie,
// so the scan's index is the number of thresholds at or below t (0 for NaN,
// as in the scan). T_i is the smallest f32 for which level i wins, found by
// bisection; the count equals the scan for every f32 in [-1, 1] and every
// NaN. 15 compares instead of 16 distance updates.
__device__ __forceinline__ uint32_t nf4_nearest(float t) {
    constexpr float kT[15] = {-0x1.b51eb6p-1f, -0x1.3fe5c8p-1f, -0x1.eacd9ep-2f, -0x1.7460a8p-2f,
                              -0x1.0d9e82p-2f, -0x1.5f3b64p-3f, -0x1.5ab9f6p-4f, 0x1p-29f,
                              0x1.5ab9f8p-4f,  0x1.5f3b66p-3f,  0x1.0d9e84p-2f,  0x1.7460acp-2f,
                              0x1.eacda0p-2f,  0x1.3fe5cap-1f,  0x1.b51ebap-1f};
    uint32_t n = 0;
#pragma unroll
    for (int i = 0; i < 15; ++i) n += t >= kT[i] ? 1u : 0u;
    return n;
}

// The quantisers' per-dim quotient x / b (b = the group's effective scale),
// correctly rounded as the reference's division is.
//
// FAST: y = RN(1 / b) once per group, then q0 = RN(x y), the remainder
// r = x - q0 b (exact in one fma) and RN(q0 + r y), which is RN(x / b) by
// Markstein's theorem (y within half an ulp of 1 / b, q0 within one ulp of
// x / b, r exact). r is a multiple of ulp(q0) ulp(b) below b ulp(q0) in
// magnitude, so it is exact once ulp(q0) ulp(b) >= 2^-149: for
// 2^-71 <= b <= 2^96 that covers every |x / b| >= 2^-32, and quantize()
// takes this path only for such b. Smaller quotients can be an ulp off,
// which none of the quantisers can see: the decisions nearest to 0 are
// TQ3's code at t = -2^-23 and NF4's choice between +-0.0421 at t = 2^-29.
// Three VALU instead of the division's eleven.
template <bool FAST>
__device__ __forceinline__ float quot(float x, float b, float y) {
    if constexpr (FAST) {
        const float q0 = x * y;
        const float r = fmaf(-q0, b, x);
        return fmaf(r, y, q0);
    } else {
        return x / b;
    }
}
__device__ __forceinline__ bool quot_fast_ok(float b) { return b >= 0x1p-71f && b <= 0x1p96f; }

// One TQ3 code + correction bit from t = val / eff (tq3.rs:31-46, mix3.rs:44-58).
// Returns the level the tile decodes to, code - 3.5 +- 0.25 (tile.rs:187-207),
// in the same f32 operations as tq3_level_exact.
__device__ __forceinline__ float tq3_put(uint32_t* lw, int codes_bit0, int corr_bit0, int ld,
                                         float t) {
    const uint32_t code = (uint32_t)clampi(rs_round_i32(t + 3.5f), 0, 7);
    put_bits(lw, codes_bit0 + 3 * ld, code);
    const float level = (float)code - 3.5f;
    const bool corr = t - level > 0.0f;
    if (corr) put_bits(lw, corr_bit0 + ld, 1u);
    return level + (corr ? 1.0f : -1.0f) * 0.25f;
}

// Codes of v for the effective scale of each group (eff[0] alone for the
// single-scale INT4 codec; eff[0] = the 8-bit section for mixed and MIX3).
// RESID (INT4 codecs and TQ3): v[d] becomes the residual v[d] - level * eff,
// the same product and difference as v[d] - dequant_dim (group_scale_exact
// is eff; for the single-scale codec gs = 255 and eff * 1 = eff).
template <int CODEC, bool FAST, bool RESID>
__device__ __forceinline__ void put_codes(float* v, const float* eff, uint32_t* lw) {
    static_assert(!RESID || CODEC == kCodecInt4Single || CODEC == kCodecInt4Grouped ||
                      CODEC == kCodecTQ3,
                  "in-place residual only for the INT4 codecs and TQ3");
    float y[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        if constexpr (FAST) y[g] = 1.0f / eff[g];
        else y[g] = 0.0f;
    }
    if constexpr (CODEC == kCodecInt4Single) {  // int4.rs:9-24
#pragma unroll
        for (int d = 0; d < 128; ++d) {
            const int32_t q = clampi(rs_round_i32(quot<FAST>(v[d], eff[0], y[0])), -8, 7);
            put_bits(lw, 4 * d, (uint32_t)(q + 8) & 0xFu);
            if constexpr (RESID) v[d] = v[d] - (float)q * eff[0];
        }
    } else if constexpr (CODEC == kCodecInt4Grouped || CODEC == kCodecNF4 ||
                         CODEC == kCodecTQ3) {  // int4.rs:52-60, nf4.rs:44-54, tq3.rs:31-46
#pragma unroll
        for (int g = 0; g < 8; ++g) {
#pragma unroll
            for (int d = 16 * g; d < 16 * g + 16; ++d) {
                const float t = quot<FAST>(v[d], eff[g], y[g]);
                if constexpr (CODEC == kCodecInt4Grouped) {
                    const int32_t q = clampi(rs_round_i32(t), -8, 7);
                    put_bits(lw, 4 * d, (uint32_t)(q + 8) & 0xFu);
                    if constexpr (RESID) v[d] = v[d] - (float)q * eff[g];
                } else if constexpr (CODEC == kCodecNF4) {
                    put_bits(lw, 4 * d, nf4_nearest(eff[g] > 0.0f ? rs_clampf(t, -1.0f, 1.0f) : 0.0f));
                } else {
                    const float level = tq3_put(lw, 0, 384, d, t);
                    if constexpr (RESID) v[d] = v[d] - level * eff[g];
                }
            }
        }
    } else {  // mixed.rs:38-55, mix3.rs:36-60
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            const int32_t q = rs_round_i32(quot<FAST>(v[d], eff[0], y[0]));
            put_bits(lw, 8 * d, (uint32_t)(clampi(q, -128, 127) + 128));
        }
#pragma unroll
        for (int g = 0; g < 7; ++g) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int ld = 16 * g + i;
                const float t = quot<FAST>(v[8 + ld], eff[1 + g], y[1 + g]);
                if constexpr (CODEC == kCodecMixed) {
                    const int32_t q = rs_round_i32(t);
                    put_bits(lw, 64 + 4 * ld, (uint32_t)(clampi(q, -8, 7) + 8) & 0xFu);
                } else {
                    tq3_put(lw, 64, 400, ld, t);
                }
            }
        }
    }
}

template <int CODEC>
__device__ __forceinline__ float dequant_dim(const uint32_t* lw, const uint32_t* gsw, float scale,
                                             int d);

// Quantise v into (lw, scale, gsw); returns the codec flag. The codes come
// from the three-operation quotient when every scale of the key is in its
// range (nearly always), else from the division; both give the same bits.
// RESID: v is replaced by the residual v - dequant (tile.rs:141-246), in the
// code loop for the INT4 codecs and TQ3 and by dequant_dim for the others.
template <int CODEC, bool RESID>
__device__ __forceinline__ uint32_t quantize_impl(float* v, uint32_t* lw, float* scale_out,
                                                  uint32_t* gsw) {
    constexpr bool kInPlace =
        CODEC == kCodecInt4Single || CODEC == kCodecInt4Grouped || CODEC == kCodecTQ3;
#pragma unroll
    for (int i = 0; i < 16; ++i) lw[i] = 0u;
    float steps[8], eff[8];
    float global;
    uint32_t flag;
    if constexpr (CODEC == kCodecInt4Single) {  // int4.rs:9-24
        const float max_abs = absmax<0, 128>(v);
        global = max_abs > 0.0f ? max_abs / 7.0f : 1.0f;
        gsw[0] = gsw[1] = 0xFFFFFFFFu;
#pragma unroll
        for (int g = 0; g < 8; ++g) eff[g] = global;
        flag = 0u;
    } else if constexpr (CODEC == kCodecInt4Grouped || CODEC == kCodecNF4 ||
                         CODEC == kCodecTQ3) {  // int4.rs:34-63, nf4.rs:23-57, tq3.rs:10-49
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            float m = 0.0f;
#pragma unroll
            for (int d = 16 * g; d < 16 * g + 16; ++d) m = fmaxf(m, fabsf(v[d]));
            steps[g] = CODEC == kCodecInt4Grouped ? m / 7.0f
                       : CODEC == kCodecNF4       ? m
                                                  : m / 3.5f;
        }
        global = group_bytes(steps, gsw);
#pragma unroll
        for (int g = 0; g < 8; ++g) eff[g] = global * (gs_at(gsw, g) / 255.0f);
        flag = CODEC == kCodecInt4Grouped ? 0u : (CODEC == kCodecNF4 ? kFlagNF4 : kFlagTQ3);
    } else {  // mixed.rs:13-57, mix3.rs:11-62
        steps[0] = absmax<0, 8>(v) / 127.0f;
#pragma unroll
        for (int g = 0; g < 7; ++g) {
            float m = 0.0f;
#pragma unroll
            for (int d = 8 + 16 * g; d < 24 + 16 * g; ++d) m = fmaxf(m, fabsf(v[d]));
            steps[1 + g] = CODEC == kCodecMixed ? m / 7.0f : m / 3.5f;
        }
        global = group_bytes(steps, gsw);
#pragma unroll
        for (int g = 0; g < 8; ++g) eff[g] = global * (gs_at(gsw, g) / 255.0f);
        flag = CODEC == kCodecMixed ? kFlagMixed : kFlagMix3;
    }
    bool fast = true;
#pragma unroll
    for (int g = 0; g < 8; ++g) fast = fast && quot_fast_ok(eff[g]);
    if (fast)
        put_codes<CODEC, true, RESID && kInPlace>(v, eff, lw);
    else
        put_codes<CODEC, false, RESID && kInPlace>(v, eff, lw);
    if constexpr (RESID && !kInPlace) {
#pragma unroll
        for (int d = 0; d < kDC; ++d) v[d] = v[d] - dequant_dim<CODEC>(lw, gsw, global, d);
    }
    *scale_out = global;
    return flag;
}
template <int CODEC>
__device__ __forceinline__ uint32_t quantize(const float* v, uint32_t* lw, float* scale_out,
                                             uint32_t* gsw) {
    return quantize_impl<CODEC, false>(const_cast<float*>(v), lw, scale_out, gsw);  // v unchanged
}

// Exact dequant of dim d for a statically known codec (tile.rs:141-246).
template <int CODEC>
__device__ __forceinline__ float dequant_dim(const uint32_t* lw, const uint32_t* gsw, float scale,
                                             int d) {
    if constexpr (CODEC == kCodecInt4Single || CODEC == kCodecInt4Grouped) {
        return (float)((int)nib_at(lw, d) - 8) * group_scale_exact(scale, gs_at(gsw, d / 16));
    } else if constexpr (CODEC == kCodecNF4) {
        return nf4_level(nib_at(lw, d)) * group_scale_exact(scale, gs_at(gsw, d / 16));
    } else if constexpr (CODEC == kCodecTQ3) {
        return tq3_level_exact(lw, 0, 384, d, false) * group_scale_exact(scale, gs_at(gsw, d / 16));
    } else {
        if (d < 8) return (float)((int)byte_at(lw, d) - 128) * section_scale_exact(scale, gs_at(gsw, 0));
        if (d >= 120) return 0.0f;
        const int ld = d - 8;
        const float sec = section_scale_exact(scale, gs_at(gsw, 1 + ld / 16));
        if constexpr (CODEC == kCodecMixed)
            return (float)((int)nib_at(lw, 16 + ld) - 8) * sec;
        else
            return tq3_level_exact(lw, 64, 400, ld, false) * sec;
    }
}

// Orthonormal FWHT of 128 register values (incoherence.rs:45-70), after the
// +-1 diagonal (incoherence.rs:114-125). Butterflies of one stage are
// independent, so evaluating them in register order is bit-identical.
__device__ __forceinline__ void rht128(float* v, const float* __restrict__ diag, float inv) {
#pragma unroll
    for (int i = 0; i < 128; ++i) v[i] *= diag[i];
#pragma unroll
    for (int h = 1; h < 128; h <<= 1) {
#pragma unroll
        for (int i = 0; i < 128; i += 2 * h) {
#pragma unroll
            for (int j = i; j < i + h; ++j) {
                const float a = v[j], b = v[j + h];
                v[j] = a + b;
                v[j + h] = a - b;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 128; ++i) v[i] *= inv;
}

// Packed sign(Z v) (scenario.rs:70-83): bit s = (sum_k Z[s][k] * v[k] < 0),
// sequential f32 from 0.0 with no contraction. Z rows are wave-uniform and are
// read through the scalar cache.
__device__ __forceinline__ void sign_bits_exact(const float* v, const float* __restrict__ z,
                                                uint32_t* bits) {
    // Four rows at a time: four independent sequential accumulation chains
    // give the VALU instruction-level parallelism without changing any
    // row's own operation order.
#pragma unroll
    for (int wd = 0; wd < 8; ++wd) {
        uint32_t word = 0u;
        for (int b = 0; b < 32; b += 4) {
            const float* zr = z + (size_t)(32 * wd + b) * kDC;
            float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
            for (int k = 0; k < kDC; ++k) {
                const float x = v[k];
                a0 += zr[k] * x;
                a1 += zr[kDC + k] * x;
                a2 += zr[2 * kDC + k] * x;
                a3 += zr[3 * kDC + k] * x;
            }
            word |= ((a0 < 0.0f ? 1u : 0u) | (a1 < 0.0f ? 2u : 0u) | (a2 < 0.0f ? 4u : 0u) |
                     (a3 < 0.0f ? 8u : 0u))
                    << b;
        }
        bits[wd] = word;
    }
}

__device__ __forceinline__ void load_vec128(const void* __restrict__ src, int dtype, size_t idx,
                                            float* v) {
    if (dtype == kDtypeBF16) {
        const uint4* p = reinterpret_cast<const uint4*>(src) + idx * 16;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint4 x = p[j];
            const uint32_t u[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                v[8 * j + 2 * k] = __uint_as_float(u[k] << 16);
                v[8 * j + 2 * k + 1] = __uint_as_float(u[k] & 0xFFFF0000u);
            }
        }
    } else {
        const float4* p = reinterpret_cast<const float4*>(src) + idx * 32;
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const float4 x = p[j];
            v[4 * j] = x.x;
            v[4 * j + 1] = x.y;
            v[4 * j + 2] = x.z;
            v[4 * j + 3] = x.w;
        }
    }
}

// Tile encode, mode R (e = key - dequant) or mode Z (e = 0). One lane per key.
template <int CODEC>
__global__ __launch_bounds__(256) void encode_kernel(const void* __restrict__ keys, int dtype,
                                                     uint64_t n_keys, uint32_t n_tok,
                                                     uint32_t n_kv, uint32_t pos0,
                                                     int residual_mode, int warm,
                                                     const float* __restrict__ z,
                                                     const float* __restrict__ diag,
                                                     float lambda_c, float rht_inv,
                                                     uint4* __restrict__ tiles) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_keys) return;
    const uint32_t row = (uint32_t)(i / n_tok);
    const uint32_t t = (uint32_t)(i - (uint64_t)row * n_tok);

    float v[kDC];
    load_vec128(keys, dtype, i, v);

    uint32_t lw[16], gsw[2];
    float scale;
    const uint32_t codec_flag = quantize<CODEC>(v, lw, &scale, gsw);

    uint32_t bits[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float sigma = 0.0f, lambda = 0.0f;
    if (residual_mode == kResidualR) {
        double acc = 0.0;
#pragma unroll
        for (int d = 0; d < kDC; ++d) {
            v[d] = v[d] - dequant_dim<CODEC>(lw, gsw, scale, d);
            const double x = (double)v[d];
            acc = fma(x, x, acc);  // x*x is exact in f64, so this equals acc + x*x
        }
        // Every v[d] is finite iff acc is: 128 squares of finite f32 values sum
        // to at most 2^263, while an inf or NaN v[d] makes acc inf or NaN.
        const bool finite = isfinite(acc);
        sigma = finite ? (float)sqrt(acc / 128.0) : __uint_as_float(0x7FC00000u);  // metrics.rs:207-226
        lambda = sigma * lambda_c;
        if (diag) rht128(v, diag, rht_inv);
        sign_bits_exact(v, z, bits);
    }

    const uint32_t flags = codec_flag | (warm ? kFlagWarm : 0u);
    const uint32_t pos = pos0 + t;
    uint4* out = tiles + i * 8;
    out[0] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    out[1] = make_uint4(lw[4], lw[5], lw[6], lw[7]);
    out[2] = make_uint4(lw[8], lw[9], lw[10], lw[11]);
    out[3] = make_uint4(lw[12], lw[13], lw[14], lw[15]);
    out[4] = make_uint4(bits[0], bits[1], bits[2], bits[3]);
    out[5] = make_uint4(bits[4], bits[5], bits[6], bits[7]);
    out[6] = make_uint4(__float_as_uint(scale), __float_as_uint(lambda), __float_as_uint(sigma), pos);
    out[7] = make_uint4(pos, (row % n_kv) | (flags << 16), gsw[0], gsw[1]);
}

// ---------------------------------------------------------------------------
// Encode, mode R, with the sign sketch on MFMA.
//
// Bit s of the sketch is (p_seq < 0), where p_seq = sum_k Z[s][k] v[k] is the
// reference's sequential f32 sum (scenario.rs:70-83). The kernel approximates
// every projection of a wave's 64 keys with v_mfma_f32_16x16x32_bf16 on a
// two-term RNE bf16 split of both operands, v = vh + vm + rv and
// z = zh + zm + rz with |rv| <= 2^-16 |v|, |rz| <= 2^-16 |z|:
//     p~ = sum_k (zh vh + zh vm + zm vh)
// With S = sum_k |z_k v_k| <= ||z_s|| ||v||, |p~ - p_seq| is at most
//     dropped split terms        3.04 * 2^-16 * S        = 4.64e-5 S
//     MFMA f32 accumulation      384 * 2^-22 * 1.016 S   = 9.30e-5 S
//                                (384 exact bf16 products; twice the f32
//                                 unit per addition, for any summation order)
//     reference sequential sum   gamma_128 = 7.63e-6 S
// which kEncCertRel = 1.5e-4 covers, plus 2^-100 for underflow. A bit whose
// |p~| does not exceed the bound is marked uncertain and recomputed by the
// key's own lane with the reference's sequential sum over the exact v (kept
// in LDS), so every bit equals the reference's. With N(0,1)-like residuals a
// key has about 0.4 uncertain bits. Keys with a non-finite or huge residual
// (|v| > 2^100) have all 256 bits recomputed.
//
// Layout: one workgroup of 4 waves, one key per lane for the codec part (the
// same code as encode_kernel), then per wave a 16x16x32 MFMA grid with Z rows
// as M (16 rows per block sb) and the wave's keys as N (16 per block kb):
// lane L (c = L%16, g = L/16) supplies row m = c of row block sb and column
// 16kb+c of v for dims 32ks+8g..+7, and receives p~ for rows 4g+r, r = 0..3,
// of key 16kb+c. Row m of block sb is sign bit 32(sb/2) + 8(m/4) + 4(sb%2) +
// m%4, so the lane's 16 row blocks give byte g of each of the key's 8 words.

constexpr uint32_t kEncQueue = 256;  // queued (key, bit) recomputations per wave
constexpr uint32_t kEncZAhead = 2;   // Z row blocks in flight ahead of the MFMAs (divides 8)
static_assert(8u % kEncZAhead == 0u, "the sign registers move to slo / clo after row block 7");
constexpr uint32_t kEncQueueKey = 32;  // keys with more uncertain bits keep them

struct EncWaveLds {
    float v[64 * kDC];       // exact v, row = key, 16-B chunk q at q ^ (key & 7)
    uint32_t bits[64 * 8];   // sketch words of each key
    uint32_t umask[64 * 8];  // uncertain bits of each key
    float bound[64];         // certification bound (< 0: all bits certain, inf: none)
    uint32_t queue[kEncQueue];  // (key << 8) | bit
};

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float* enc_chunk(EncWaveLds& w, uint32_t key, uint32_t q) {
    return &w.v[key * kDC + 4u * (q ^ (key & 7u))];
}

// Bit s of one key with the reference's arithmetic: sequential f32 sum from
// 0.0 of Z[s][k] * v[k], k = 0..127, no contraction (scenario.rs:70-83).
__device__ __forceinline__ uint32_t enc_exact_bit(EncWaveLds& w, uint32_t key,
                                                  const float* __restrict__ zrow) {
    const float4* zr = reinterpret_cast<const float4*>(zrow);
    float acc = 0.0f;
#pragma unroll 4
    for (uint32_t q = 0; q < 32; ++q) {
        const float4 x = *reinterpret_cast<const float4*>(enc_chunk(w, key, q));
        const float4 zz = zr[q];
        acc += zz.x * x.x;
        acc += zz.y * x.y;
        acc += zz.z * x.z;
        acc += zz.w * x.w;
    }
    return acc < 0.0f ? 1u : 0u;
}


// RNE bf16 split of two floats: hi = bf16(a, b), mid = bf16((a, b) - hi).
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi, uint32_t& mid) {
    const v2f x = {a, b};
    hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(x, v2bf));
    const v2f r = {a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xFFFF0000u)};
    mid = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, v2bf));
}

template <int CODEC>
__global__ __launch_bounds__(256) void encode_mfma_kernel(
    const void* __restrict__ keys, int dtype, uint64_t n_keys, uint32_t n_tok, uint32_t n_kv,
    uint32_t pos0, int warm, const float* __restrict__ z, const uint4* __restrict__ zpack,
    float cert_scale, const float* __restrict__ diag, float lambda_c, float rht_inv,
    uint4* __restrict__ tiles) {
    __shared__ __align__(16) EncWaveLds lds_all[4];
    const uint32_t lane = threadIdx.x & 63u;
    EncWaveLds& W = lds_all[threadIdx.x >> 6];
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const bool valid = i < n_keys;

    // Codec part, one lane per key: identical arithmetic to encode_kernel.
    {
        float v[kDC];
        float bound = -1.0f;
        bool full = false;
        if (valid) {
            const uint32_t row = (uint32_t)(i / n_tok);
            const uint32_t t = (uint32_t)(i - (uint64_t)row * n_tok);
            load_vec128(keys, dtype, i, v);
            uint32_t lw[16], gsw[2];
            float scale;
            // v becomes the residual e = key - dequant (mode R)
            const uint32_t codec_flag = quantize_impl<CODEC, true>(v, lw, &scale, gsw);
            double acc = 0.0;
#pragma unroll
            for (int d = 0; d < kDC; ++d) {
                const double x = (double)v[d];
                acc = fma(x, x, acc);
            }
            const bool finite = isfinite(acc);  // as in encode_kernel
            const float sigma = finite ? (float)sqrt(acc / 128.0) : __uint_as_float(0x7FC00000u);
            if (diag) rht128(v, diag, rht_inv);
            // ||RHT(e)|| = ||e|| up to ~2^-20; the 2^-10 margin covers it and
            // the rounding of this bound.
            const float nv = (float)sqrt(acc);
            if (!finite || !(nv <= 0x1p100f)) {
                full = true;
            } else if (acc > 0.0) {
                bound = nv * 1.0009765625f * cert_scale + 0x1p-100f;
            }  // acc == 0: v is all +-0, every sum is +0 and every bit 0
            const uint32_t flags = codec_flag | (warm ? kFlagWarm : 0u);
            const uint32_t pos = pos0 + t;
            uint4* out = tiles + i * 8;
            out[0] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
            out[1] = make_uint4(lw[4], lw[5], lw[6], lw[7]);
            out[2] = make_uint4(lw[8], lw[9], lw[10], lw[11]);
            out[3] = make_uint4(lw[12], lw[13], lw[14], lw[15]);
            out[6] = make_uint4(__float_as_uint(scale), __float_as_uint(sigma * lambda_c),
                                __float_as_uint(sigma), pos);
            out[7] = make_uint4(pos, (row % n_kv) | (flags << 16), gsw[0], gsw[1]);
        } else {
#pragma unroll
            for (int d = 0; d < kDC; ++d) v[d] = 0.0f;
        }
#pragma unroll
        for (uint32_t q = 0; q < 32; ++q)
            *reinterpret_cast<float4*>(enc_chunk(W, lane, q)) =
                make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
        W.bound[lane] = full ? INFINITY : bound;
    }
    __syncthreads();

    // MFMA part.
    const uint32_t c = lane & 15u, g = lane >> 4;
    uint32_t bh[4][4][4], bm[4][4][4];  // [kb][ks][dword] of the B operands
    float bk[4];
#pragma unroll
    for (uint32_t kb = 0; kb < 4; ++kb) {
        const uint32_t key = 16u * kb + c;
        bk[kb] = W.bound[key];
#pragma unroll
        for (uint32_t ks = 0; ks < 4; ++ks) {
            const float4 x0 = *reinterpret_cast<const float4*>(enc_chunk(W, key, 8u * ks + 2u * g));
            const float4 x1 = *reinterpret_cast<const float4*>(enc_chunk(W, key, 8u * ks + 2u * g + 1u));
            split2(x0.x, x0.y, bh[kb][ks][0], bm[kb][ks][0]);
            split2(x0.z, x0.w, bh[kb][ks][1], bm[kb][ks][1]);
            split2(x1.x, x1.y, bh[kb][ks][2], bm[kb][ks][2]);
            split2(x1.z, x1.w, bh[kb][ks][3], bm[kb][ks][3]);
        }
    }
    const uint4* zp = zpack + lane;
    // Per key block, one funnel shift per projection pushes its sign bit into
    // sr and its certainty bit into cr; after row blocks 0-7 the registers
    // move to slo / clo and row blocks 8-15 refill them. Bit
    // 31 - (4 (sb % 8) + r) then holds row r of row block sb.
    uint32_t sr[4] = {0u, 0u, 0u, 0u}, slo[4] = {0u, 0u, 0u, 0u};
    uint32_t cr[4] = {0u, 0u, 0u, 0u}, clo[4] = {0u, 0u, 0u, 0u};
    // Z operands of kEncZAhead row blocks in flight: block sb's 8 loads go
    // out kEncZAhead blocks before it is multiplied, so their L2 latency is
    // covered by that many blocks of MFMAs (the kernel runs one wave per SIMD,
    // so no other wave hides it). The ring is indexed statically inside the
    // unrolled inner loop.
    uint4 zr[kEncZAhead][8];
#pragma unroll
    for (uint32_t j = 0; j < kEncZAhead; ++j)
#pragma unroll
        for (uint32_t o = 0; o < 8; ++o) zr[j][o] = zp[(j * 8u + o) * 64u];
    for (uint32_t sb0 = 0; sb0 < 16; sb0 += kEncZAhead) {
#pragma unroll
        for (uint32_t j = 0; j < kEncZAhead; ++j) {
            const uint32_t sb = sb0 + j;
            v4f acc[4];
#pragma unroll
            for (uint32_t kb = 0; kb < 4; ++kb) acc[kb] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
            // Four independent accumulation chains, interleaved.
#pragma unroll
            for (uint32_t ks = 0; ks < 4; ++ks) {
                const v8bf a_h = __builtin_bit_cast(v8bf, zr[j][2 * ks]);
                const v8bf a_m = __builtin_bit_cast(v8bf, zr[j][2 * ks + 1]);
#pragma unroll
                for (uint32_t kb = 0; kb < 4; ++kb) {
                    const v8bf b_h = __builtin_bit_cast(
                        v8bf, make_uint4(bh[kb][ks][0], bh[kb][ks][1], bh[kb][ks][2], bh[kb][ks][3]));
                    acc[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_h, b_h, acc[kb], 0, 0, 0);
                }
#pragma unroll
                for (uint32_t kb = 0; kb < 4; ++kb) {
                    const v8bf b_m = __builtin_bit_cast(
                        v8bf, make_uint4(bm[kb][ks][0], bm[kb][ks][1], bm[kb][ks][2], bm[kb][ks][3]));
                    acc[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_h, b_m, acc[kb], 0, 0, 0);
                }
#pragma unroll
                for (uint32_t kb = 0; kb < 4; ++kb) {
                    const v8bf b_h = __builtin_bit_cast(
                        v8bf, make_uint4(bh[kb][ks][0], bh[kb][ks][1], bh[kb][ks][2], bh[kb][ks][3]));
                    acc[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_m, b_h, acc[kb], 0, 0, 0);
                }
            }
            // Refill this slot with block sb + kEncZAhead; the barrier keeps
            // the loads here instead of next to their use.
            if (sb + kEncZAhead < 16u) {
#pragma unroll
                for (uint32_t o = 0; o < 8; ++o) zr[j][o] = zp[((sb + kEncZAhead) * 8u + o) * 64u];
            }
            __builtin_amdgcn_sched_barrier(0);
            // Certain: |p~| > bound, i.e. bound - |p~| < 0 (bound >= 2^-100 or
            // < 0, so a nonzero difference never rounds to 0). A certain p~ is
            // nonzero, so its sign bit is (p~ < 0); an uncertain one is
            // recomputed below whatever its bit. NaN differences occur only
            // for keys whose bits are all recomputed (bound = inf).
#pragma unroll
            for (uint32_t kb = 0; kb < 4; ++kb)
#pragma unroll
                for (uint32_t r = 0; r < 4; ++r) {
                    sr[kb] = __builtin_amdgcn_alignbit(sr[kb], __float_as_uint(acc[kb][r]), 31);
                    cr[kb] = __builtin_amdgcn_alignbit(
                        cr[kb], __float_as_uint(bk[kb] - fabsf(acc[kb][r])), 31);
                }
        }
        if (sb0 + kEncZAhead == 8u) {
#pragma unroll
            for (uint32_t kb = 0; kb < 4; ++kb) {
                slo[kb] = sr[kb];
                clo[kb] = cr[kb];
            }
        }
    }
    // Lane (g, c) holds byte g of every sketch word of key 16 kb + c (the
    // row order of the Z pack, build_projection_pack): bytes 0-3 of the
    // bit-reversed slo / clo are words 0-3, those of sr / cr words 4-7. Every
    // byte of W.bits and W.umask is written here. A key whose residual is all
    // +-0 (bound < 0) gets bits 0, as every sequential sum is +0; a key with
    // bound = inf has every bit uncertain.
    uint8_t* bbytes = reinterpret_cast<uint8_t*>(W.bits);
    uint8_t* ubytes = reinterpret_cast<uint8_t*>(W.umask);
#pragma unroll
    for (uint32_t kb = 0; kb < 4; ++kb) {
        const bool zero = bk[kb] < 0.0f, full = bk[kb] == INFINITY;
        const uint32_t s0 = zero ? 0u : __builtin_bitreverse32(slo[kb]);
        const uint32_t s1 = zero ? 0u : __builtin_bitreverse32(sr[kb]);
        const uint32_t u0 = full ? 0xFFFFFFFFu : ~__builtin_bitreverse32(clo[kb]);
        const uint32_t u1 = full ? 0xFFFFFFFFu : ~__builtin_bitreverse32(cr[kb]);
        const uint32_t o = (16u * kb + c) * 32u + g;
#pragma unroll
        for (uint32_t w = 0; w < 4; ++w) {
            bbytes[o + 4u * w] = (uint8_t)(s0 >> (8u * w));
            bbytes[o + 16u + 4u * w] = (uint8_t)(s1 >> (8u * w));
            ubytes[o + 4u * w] = (uint8_t)(u0 >> (8u * w));
            ubytes[o + 16u + 4u * w] = (uint8_t)(u1 >> (8u * w));
        }
    }
    __syncthreads();

    // Uncertain bits. Keys with at most kEncQueueKey of them (nearly all)
    // queue their (key, bit) pairs, and the queue is spread over the wave's
    // lanes; a key with more (non-finite or huge residual), or whose pairs do
    // not fit, is finished by its own lane.
    const uint4 u0 = *reinterpret_cast<const uint4*>(&W.umask[lane * 8]);
    const uint4 u1 = *reinterpret_cast<const uint4*>(&W.umask[lane * 8 + 4]);
    const uint32_t um[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
    uint32_t n = 0u;
#pragma unroll
    for (uint32_t w = 0; w < 8; ++w) n += __builtin_popcount(um[w]);
    const uint32_t nq = n <= kEncQueueKey ? n : 0u;
    const uint32_t incl = wave_inclusive_sum(nq);
    const bool queued = incl <= kEncQueue;
    const unsigned long long fit = __ballot(queued);  // lanes 0.. (incl is monotonic)
    const uint32_t total =
        fit ? (uint32_t)__builtin_amdgcn_readlane((int)incl, __popcll(fit) - 1) : 0u;
    if (queued && nq != 0u) {
        uint32_t e = incl - nq;
#pragma unroll
        for (uint32_t w = 0; w < 8; ++w) {
            uint32_t m = um[w];
            while (m != 0u) {
                const uint32_t r = __builtin_ctz(m);
                m &= m - 1u;
                W.queue[e++] = (lane << 8) | (32u * w + r);
            }
        }
    }
    __syncthreads();
    for (uint32_t e = lane; e < total; e += 64u) {
        const uint32_t ent = W.queue[e];
        const uint32_t key = ent >> 8, sbit = ent & 255u;
        const uint32_t m = 1u << (sbit & 31u);
        uint32_t* word = &W.bits[key * 8u + (sbit >> 5)];
        if (enc_exact_bit(W, key, z + (size_t)sbit * kDC))
            atomicOr(word, m);
        else
            atomicAnd(word, ~m);
    }
    __syncthreads();
    if (!valid) return;
    const uint4 b0 = *reinterpret_cast<const uint4*>(&W.bits[lane * 8]);
    const uint4 b1 = *reinterpret_cast<const uint4*>(&W.bits[lane * 8 + 4]);
    uint32_t bits[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
    if (!queued || n > kEncQueueKey) {
#pragma unroll
        for (uint32_t w = 0; w < 8; ++w) {
            uint32_t m = um[w];
            while (m != 0u) {
                const uint32_t r = __builtin_ctz(m);
                m &= m - 1u;
                const uint32_t b = enc_exact_bit(W, lane, z + (size_t)(32u * w + r) * kDC);
                bits[w] = (bits[w] & ~(1u << r)) | (b << r);
            }
        }
    }
    uint4* out = tiles + i * 8;
    out[4] = make_uint4(bits[0], bits[1], bits[2], bits[3]);
    out[5] = make_uint4(bits[4], bits[5], bits[6], bits[7]);
}

// Query preparation: q_coarse = q, q_sign = sign(Z * RHT(q)). One workgroup
// per query and one lane per sign row: every lane forms RHT(q) with identical
// arithmetic, lane s accumulates row s of Z in the reference order
// (sequential f32 from 0.0, no contraction), and a wave ballot packs the 64
// bits of one q_sign word.
__global__ __launch_bounds__(256) void prepare_query_kernel(const void* __restrict__ q, int dtype,
                                                            const float* __restrict__ z,
                                                            const float* __restrict__ diag,
                                                            float rht_inv, float* __restrict__ qc,
                                                            uint64_t* __restrict__ qs) {
    const size_t i = blockIdx.x;
    const uint32_t row = threadIdx.x;
    if (row < kDC) {
        qc[i * kDC + row] = dtype == kDtypeBF16
                                ? __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(q)[i * kDC + row] << 16)
                                : reinterpret_cast<const float*>(q)[i * kDC + row];
    }
    float v[kDC];
    load_vec128(q, dtype, i, v);
    if (diag) rht128(v, diag, rht_inv);
    const float4* zr = reinterpret_cast<const float4*>(z + (size_t)row * kDC);
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < kDC / 4; ++k) {
        const float4 zz = zr[k];
        acc += zz.x * v[4 * k];
        acc += zz.y * v[4 * k + 1];
        acc += zz.z * v[4 * k + 2];
        acc += zz.w * v[4 * k + 3];
    }
    const uint64_t word = __ballot(acc < 0.0f);
    if ((row & 63u) == 0) qs[i * 4 + (row >> 6)] = word;
}

// Decode: dequant_latent (tile.rs:249-255); optionally add the sign-sketch
// residual estimate of reconstruct_from_tile (learned.rs:283-321, identity
// latent, no RHT): key[i] += (+-1 * scale_r) * Z[s][i] in s order.
__global__ __launch_bounds__(256) void decode_kernel(const uint4* __restrict__ tiles, uint64_t n,
                                                     const float* __restrict__ z,
                                                     float sqrt_half_pi, float* __restrict__ out) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint32_t w[32];
    load_tile(tiles + i * 8, w);
    const uint32_t flags = w[29] >> 16;
    float k[kDC];
    dequant_exact(w, w + 30, __uint_as_float(w[24]), flags, k);
    if (z) {
        const float sc = __uint_as_float(w[26]) * sqrt_half_pi / 256.0f;
        for (int s = 0; s < kDS; ++s) {
            const float sgn = ((w[16 + (s >> 5)] >> (s & 31)) & 1u) ? -1.0f : 1.0f;
            const float f = sgn * sc;
            const float* zr = z + (size_t)s * kDC;
#pragma unroll
            for (int d = 0; d < kDC; ++d) k[d] += f * zr[d];
        }
    }
    float4* o = reinterpret_cast<float4*>(out) + i * 32;
#pragma unroll
    for (int j = 0; j < 32; ++j) o[j] = make_float4(k[4 * j], k[4 * j + 1], k[4 * j + 2], k[4 * j + 3]);
}

// Validation (slha-c/src/lib.rs:244-286). Records the lowest failing index.
__global__ __launch_bounds__(256) void validate_kernel(const uint4* __restrict__ tiles, uint64_t n,
                                                       unsigned long long* __restrict__ status) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint4 m0 = tiles[i * 8 + 6];
    const uint4 m1 = tiles[i * 8 + 7];
    const uint32_t flags = m1.y >> 16;
    const float sc = __uint_as_float(m0.x), la = __uint_as_float(m0.y), si = __uint_as_float(m0.z);
    int code = 0;
    if (flags & ~kKnownFlags)
        code = -6;
    else if (__popc(flags & kCodecFlags) > 1)
        code = -6;
    else if ((flags & kFlagNoCorr) && !(flags & (kFlagTQ3 | kFlagMix3)))
        code = -6;
    else if (!isfinite(sc) || !isfinite(la) || !isfinite(si))
        code = -5;
    else if (sc < 0.0f || la < 0.0f || si < 0.0f)
        code = -6;
    if (code != 0) {
        const unsigned long long key = ((unsigned long long)(i + 1) << 8) | (unsigned long long)(-code);
        atomicMin(status, key);
    }
}

// CCOS ladder (ccos.rs:369-438) on device tiles: op 0 page_out, op 1
// drop_correction, op 2 evict (the tile stays, its state becomes COLD). The
// slots are slots[0, n), or the one slot `slot0` when slots is NULL. With a
// state array (0 HOT, 1 WARM, 2 COLD), page_out and evict also write the
// slot's new state.
__global__ __launch_bounds__(256) void ccos_apply_kernel(uint4* __restrict__ tiles,
                                                         uint8_t* __restrict__ state,
                                                         const uint32_t* __restrict__ slots,
                                                         uint32_t slot0, uint64_t n, int op) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t slot = slots ? slots[i] : slot0;
    if (op == 2) {
        if (state) state[slot] = 2;
        return;
    }
    if (op == 0 && state) state[slot] = 1;
    uint4* t = tiles + (size_t)slot * 8;
    uint4 m0 = t[6], m1 = t[7];
    uint32_t flags = m1.y >> 16;
    if (op == 0) {  // page_out: residual := 0, lambda := 0, |WARM
        t[4] = make_uint4(0, 0, 0, 0);
        t[5] = make_uint4(0, 0, 0, 0);
        m0.y = 0u;
        flags |= kFlagWarm;
        t[6] = m0;
    } else {  // drop_correction
        const int nb = (flags & kFlagTQ3) ? 16 : ((flags & kFlagMix3) ? 14 : 0);
        if (nb == 0 || (flags & kFlagNoCorr)) return;
        uint4 l3 = t[3];  // latent bytes 48..63
        if (nb == 16) {
            l3 = make_uint4(0, 0, 0, 0);
        } else {  // bytes 50..63: keep bytes 48, 49
            l3.x &= 0x0000FFFFu;
            l3.y = l3.z = l3.w = 0u;
        }
        t[3] = l3;
        flags |= kFlagNoCorr;
    }
    m1.y = (m1.y & 0xFFFFu) | (flags << 16);
    t[7] = m1;
}

// ---------------------------------------------------------------------------
// Learned models (d > 128): LearnedModel built from a .slhw projection
// (learned.rs:218-257, weights.rs:159-270). P is [128][d] row-major with
// per-component scale 1 (so h_k / s_k and h_k * s_k are exact no-ops), Z is
// [256][d_pad] and the optional RHT diagonal is [d_pad], d_pad = next_pow2(d)
// with RHT and d without (incoherence.rs:29-35, 89-98).
//
// One workgroup of 256 threads per vector. Every sum keeps the reference's
// sequential f32 order (mul then add, no contraction), so latent codes, sign
// bits and reconstructions are bit-exact:
//   latent   h_k = sum_i P[k][i] key[i]          thread k < 128   (evec_dot, learned.rs:257-273)
//   recon    r_i = sum_k h_k P[k][i]             one thread per i (reconstruct, learned.rs:276-286)
//   sigma    sqrt((sum_i e_i e_i) / d), f32      thread 0         (encode_with, learned.rs:398)
//   sketch   bit s = (sum_i Z[s][i] buf[i] < 0)  thread s         (sign_bits, learned.rs:326-347)
// where e = key - r and buf = e, or FWHT(diag . pad(e)) / sqrt(d_pad)
// (transform_into, incoherence.rs:114-125; fwht_inplace, :45-70). The FWHT
// runs stage by stage in LDS; each butterfly is the same IEEE add/sub as in
// the sequential loop, so the order of pairs within a stage does not matter.

struct LearnedArgs {
    const float* p;     // [128][d]
    const float* z;     // [256][d_pad]
    const float* diag;  // [d_pad] +-1, or null without RHT
    const float4* p4;   // P interleaved by 4 columns: [ceil(d / 4)][128] float4
    const float4* z4;   // Z interleaved by 4 columns: [ceil(d_pad / 4)][256] float4
    uint32_t d, d_pad;
    float rht_inv;      // 1 / sqrt(d_pad)
};

// Dynamic LDS of the learned kernels: vec[d], buf[d_pad], h[128], 32 words.
__host__ __device__ constexpr size_t learned_lds_bytes(uint32_t d, uint32_t d_pad) {
    return ((size_t)d + d_pad + 128 + 32) * 4;
}

// Sequential f32 dot product sum_i M[r][i] * v[i], i = 0 .. n-1 (v in LDS),
// of row r of an [R][n] matrix (P or Z, read from L2) stored interleaved by
// 4 columns: element (r, i) at m4[(i / 4) R + r], component i % 4, zero past
// n. Lanes holding consecutive rows read consecutive float4s, so each load
// instruction of a wave reads 1 KiB contiguous (a row-major row per lane
// touches 64 cache lines per load). The row is loaded kDotBatch float4s at a
// time, all issued before the batch's sequential adds, so one L2 latency is
// paid per 64 terms; the sum order is unchanged.
constexpr uint32_t kDotBatch = 16;

template <uint32_t R>
__device__ __forceinline__ float seq_dot4(const float4* __restrict__ m4, uint32_t r, const float* v,
                                          uint32_t n) {
    const float4* col = m4 + r;
    float acc = 0.0f;
    uint32_t i = 0;
    for (; i + 4 * kDotBatch <= n; i += 4 * kDotBatch) {
        float4 x[kDotBatch];
#pragma unroll
        for (uint32_t b = 0; b < kDotBatch; ++b) x[b] = col[(size_t)(i / 4 + b) * R];
#pragma unroll
        for (uint32_t b = 0; b < kDotBatch; ++b) {
            const uint32_t j = i + 4 * b;
            acc += x[b].x * v[j];
            acc += x[b].y * v[j + 1];
            acc += x[b].z * v[j + 2];
            acc += x[b].w * v[j + 3];
        }
    }
    for (; i < n; i += 4) {
        const float4 x = col[(size_t)(i / 4) * R];
        acc += x.x * v[i];
        if (i + 1 < n) acc += x.y * v[i + 1];
        if (i + 2 < n) acc += x.z * v[i + 2];
        if (i + 3 < n) acc += x.w * v[i + 3];
    }
    return acc;
}

__device__ __forceinline__ void lds_load_vec(const void* __restrict__ src, int dtype, uint64_t idx,
                                             uint32_t d, float* out) {
    for (uint32_t i = threadIdx.x; i < d; i += blockDim.x)
        out[i] = dtype == kDtypeBF16
                     ? __uint_as_float((uint32_t)static_cast<const uint16_t*>(src)[idx * d + i] << 16)
                     : static_cast<const float*>(src)[idx * d + i];
}

// buf <- FWHT(diag . buf) / sqrt(d_pad), in place in LDS (all threads).
__device__ __forceinline__ void block_rht(float* buf, const float* __restrict__ diag,
                                          uint32_t d_pad, float inv) {
    for (uint32_t i = threadIdx.x; i < d_pad; i += blockDim.x) buf[i] *= diag[i];
    __syncthreads();
    for (uint32_t h = 1; h < d_pad; h <<= 1) {
        for (uint32_t q = threadIdx.x; q < d_pad / 2; q += blockDim.x) {
            const uint32_t j = ((q & ~(h - 1u)) << 1) | (q & (h - 1u));  // pair (j, j + h)
            const float a = buf[j], b = buf[j + h];
            buf[j] = a + b;
            buf[j + h] = a - b;
        }
        __syncthreads();
    }
    for (uint32_t i = threadIdx.x; i < d_pad; i += blockDim.x) buf[i] *= inv;
    __syncthreads();
}

// words[0..7] <- sign bits of Z . buf (bit s = 1 iff the sum is negative);
// thread s computes row s, wave w's ballot is u64 word w. blockDim.x == 256.
__device__ __forceinline__ void block_sign_bits(const float* buf, const float4* __restrict__ z4,
                                                uint32_t d_pad, uint32_t* words) {
    const uint32_t s = threadIdx.x;
    const float acc = seq_dot4<kDS>(z4, s, buf, d_pad);
    const uint64_t m = __ballot(acc < 0.0f);
    if ((s & 63u) == 0) {
        words[2 * (s >> 6)] = (uint32_t)m;
        words[2 * (s >> 6) + 1] = (uint32_t)(m >> 32);
    }
}

// Key -> tile (encode_with, learned.rs:353-408). Keys [n][d]; key i is token
// t = i % n_tok of row i / n_tok: token_id = position = pos0 + t, head_id =
// row % n_kv (head 0 for a single key, as the reference).
template <int CODEC>
__global__ __launch_bounds__(256) void learned_encode_kernel(const void* __restrict__ keys, int dtype,
                                                             uint64_t n_keys, uint32_t n_tok,
                                                             uint32_t n_kv, uint32_t pos0, int warm,
                                                             LearnedArgs a, float lambda_c,
                                                             uint4* __restrict__ tiles) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    float* key = lds;
    float* buf = lds + a.d;
    float* h = buf + a.d_pad;
    uint32_t* misc = reinterpret_cast<uint32_t*>(h + 128);  // sign words 0..7, sigma 8
    const uint32_t tid = threadIdx.x;
    for (uint64_t ki = blockIdx.x; ki < n_keys; ki += gridDim.x) {
        lds_load_vec(keys, dtype, ki, a.d, key);
        __syncthreads();
        if (tid < 128) h[tid] = seq_dot4<128>(a.p4, tid, key, a.d);
        __syncthreads();
        // Residual from the un-quantised latent.
        for (uint32_t i = tid; i < a.d; i += blockDim.x) {
            float r = 0.0f;
            for (uint32_t k = 0; k < 128; ++k) r += h[k] * a.p[(size_t)k * a.d + i];
            buf[i] = key[i] - r;
        }
        for (uint32_t i = a.d + tid; i < a.d_pad; i += blockDim.x) buf[i] = 0.0f;
        __syncthreads();
        if (tid == 0) {
            float acc = 0.0f;
            for (uint32_t i = 0; i < a.d; ++i) acc += buf[i] * buf[i];
            misc[8] = __float_as_uint(sqrtf(acc / (float)a.d));
        }
        __syncthreads();  // sigma has read buf before the RHT rewrites it
        if (a.diag) block_rht(buf, a.diag, a.d_pad, a.rht_inv);
        block_sign_bits(buf, a.z4, a.d_pad, misc);
        __syncthreads();
        if (tid == 0) {
            uint32_t lw[16], gsw[2];
            float scale;
            const uint32_t codec_flag = quantize<CODEC>(h, lw, &scale, gsw);
            const float sigma = __uint_as_float(misc[8]);
            const float lambda = sigma * lambda_c;
            const uint32_t row = (uint32_t)(ki / n_tok);
            const uint32_t pos = pos0 + (uint32_t)(ki - (uint64_t)row * n_tok);
            const uint32_t flags = codec_flag | (warm ? kFlagWarm : 0u);
            uint4* out = tiles + ki * 8;
            out[0] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
            out[1] = make_uint4(lw[4], lw[5], lw[6], lw[7]);
            out[2] = make_uint4(lw[8], lw[9], lw[10], lw[11]);
            out[3] = make_uint4(lw[12], lw[13], lw[14], lw[15]);
            out[4] = make_uint4(misc[0], misc[1], misc[2], misc[3]);
            out[5] = make_uint4(misc[4], misc[5], misc[6], misc[7]);
            out[6] = make_uint4(__float_as_uint(scale), __float_as_uint(lambda), misc[8], pos);
            out[7] = make_uint4(pos, (row % n_kv) | (flags << 16), gsw[0], gsw[1]);
        }
        __syncthreads();
    }
}

// Two keys per workgroup (learned_encode_kernel's steps, each key's sums in
// the same order): threads 0-127 form key 0's latent and 128-255 key 1's;
// every reconstruction and sign-sketch thread runs both keys' chains side by
// side on one load of P or Z. Used when both keys' vectors fit in LDS.
__host__ __device__ constexpr size_t learned_lds_bytes2(uint32_t d, uint32_t d_pad) {
    return (2 * (size_t)d + 2 * (size_t)d_pad + 256 + 64) * 4;
}

constexpr uint32_t kDot2Batch = 8;  // float4s per batch with two chains (register budget)

// seq_dot4 of one row against two vectors, one load of the row for both
// chains (each chain in its own sequential order).
template <uint32_t R>
__device__ __forceinline__ void seq_dot4x2(const float4* __restrict__ m4, uint32_t r, const float* v0,
                                           const float* v1, uint32_t n, float& a0, float& a1) {
    const float4* col = m4 + r;
    float x0 = 0.0f, x1 = 0.0f;
    uint32_t i = 0;
    for (; i + 4 * kDot2Batch <= n; i += 4 * kDot2Batch) {
        float4 x[kDot2Batch];
#pragma unroll
        for (uint32_t b = 0; b < kDot2Batch; ++b) x[b] = col[(size_t)(i / 4 + b) * R];
#pragma unroll
        for (uint32_t b = 0; b < kDot2Batch; ++b) {
            const uint32_t j = i + 4 * b;
            x0 += x[b].x * v0[j];
            x1 += x[b].x * v1[j];
            x0 += x[b].y * v0[j + 1];
            x1 += x[b].y * v1[j + 1];
            x0 += x[b].z * v0[j + 2];
            x1 += x[b].z * v1[j + 2];
            x0 += x[b].w * v0[j + 3];
            x1 += x[b].w * v1[j + 3];
        }
    }
    for (; i < n; i += 4) {
        const float4 x = col[(size_t)(i / 4) * R];
        const float e[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (uint32_t c = 0; c < 4; ++c)
            if (i + c < n) {
                x0 += e[c] * v0[i + c];
                x1 += e[c] * v1[i + c];
            }
    }
    a0 = x0, a1 = x1;
}

// block_rht over two buffers with one set of workgroup barriers.
__device__ __forceinline__ void block_rht2(float* b0, float* b1, const float* __restrict__ diag,
                                           uint32_t d_pad, float inv) {
    for (uint32_t i = threadIdx.x; i < 2 * d_pad; i += blockDim.x) {
        float* b = i < d_pad ? b0 : b1;
        const uint32_t e = i < d_pad ? i : i - d_pad;
        b[e] *= diag[e];
    }
    __syncthreads();
    const uint32_t half = d_pad / 2;
    for (uint32_t h = 1; h < d_pad; h <<= 1) {
        for (uint32_t q2 = threadIdx.x; q2 < 2 * half; q2 += blockDim.x) {
            float* b = q2 < half ? b0 : b1;
            const uint32_t q = q2 < half ? q2 : q2 - half;
            const uint32_t j = ((q & ~(h - 1u)) << 1) | (q & (h - 1u));
            const float x = b[j], y = b[j + h];
            b[j] = x + y;
            b[j + h] = x - y;
        }
        __syncthreads();
    }
    for (uint32_t i = threadIdx.x; i < 2 * d_pad; i += blockDim.x) {
        float* b = i < d_pad ? b0 : b1;
        b[i < d_pad ? i : i - d_pad] *= inv;
    }
    __syncthreads();
}

template <int CODEC>
__global__ __launch_bounds__(256, (CODEC == kCodecInt4Single || CODEC == kCodecInt4Grouped || CODEC == kCodecMixed) ? 3 : 2) void learned_encode2_kernel(const void* __restrict__ keys, int dtype,
                                                              uint64_t n_keys, uint32_t n_tok,
                                                              uint32_t n_kv, uint32_t pos0, int warm,
                                                              LearnedArgs a, float lambda_c,
                                                              uint4* __restrict__ tiles) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    float* key0 = lds;
    float* key1 = key0 + a.d;
    float* buf0 = key1 + a.d;
    float* buf1 = buf0 + a.d_pad;
    float* h0 = buf1 + a.d_pad;
    float* h1 = h0 + 128;
    uint32_t* misc0 = reinterpret_cast<uint32_t*>(h1 + 128);  // sign words 0..7, sigma 8
    uint32_t* misc1 = misc0 + 32;
    const uint32_t tid = threadIdx.x, wave = tid >> 6;
    for (uint64_t k0 = 2 * (uint64_t)blockIdx.x; k0 < n_keys; k0 += 2 * (uint64_t)gridDim.x) {
        const bool two = k0 + 1 < n_keys;  // uniform over the workgroup
        lds_load_vec(keys, dtype, k0, a.d, key0);
        if (two) lds_load_vec(keys, dtype, k0 + 1, a.d, key1);
        __syncthreads();
        if (tid < 128) h0[tid] = seq_dot4<128>(a.p4, tid, key0, a.d);
        else if (two) h1[tid - 128] = seq_dot4<128>(a.p4, tid - 128, key1, a.d);
        __syncthreads();
        for (uint32_t i = tid; i < a.d; i += blockDim.x) {
            float r0 = 0.0f, r1 = 0.0f;
            for (uint32_t k = 0; k < 128; ++k) {
                const float pk = a.p[(size_t)k * a.d + i];
                r0 += h0[k] * pk;
                r1 += h1[k] * pk;
            }
            buf0[i] = key0[i] - r0;
            buf1[i] = key1[i] - r1;
        }
        for (uint32_t i = a.d + tid; i < a.d_pad; i += blockDim.x) buf0[i] = buf1[i] = 0.0f;
        __syncthreads();
        if ((tid & 63u) == 0 && wave < 2) {  // sigma of key `wave` (learned.rs:392-396)
            const float* b = wave == 0 ? buf0 : buf1;
            float acc = 0.0f;
            for (uint32_t i = 0; i < a.d; ++i) acc += b[i] * b[i];
            (wave == 0 ? misc0 : misc1)[8] = __float_as_uint(sqrtf(acc / (float)a.d));
        }
        __syncthreads();
        if (a.diag) block_rht2(buf0, buf1, a.diag, a.d_pad, a.rht_inv);
        {
            float acc0, acc1;
            seq_dot4x2<kDS>(a.z4, tid, buf0, buf1, a.d_pad, acc0, acc1);
            const uint64_t m0 = __ballot(acc0 < 0.0f), m1 = __ballot(acc1 < 0.0f);
            if ((tid & 63u) == 0) {
                misc0[2 * wave] = (uint32_t)m0, misc0[2 * wave + 1] = (uint32_t)(m0 >> 32);
                misc1[2 * wave] = (uint32_t)m1, misc1[2 * wave + 1] = (uint32_t)(m1 >> 32);
            }
        }
        __syncthreads();
        if ((tid & 63u) == 0 && (wave == 0 || (wave == 1 && two))) {
            const uint64_t ki = k0 + wave;
            const float* h = wave == 0 ? h0 : h1;
            const uint32_t* misc = wave == 0 ? misc0 : misc1;
            uint32_t lw[16], gsw[2];
            float scale;
            const uint32_t codec_flag = quantize<CODEC>(h, lw, &scale, gsw);
            const float sigma = __uint_as_float(misc[8]);
            const float lambda = sigma * lambda_c;
            const uint32_t row = (uint32_t)(ki / n_tok);
            const uint32_t pos = pos0 + (uint32_t)(ki - (uint64_t)row * n_tok);
            const uint32_t flags = codec_flag | (warm ? kFlagWarm : 0u);
            uint4* out = tiles + ki * 8;
            out[0] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
            out[1] = make_uint4(lw[4], lw[5], lw[6], lw[7]);
            out[2] = make_uint4(lw[8], lw[9], lw[10], lw[11]);
            out[3] = make_uint4(lw[12], lw[13], lw[14], lw[15]);
            out[4] = make_uint4(misc[0], misc[1], misc[2], misc[3]);
            out[5] = make_uint4(misc[4], misc[5], misc[6], misc[7]);
            out[6] = make_uint4(__float_as_uint(scale), __float_as_uint(lambda), misc[8], pos);
            out[7] = make_uint4(pos, (row % n_kv) | (flags << 16), gsw[0], gsw[1]);
        }
        __syncthreads();
    }
}

// Four keys per workgroup: the steps of learned_encode2_kernel with every
// load of P or Z feeding four keys' chains (each in its own sequential
// order): threads 0-127 form the latents of keys 0 and 1, threads 128-255
// those of keys 2 and 3; each reconstruction and sign-sketch thread runs all
// four. Lanes 0-3 of wave 0 compute the keys' sigmas and quantise them side
// by side. Key slots past n_keys are computed on and not stored. Used while
// the four keys' vectors fit in LDS.
__host__ __device__ constexpr size_t learned_lds_bytes4(uint32_t nk, uint32_t d, uint32_t d_pad) {
    return (nk * ((size_t)d + d_pad + 128 + 32)) * 4;
}

// seq_dot4 of one row against M vectors v + j vstride, one load of the row
// for all M chains (each in its own sequential order), B float4s a batch.
template <uint32_t R, uint32_t M, uint32_t B>
__device__ __forceinline__ void seq_dot4xm(const float4* __restrict__ m4, uint32_t r, const float* v,
                                           uint32_t vstride, uint32_t n, float (&acc)[M]) {
    const float4* col = m4 + r;
    float x[M];
#pragma unroll
    for (uint32_t j = 0; j < M; ++j) x[j] = 0.0f;
    uint32_t i = 0;
    for (; i + 4 * B <= n; i += 4 * B) {
        float4 y[B];
#pragma unroll
        for (uint32_t b = 0; b < B; ++b) y[b] = col[(size_t)(i / 4 + b) * R];
#pragma unroll
        for (uint32_t b = 0; b < B; ++b) {
            const float e[4] = {y[b].x, y[b].y, y[b].z, y[b].w};
#pragma unroll
            for (uint32_t c = 0; c < 4; ++c)
#pragma unroll
                for (uint32_t j = 0; j < M; ++j) x[j] += e[c] * v[j * vstride + i + 4 * b + c];
        }
    }
    for (; i < n; i += 4) {
        const float4 y = col[(size_t)(i / 4) * R];
        const float e[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
        for (uint32_t c = 0; c < 4; ++c)
            if (i + c < n)
#pragma unroll
                for (uint32_t j = 0; j < M; ++j) x[j] += e[c] * v[j * vstride + i + c];
    }
#pragma unroll
    for (uint32_t j = 0; j < M; ++j) acc[j] = x[j];
}

// block_rht over nb contiguous buffers of d_pad floats, one set of barriers.
__device__ __forceinline__ void block_rht_n(float* buf, uint32_t nb, const float* __restrict__ diag,
                                            uint32_t d_pad, float inv) {
    const uint32_t log_pad = 31u - (uint32_t)__builtin_clz(d_pad);
    for (uint32_t i = threadIdx.x; i < nb * d_pad; i += blockDim.x) buf[i] *= diag[i & (d_pad - 1u)];
    __syncthreads();
    const uint32_t half = d_pad / 2;
    for (uint32_t h = 1; h < d_pad; h <<= 1) {
        for (uint32_t q2 = threadIdx.x; q2 < nb * half; q2 += blockDim.x) {
            float* b = buf + ((q2 >> (log_pad - 1u)) << log_pad);
            const uint32_t q = q2 & (half - 1u);
            const uint32_t j = ((q & ~(h - 1u)) << 1) | (q & (h - 1u));
            const float x = b[j], y = b[j + h];
            b[j] = x + y;
            b[j + h] = x - y;
        }
        __syncthreads();
    }
    for (uint32_t i = threadIdx.x; i < nb * d_pad; i += blockDim.x) buf[i] *= inv;
    __syncthreads();
}

constexpr uint32_t kLearnedKeysPerBlock = 4;  // 8 measured slower (1.71 against 1.47 ms at d = 1024)

template <int CODEC>
__global__ __launch_bounds__(256, (CODEC == kCodecInt4Single || CODEC == kCodecInt4Grouped || CODEC == kCodecMixed) ? 3 : 2) void learned_encode4_kernel(const void* __restrict__ keys, int dtype,
                                                              uint64_t n_keys, uint32_t n_tok,
                                                              uint32_t n_kv, uint32_t pos0, int warm,
                                                              LearnedArgs a, float lambda_c,
                                                              uint4* __restrict__ tiles) {
    constexpr uint32_t NK = kLearnedKeysPerBlock;
    extern __shared__ __attribute__((aligned(16))) float lds[];
    float* key = lds;                    // [NK][d]
    float* buf = key + NK * a.d;         // [NK][d_pad]
    float* hs = buf + NK * a.d_pad;      // [NK][128]
    uint32_t* misc = reinterpret_cast<uint32_t*>(hs + NK * 128);  // [NK][32]: sign words 0..7, sigma 8
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
    constexpr uint32_t HK = NK / 2;  // keys per latent half
    for (uint64_t k0 = NK * (uint64_t)blockIdx.x; k0 < n_keys; k0 += NK * (uint64_t)gridDim.x) {
        const uint32_t nk = n_keys - k0 < NK ? (uint32_t)(n_keys - k0) : NK;  // uniform
        for (uint32_t j = 0; j < nk; ++j) lds_load_vec(keys, dtype, k0 + j, a.d, key + j * a.d);
        __syncthreads();
        {
            const uint32_t half = tid >> 7, k = tid & 127u;  // keys HK half .. HK half + HK - 1
            if (HK * half < nk) {
                float h[HK];
                seq_dot4xm<128, HK, (HK > 2 ? 4 : 8)>(a.p4, k, key + HK * half * a.d, a.d, a.d, h);
#pragma unroll
                for (uint32_t j = 0; j < HK; ++j) hs[(HK * half + j) * 128 + k] = h[j];
            }
        }
        __syncthreads();
        for (uint32_t i = tid; i < a.d; i += blockDim.x) {
            float r[NK];
#pragma unroll
            for (uint32_t j = 0; j < NK; ++j) r[j] = 0.0f;
#pragma unroll 4
            for (uint32_t k = 0; k < 128; ++k) {
                const float pk = a.p[(size_t)k * a.d + i];
#pragma unroll
                for (uint32_t j = 0; j < NK; ++j) r[j] += hs[j * 128 + k] * pk;
            }
#pragma unroll
            for (uint32_t j = 0; j < NK; ++j) buf[j * a.d_pad + i] = key[j * a.d + i] - r[j];
        }
        for (uint32_t i = a.d + tid; i < a.d_pad; i += blockDim.x)
#pragma unroll
            for (uint32_t j = 0; j < NK; ++j) buf[j * a.d_pad + i] = 0.0f;
        __syncthreads();
        if (tid < nk) {  // sigma of key tid (learned.rs:392-396), the keys side by side in wave 0
            const float* b = buf + tid * a.d_pad;
            float acc = 0.0f;
            for (uint32_t i = 0; i < a.d; ++i) acc += b[i] * b[i];
            misc[tid * 32 + 8] = __float_as_uint(sqrtf(acc / (float)a.d));
        }
        __syncthreads();
        if (a.diag) block_rht_n(buf, NK, a.diag, a.d_pad, a.rht_inv);
        {
            float acc[NK];
            seq_dot4xm<kDS, NK, 4>(a.z4, tid, buf, a.d_pad, a.d_pad, acc);
#pragma unroll
            for (uint32_t j = 0; j < NK; ++j) {
                const uint64_t m = __ballot(acc[j] < 0.0f);
                if (lane == 0) {
                    misc[j * 32 + 2 * wave] = (uint32_t)m;
                    misc[j * 32 + 2 * wave + 1] = (uint32_t)(m >> 32);
                }
            }
        }
        __syncthreads();
        if (tid < nk) {  // key tid quantised, the keys side by side in wave 0
            const uint64_t ki = k0 + tid;
            const float* h = hs + tid * 128;
            const uint32_t* mw = misc + tid * 32;
            uint32_t lw[16], gsw[2];
            float scale;
            const uint32_t codec_flag = quantize<CODEC>(h, lw, &scale, gsw);
            const float sigma = __uint_as_float(mw[8]);
            const float lambda = sigma * lambda_c;
            const uint32_t row = (uint32_t)(ki / n_tok);
            const uint32_t pos = pos0 + (uint32_t)(ki - (uint64_t)row * n_tok);
            const uint32_t flags = codec_flag | (warm ? kFlagWarm : 0u);
            uint4* out = tiles + ki * 8;
            out[0] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
            out[1] = make_uint4(lw[4], lw[5], lw[6], lw[7]);
            out[2] = make_uint4(lw[8], lw[9], lw[10], lw[11]);
            out[3] = make_uint4(lw[12], lw[13], lw[14], lw[15]);
            out[4] = make_uint4(mw[0], mw[1], mw[2], mw[3]);
            out[5] = make_uint4(mw[4], mw[5], mw[6], mw[7]);
            out[6] = make_uint4(__float_as_uint(scale), __float_as_uint(lambda), mw[8], pos);
            out[7] = make_uint4(pos, (row % n_kv) | (flags << 16), gsw[0], gsw[1]);
        }
        __syncthreads();
    }
}

// Query -> (q_coarse [128], q_sign [4]) (slha_prepare_query, lib.rs:420-463:
// query_coarse, learned.rs:267-273, and sign_bits of the query itself).
__global__ __launch_bounds__(256) void learned_prepare_kernel(const void* __restrict__ q, int dtype,
                                                              uint64_t n_q, LearnedArgs a,
                                                              float* __restrict__ qc,
                                                              uint64_t* __restrict__ qs) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    float* vec = lds;
    float* buf = lds + a.d;
    uint32_t* words = reinterpret_cast<uint32_t*>(buf + a.d_pad + 128);
    const uint32_t tid = threadIdx.x;
    for (uint64_t qi = blockIdx.x; qi < n_q; qi += gridDim.x) {
        lds_load_vec(q, dtype, qi, a.d, vec);
        __syncthreads();
        for (uint32_t i = tid; i < a.d_pad; i += blockDim.x) buf[i] = i < a.d ? vec[i] : 0.0f;
        if (tid < 128) qc[qi * 128 + tid] = seq_dot4<128>(a.p4, tid, vec, a.d);
        __syncthreads();
        if (a.diag) block_rht(buf, a.diag, a.d_pad, a.rht_inv);
        block_sign_bits(buf, a.z4, a.d_pad, words);
        __syncthreads();
        if (tid < 4) qs[qi * 4 + tid] = (uint64_t)words[2 * tid] | ((uint64_t)words[2 * tid + 1] << 32);
        __syncthreads();
    }
}

// Two queries per workgroup (learned_prepare_kernel's steps, each sum in its
// order): threads 0-127 form query 0's q_coarse and 128-255 query 1's; the
// sketch threads run both chains on one load of Z.
__global__ __launch_bounds__(256) void learned_prepare2_kernel(const void* __restrict__ q, int dtype,
                                                               uint64_t n_q, LearnedArgs a,
                                                               float* __restrict__ qc,
                                                               uint64_t* __restrict__ qs) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    float* vec0 = lds;
    float* vec1 = vec0 + a.d;
    float* buf0 = vec1 + a.d;
    float* buf1 = buf0 + a.d_pad;
    uint32_t* words = reinterpret_cast<uint32_t*>(buf1 + a.d_pad);  // [2][8]
    const uint32_t tid = threadIdx.x, wave = tid >> 6;
    for (uint64_t q0 = 2 * (uint64_t)blockIdx.x; q0 < n_q; q0 += 2 * (uint64_t)gridDim.x) {
        const bool two = q0 + 1 < n_q;  // uniform over the workgroup
        lds_load_vec(q, dtype, q0, a.d, vec0);
        if (two) lds_load_vec(q, dtype, q0 + 1, a.d, vec1);
        __syncthreads();
        for (uint32_t i = tid; i < a.d_pad; i += blockDim.x) {
            buf0[i] = i < a.d ? vec0[i] : 0.0f;
            buf1[i] = i < a.d && two ? vec1[i] : 0.0f;
        }
        if (tid < 128) qc[q0 * 128 + tid] = seq_dot4<128>(a.p4, tid, vec0, a.d);
        else if (two) qc[(q0 + 1) * 128 + tid - 128] = seq_dot4<128>(a.p4, tid - 128, vec1, a.d);
        __syncthreads();
        if (a.diag) block_rht2(buf0, buf1, a.diag, a.d_pad, a.rht_inv);
        {
            float acc0, acc1;
            seq_dot4x2<kDS>(a.z4, tid, buf0, buf1, a.d_pad, acc0, acc1);
            const uint64_t m0 = __ballot(acc0 < 0.0f), m1 = __ballot(acc1 < 0.0f);
            if ((tid & 63u) == 0) {
                words[2 * wave] = (uint32_t)m0, words[2 * wave + 1] = (uint32_t)(m0 >> 32);
                words[8 + 2 * wave] = (uint32_t)m1, words[8 + 2 * wave + 1] = (uint32_t)(m1 >> 32);
            }
        }
        __syncthreads();
        if (tid < (two ? 8u : 4u)) {
            const uint32_t w = tid & 3u, which = tid >> 2;
            qs[(q0 + which) * 4 + w] =
                (uint64_t)words[8 * which + 2 * w] | ((uint64_t)words[8 * which + 2 * w + 1] << 32);
        }
        __syncthreads();
    }
}

// Four queries per workgroup (learned_prepare2_kernel's steps, each sum in
// its order): threads 0-127 form the q_coarse of queries 0 and 1, threads
// 128-255 those of queries 2 and 3, on one load of P each; the sketch
// threads run the four chains on one load of Z. Query slots past n_q are
// computed on and not stored.
__global__ __launch_bounds__(256) void learned_prepare4_kernel(const void* __restrict__ q, int dtype,
                                                               uint64_t n_q, LearnedArgs a,
                                                               float* __restrict__ qc,
                                                               uint64_t* __restrict__ qs) {
    constexpr uint32_t NQ = 4;
    extern __shared__ __attribute__((aligned(16))) float lds[];
    float* vec = lds;                                                // [NQ][d]
    float* buf = vec + NQ * a.d;                                     // [NQ][d_pad]
    uint32_t* words = reinterpret_cast<uint32_t*>(buf + NQ * a.d_pad);  // [NQ][8]
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
    for (uint64_t q0 = NQ * (uint64_t)blockIdx.x; q0 < n_q; q0 += NQ * (uint64_t)gridDim.x) {
        const uint32_t nq = n_q - q0 < NQ ? (uint32_t)(n_q - q0) : NQ;  // uniform
        for (uint32_t j = 0; j < nq; ++j) lds_load_vec(q, dtype, q0 + j, a.d, vec + j * a.d);
        __syncthreads();
        for (uint32_t i = tid; i < a.d_pad; i += blockDim.x)
#pragma unroll
            for (uint32_t j = 0; j < NQ; ++j) buf[j * a.d_pad + i] = i < a.d ? vec[j * a.d + i] : 0.0f;
        {
            const uint32_t half = tid >> 7, k = tid & 127u;  // queries 2 half, 2 half + 1
            if (2 * half < nq) {
                float c[2];
                seq_dot4xm<128, 2, 8>(a.p4, k, vec + 2 * half * a.d, a.d, a.d, c);
                qc[(q0 + 2 * half) * 128 + k] = c[0];
                if (2 * half + 1 < nq) qc[(q0 + 2 * half + 1) * 128 + k] = c[1];
            }
        }
        __syncthreads();
        if (a.diag) block_rht_n(buf, NQ, a.diag, a.d_pad, a.rht_inv);
        {
            float acc[NQ];
            seq_dot4xm<kDS, NQ, 4>(a.z4, tid, buf, a.d_pad, a.d_pad, acc);
#pragma unroll
            for (uint32_t j = 0; j < NQ; ++j) {
                const uint64_t m = __ballot(acc[j] < 0.0f);
                if (lane == 0) {
                    words[8 * j + 2 * wave] = (uint32_t)m;
                    words[8 * j + 2 * wave + 1] = (uint32_t)(m >> 32);
                }
            }
        }
        __syncthreads();
        if (tid < 4 * nq) {
            const uint32_t w = tid & 3u, which = tid >> 2;
            qs[(q0 + which) * 4 + w] =
                (uint64_t)words[8 * which + 2 * w] | ((uint64_t)words[8 * which + 2 * w + 1] << 32);
        }
        __syncthreads();
    }
}

// Tile -> key estimate [d]: reconstruct(dequant_latent) (slha_decode_latent,
// lib.rs:763-822), plus with_residual the sign-sketch term of
// reconstruct_from_tile (learned.rs:288-320), omitted for RHT models.
// kDecTiles tiles per workgroup: every load of P (and Z) feeds their chains,
// each output its own sequential sum. Tile slots past n are computed on and
// not stored.
constexpr uint32_t kDecTiles = 4;

__global__ __launch_bounds__(256) void learned_decode_kernel(const uint4* __restrict__ tiles,
                                                             uint64_t n, LearnedArgs a,
                                                             int with_residual, float sqrt_half_pi,
                                                             float* __restrict__ out) {
    constexpr uint32_t NT = kDecTiles;
    extern __shared__ __attribute__((aligned(16))) float lds[];
    float* hs = lds;                                          // [NT][128]
    uint32_t* misc = reinterpret_cast<uint32_t*>(hs + NT * 128);  // [NT][32]: residual words 0..7, sigma 8
    __shared__ float cb[16];
    const uint32_t tid = threadIdx.x;
    const bool resid = with_residual && !a.diag;
    stage_codebook(cb);
    __syncthreads();
    for (uint64_t t0 = NT * (uint64_t)blockIdx.x; t0 < n; t0 += NT * (uint64_t)gridDim.x) {
        // thread 8 t + g dequantises dims [16g, 16g + 16) of tile t0 + t,
        // operation for operation
        if (tid < 8 * NT && t0 + tid / 8 < n) {
            const uint32_t t = tid / 8, g = tid % 8;
            uint32_t w[32];
            load_tile(tiles + (t0 + t) * 8, w);
            float k[16];
            switch (codec_class(w[29] >> 16)) {
                case kClsInt4: decode_group_exact<kClsInt4>(w, (int)g, cb, k); break;
                case kClsNF4: decode_group_exact<kClsNF4>(w, (int)g, cb, k); break;
                case kClsTQ3: decode_group_exact<kClsTQ3>(w, (int)g, cb, k); break;
                case kClsMixed: decode_group_exact<kClsMixed>(w, (int)g, cb, k); break;
                default: decode_group_exact<kClsMix3>(w, (int)g, cb, k); break;
            }
#pragma unroll
            for (int j = 0; j < 16; ++j) hs[t * 128 + 16 * g + j] = k[j];
            if (g == 0) {
                for (int j = 0; j < 8; ++j) misc[t * 32 + j] = w[16 + j];
                misc[t * 32 + 8] = w[26];
            }
        }
        __syncthreads();
        // (sigma * sqrt(pi/2)) / 256, learned.rs:303
        float sc[NT];
#pragma unroll
        for (uint32_t t = 0; t < NT; ++t) sc[t] = __uint_as_float(misc[t * 32 + 8]) * sqrt_half_pi / 256.0f;
        // kDecU outputs per thread and tile side by side (each its own
        // sequential sum), so every step has kDecU independent loads feeding
        // NT kDecU adds; lanes past d compute a clamped copy and do not store.
        constexpr uint32_t kDecU = 4;
        for (uint32_t i0 = tid; i0 < a.d; i0 += blockDim.x * kDecU) {
            uint32_t ii[kDecU];
            float r[NT][kDecU];
#pragma unroll
            for (uint32_t u = 0; u < kDecU; ++u) {
                const uint32_t i = i0 + u * blockDim.x;
                ii[u] = i < a.d ? i : a.d - 1u;
#pragma unroll
                for (uint32_t t = 0; t < NT; ++t) r[t][u] = 0.0f;
            }
            for (uint32_t k = 0; k < 128; ++k) {
                const float* pk = a.p + (size_t)k * a.d;
                float pv[kDecU];
#pragma unroll
                for (uint32_t u = 0; u < kDecU; ++u) pv[u] = pk[ii[u]];
#pragma unroll
                for (uint32_t t = 0; t < NT; ++t) {
                    const float hk = hs[t * 128 + k];
#pragma unroll
                    for (uint32_t u = 0; u < kDecU; ++u) r[t][u] += hk * pv[u];
                }
            }
            if (resid) {
                for (uint32_t s = 0; s < kDS; ++s) {
                    const float* zs = a.z + (size_t)s * a.d_pad;
                    float zv[kDecU];
#pragma unroll
                    for (uint32_t u = 0; u < kDecU; ++u) zv[u] = zs[ii[u]];
#pragma unroll
                    for (uint32_t t = 0; t < NT; ++t) {
                        const float sgn = ((misc[t * 32 + (s >> 5)] >> (s & 31u)) & 1u) ? -1.0f : 1.0f;
#pragma unroll
                        for (uint32_t u = 0; u < kDecU; ++u) r[t][u] += sgn * sc[t] * zv[u];
                    }
                }
            }
#pragma unroll
            for (uint32_t t = 0; t < NT; ++t)
                if (t0 + t < n)
#pragma unroll
                    for (uint32_t u = 0; u < kDecU; ++u)
                        if (i0 + u * blockDim.x < a.d) out[(t0 + t) * a.d + i0 + u * blockDim.x] = r[t][u];
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Decode attention over compressed keys (benchmark_decode.rs:29-90): for
// query head qh = r*group + j of row r,
//     w = softmax(scores[qh] * scale)      (metrics.rs:338, softmax_into)
//     out[qh][d] = sum_t w_t V[r][t][d]     (aggregate_v, benchmark_decode.rs:29-38)
// with the scores of slha_gpu_score (fast mode). Split over tokens as in
// flash decoding: attn_partial_kernel turns each segment of kAttnSeg tokens
// of a row into (max m, sum l of exp(logit - m), o = sum exp(logit - m) V)
// for every query of the row, reading each V row once for the whole group;
// attn_combine_kernel merges the segments: out = sum_s e^(m_s - M) o_s /
// sum_s e^(m_s - M) l_s. A NaN score, as in softmax_into, zeroes the query's
// output; scores of valid tiles against prepared (finite) queries are
// finite, so the other degenerate cases of softmax_into (+inf logits, all
// logits -inf) do not arise here.
// softmax_into forms its logits in f64, where a finite f32 score times a
// finite scale never overflows. In f32 score * scale can, so the kernels work
// on t = score * sign(scale) and weigh each token with
// exp((t - max t) * |scale|): the same weights, and a difference that
// overflows only pushes a weight to 0, as it is in f64. Partial maxima are
// kept in t, and the combine scales their differences by |scale| the same way.
constexpr uint32_t kAttnSeg = 256;  // tokens per partial block (one per thread in phase 1)
constexpr uint32_t kAttnMaxGroup = 16;
// Groups scored inside attn_fused_kernel: up to 4 at any d_v, up to 8 while
// a wave's weights and o_w ([G][64 + d_v] floats) fit its 8 KiB tile region.
__host__ __device__ constexpr bool attn_fused_ok(uint32_t group, uint32_t d_v) {
    return group <= 4 || (group <= 8 && d_v <= 128);
}

__host__ __device__ constexpr size_t attn_partial_floats(uint32_t d_v) { return (size_t)d_v + 4; }

// Max (or sum) over the 256 threads of each of G values, in place: xor
// shuffles within each wave, then the 4 wave results through LDS.
template <int G, bool MAX>
__device__ __forceinline__ void block_reduce_g(float* x, float (*tmp)[4]) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const float y = __shfl_xor(x[j], o);
            x[j] = MAX ? fmaxf(x[j], y) : x[j] + y;
        }
    __syncthreads();
    if ((threadIdx.x & 63u) == 0)
#pragma unroll
        for (int j = 0; j < G; ++j) tmp[j][threadIdx.x >> 6] = x[j];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < G; ++j)
        x[j] = MAX ? fmaxf(fmaxf(tmp[j][0], tmp[j][1]), fmaxf(tmp[j][2], tmp[j][3]))
                   : (tmp[j][0] + tmp[j][1]) + (tmp[j][2] + tmp[j][3]);
}

// grid (n_seg, n_rows), 256 threads; group <= G (a power of two <=
// kAttnMaxGroup), VDT the V element type, DV = d_v.
// part[((r * n_seg + seg) * group + j)] = {m, l, -, -, o[DV]} (l = NaN when a
// score of the segment is NaN).
//  phase 1: thread t holds token t0 + t: logits, per-query max and sum of
//           exp(logit - max) over the segment, weights e[j][t] in LDS;
//  phase 2: lane group of LPT = DV / VEC lanes reads one token's V row as
//           16-byte vectors (VEC elements per lane), TPS = 256 / LPT tokens
//           per step; each lane accumulates G x VEC outputs, then the TPS
//           token slots are summed (xor shuffles inside the wave, LDS across
//           the waves).
template <int VDT, int G, int DV>
__global__ __launch_bounds__(256) void attn_partial_kernel(const float* __restrict__ scores,
                                                           const void* __restrict__ vals,
                                                           uint32_t n_tok, uint32_t group,
                                                           float scale, float* __restrict__ part) {
    constexpr int VEC = VDT == kDtypeBF16 ? 8 : 4;  // V elements per 16-byte lane load
    constexpr int LPT = DV / VEC;                   // lanes per token row
    constexpr int TPW = 64 / LPT;                   // tokens per wave step
    constexpr int TPS = 4 * TPW;                    // tokens per block step
    __shared__ float e[G][kAttnSeg];
    __shared__ float tmp[G][4];
    __shared__ float red[4][G][DV];
    const uint32_t seg = blockIdx.x, row = blockIdx.y, n_seg = gridDim.x;
    const uint32_t t0 = seg * kAttnSeg;
    const uint32_t nt = n_tok - t0 < kAttnSeg ? n_tok - t0 : kAttnSeg;
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6, lane = tid & 63u;
    const uint32_t slot = wave * TPW + lane / LPT;  // token slot 0 .. TPS-1
    const uint32_t dc = lane % LPT;                 // this lane's VEC dims: dc*VEC ..
    const char* vrow = static_cast<const char*>(vals) +
                       (((size_t)row * n_tok + t0) * DV + (size_t)dc * VEC) * (VDT == kDtypeBF16 ? 2 : 4);
    constexpr size_t kRowBytes = (size_t)DV * (VDT == kDtypeBF16 ? 2 : 4);
    // V is read through a ring of kDepth 16-byte loads running ahead of the
    // FMAs, at a token clamped into the segment (nt >= 1; no branch between
    // the loads; a slot past the last token then uses V = 0). The ring is
    // filled before the softmax reductions, so those loads overlap the
    // block's barriers.
    constexpr uint32_t kSteps = kAttnSeg / TPS, kDepth = kSteps < 8 ? kSteps : 8;
    const auto load = [&](uint32_t step) {
        const uint32_t t = step * TPS + slot;
        const uint32_t tc = t < nt ? t : nt - 1u;
        return *reinterpret_cast<const uint4*>(vrow + (size_t)tc * kRowBytes);
    };
    uint4 x[kDepth];
#pragma unroll
    for (uint32_t u = 0; u < kDepth; ++u) x[u] = load(u);
    // phase 1 (t = score * sign(scale), weights exp((t - max t) * |scale|))
    const float sgn = scale < 0.0f ? -1.0f : 1.0f, sa = fabsf(scale);
    float lg[G], m[G], l[G], nan[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        lg[j] = -INFINITY;
        nan[j] = 0.0f;
        if (tid < nt && (uint32_t)j < group) {
            const float sc = scores[((size_t)row * group + j) * n_tok + t0 + tid];
            nan[j] = isnan(sc) ? 1.0f : 0.0f;
            lg[j] = sc * sgn;
        }
        m[j] = lg[j];
    }
    block_reduce_g<G, true>(m, tmp);
    block_reduce_g<G, true>(nan, tmp);
#pragma unroll
    for (int j = 0; j < G; ++j) {
        const float w = tid < nt ? __expf((lg[j] - m[j]) * sa) : 0.0f;
        e[j][tid] = w;
        l[j] = w;
    }
    block_reduce_g<G, false>(l, tmp);  // its barriers also publish e
    // phase 2
    float o[G][VEC];
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
        for (int k = 0; k < VEC; ++k) o[j][k] = 0.0f;
#pragma unroll
    for (uint32_t step = 0; step < kSteps; ++step) {
        const uint4 cur = x[step % kDepth];
        if (step + kDepth < kSteps) x[step % kDepth] = load(step + kDepth);
        const uint32_t t = step * TPS + slot;
        const bool in = t < nt;
        float v[VEC];
        if constexpr (VDT == kDtypeBF16) {
            const uint32_t u[4] = {cur.x, cur.y, cur.z, cur.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                v[2 * k] = __uint_as_float(u[k] << 16);
                v[2 * k + 1] = __uint_as_float(u[k] & 0xFFFF0000u);
            }
        } else {
            v[0] = __uint_as_float(cur.x), v[1] = __uint_as_float(cur.y);
            v[2] = __uint_as_float(cur.z), v[3] = __uint_as_float(cur.w);
        }
#pragma unroll
        for (int k = 0; k < VEC; ++k) v[k] = in ? v[k] : 0.0f;
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const float w = e[j][t < nt ? t : 0u];
#pragma unroll
            for (int k = 0; k < VEC; ++k) o[j][k] = fmaf(w, v[k], o[j][k]);
        }
    }
    // sum over the TPW token slots of the wave (lanes lane % LPT equal) ...
#pragma unroll
    for (int off = LPT; off < 64; off <<= 1)
#pragma unroll
        for (int j = 0; j < G; ++j)
#pragma unroll
            for (int k = 0; k < VEC; ++k) o[j][k] += __shfl_xor(o[j][k], off);
    // ... then over the 4 waves
    if (lane < LPT)
#pragma unroll
        for (int j = 0; j < G; ++j)
#pragma unroll
            for (int k = 0; k < VEC; ++k) red[wave][j][dc * VEC + k] = o[j][k];
    __syncthreads();
    for (uint32_t i = tid; i < group * DV; i += 256u) {
        const uint32_t j = i / DV, d = i % DV;
        float* pp = part + (((size_t)row * n_seg + seg) * group + j) * attn_partial_floats(DV);
        pp[4 + d] = (red[0][j][d] + red[1][j][d]) + (red[2][j][d] + red[3][j][d]);
        if (d == 0) pp[0] = m[j], pp[1] = nan[j] != 0.0f ? NAN : l[j];
    }
}

// Fused segment kernel for attn_fused_ok(group, d_v), G = 4 or 8 (queries
// staged per row), grid (n_seg, n_rows), 256 threads.
// Wave w scores tokens t0 + 64 w .. +63 exactly as score_rows_fast_kernel<4>
// scores them (same tile DMA, query staging and MFMA paths) and runs a
// flash-decoding step over its own 64 tokens: wave max m_w, weights
// exp(logit - m_w), sum l_w and o_w = sum weight * V. The block merges its four
// waves with exp(m_w - M) into one partial {M, L, -, -, O[DV]} (L = NaN when a
// score of the segment is NaN), read by attn_combine_kernel. Once a wave has
// read its tiles back, its 8 KiB tile region holds its weights [G][64] and
// then its o_w [G][DV], so the block needs about 37 KiB of LDS and, at <= 128
// VGPRs, four blocks share a CU: the decode grid (128 x 8) is resident at once.
template <int VDT, int DV, int G>
__global__ __launch_bounds__(256, G <= 4 ? 4 : 3) void attn_fused_kernel(const uint4* __restrict__ tiles,
                                                            uint32_t n_tok, uint32_t group,
                                                            const float* __restrict__ qc,
                                                            const uint32_t* __restrict__ qs,
                                                            const void* __restrict__ vals,
                                                            float scale, float* __restrict__ part) {
    constexpr int VEC = VDT == kDtypeBF16 ? 8 : 4;  // V elements per 16-byte load
    constexpr int LPT = DV / VEC, TPW = 64 / LPT;   // lanes per token, tokens per wave step
    constexpr uint32_t kSteps = 64 / TPW;
    constexpr size_t kRowBytes = (size_t)DV * (VDT == kDtypeBF16 ? 2 : 4);
    static_assert(G * (64 + DV) * 4 <= 512 * 16, "weights and o_w fit the tile region");
    __shared__ float cb[16];
    __shared__ uint4 tile_lds[4][512];
    __shared__ __attribute__((aligned(16))) float qstatic[staging_bytes(G) / 4];
    __shared__ float wst[4][G][3];  // per wave: m_w, l_w, NaN seen
    const uint32_t seg = blockIdx.x, row = blockIdx.y, n_seg = gridDim.x;
    const uint32_t tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63u;
    const size_t qrow0 = (size_t)row * group;
    const uint32_t wave0 = seg * kAttnSeg + 64u * wave;
    const uint32_t n_valid = wave0 < n_tok ? n_tok - wave0 : 0u;
    const uint32_t nw = n_valid < 64u ? n_valid : 64u;  // tokens of this wave
    float* ew = reinterpret_cast<float*>(tile_lds[wave]);  // [G][64] after the readback
    float* ow = ew + G * 64;                               // [G][DV]
    {
        const StagedQueries sq = carve_staging(qstatic, G);
        QueryRegs<G> qr;
        stage_issue<G>(qc, qrow0, group, qr);
        fetch_tiles_lds(tiles + ((size_t)row * n_tok + wave0) * 8, n_valid, tile_lds[wave]);
        stage_codebook(cb);
        stage_commit<G>(qr, group, sq);
        lds_barrier();
        uint32_t w[32];
        fetch_tiles_readback(tile_lds[wave], w);
        const bool valid = lane < nw;
        if (!score_wave_try_mfma(w, valid, group, qrow0, sq.q32, cb, sq.q16, sq.qexp, qs, ew, 64,
                                 lane) &&
            valid)
            score_dispatch<false, false>(w, group, qrow0, qc, qs, cb, ew, nullptr, 64, lane);
    }
    // Softmax statistics of the wave; lane holds token wave0 + lane.
    // t = score * sign(scale), weights exp((t - max t) * |scale|).
    const float sgn = scale < 0.0f ? -1.0f : 1.0f, sa = fabsf(scale);
    float m[G], l[G];
    bool bad[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        float lg = -INFINITY;
        bool nan_j = false;
        if (lane < nw && (uint32_t)j < group) {
            const float sc = ew[j * 64 + lane];
            nan_j = isnan(sc);
            lg = sc * sgn;
        }
        bad[j] = __any(nan_j);
        float mx = lg;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        m[j] = mx;
        const float wgt = lane < nw ? __expf((lg - mx) * sa) : 0.0f;
        ew[j * 64 + lane] = wgt;
        float sm = wgt;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) sm += __shfl_xor(sm, o);
        l[j] = sm;
    }
    // o_w: lane group slot = lane / LPT reads token slot + TPW * step, dims
    // dc * VEC .. +VEC-1, with one 16-byte load. Loads run 8 steps ahead in
    // a ring, at a token clamped into the wave's range (no branch between
    // them); a lane past the last token then uses V = 0.
    const uint32_t slot = lane / LPT, dc = lane % LPT;
    const char* vrow = static_cast<const char*>(vals) +
                       (((size_t)row * n_tok + wave0) * DV + (size_t)dc * VEC) * (VDT == kDtypeBF16 ? 2 : 4);
    float o[G][VEC];
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
        for (int k = 0; k < VEC; ++k) o[j][k] = 0.0f;
    if (nw > 0) {
        constexpr uint32_t kDepth = kSteps < 8 ? kSteps : 8;
        const auto load = [&](uint32_t step) {
            const uint32_t t = step * TPW + slot;
            const uint32_t tc = t < nw ? t : nw - 1u;
            return *reinterpret_cast<const uint4*>(vrow + (size_t)tc * kRowBytes);
        };
        uint4 x[kDepth];
#pragma unroll
        for (uint32_t u = 0; u < kDepth; ++u) x[u] = load(u);
#pragma unroll
        for (uint32_t step = 0; step < kSteps; ++step) {
            const uint4 cur = x[step % kDepth];
            if (step + kDepth < kSteps) x[step % kDepth] = load(step + kDepth);
            const uint32_t t = step * TPW + slot;
            const bool in = t < nw;
            float v[VEC];
            if constexpr (VDT == kDtypeBF16) {
                const uint32_t w4[4] = {cur.x, cur.y, cur.z, cur.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    v[2 * k] = __uint_as_float(w4[k] << 16);
                    v[2 * k + 1] = __uint_as_float(w4[k] & 0xFFFF0000u);
                }
            } else {
                v[0] = __uint_as_float(cur.x), v[1] = __uint_as_float(cur.y);
                v[2] = __uint_as_float(cur.z), v[3] = __uint_as_float(cur.w);
            }
#pragma unroll
            for (int k = 0; k < VEC; ++k) v[k] = in ? v[k] : 0.0f;
#pragma unroll
            for (int j = 0; j < G; ++j) {
                const float wgt = ew[j * 64 + (t & 63u)];
#pragma unroll
                for (int k = 0; k < VEC; ++k) o[j][k] = fmaf(wgt, v[k], o[j][k]);
            }
        }
    }
#pragma unroll
    for (int off = LPT; off < 64; off <<= 1)
#pragma unroll
        for (int j = 0; j < G; ++j)
#pragma unroll
            for (int k = 0; k < VEC; ++k) o[j][k] += __shfl_xor(o[j][k], off);
    if (lane < LPT)
#pragma unroll
        for (int j = 0; j < G; ++j)
#pragma unroll
            for (int k = 0; k < VEC; ++k) ow[j * DV + dc * VEC + k] = o[j][k];
    if (lane == 0)
#pragma unroll
        for (int j = 0; j < G; ++j) {
            wst[wave][j][0] = m[j];
            wst[wave][j][1] = l[j];
            wst[wave][j][2] = bad[j] ? 1.0f : 0.0f;
        }
    __syncthreads();
    // Merge the four waves: a wave with no token (m_w = -inf) weighs 0.
    for (uint32_t i = tid; i < group * DV; i += 256u) {
        const uint32_t j = i / DV, d = i % DV;
        const float M = fmaxf(fmaxf(wst[0][j][0], wst[1][j][0]), fmaxf(wst[2][j][0], wst[3][j][0]));
        float c[4], od[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            c[k] = wst[k][j][0] == -INFINITY ? 0.0f : __expf((wst[k][j][0] - M) * sa);
            od[k] = reinterpret_cast<const float*>(tile_lds[k])[G * 64 + j * DV + d];
        }
        float* pp = part + (((size_t)row * n_seg + seg) * group + j) * attn_partial_floats(DV);
        pp[4 + d] = (od[0] * c[0] + od[1] * c[1]) + (od[2] * c[2] + od[3] * c[3]);
        if (d == 0) {
            const bool any_bad = (wst[0][j][2] + wst[1][j][2]) + (wst[2][j][2] + wst[3][j][2]) != 0.0f;
            pp[0] = M;
            pp[1] = any_bad ? NAN
                            : (wst[0][j][1] * c[0] + wst[1][j][1] * c[1]) +
                                  (wst[2][j][1] * c[2] + wst[3][j][1] * c[3]);
        }
    }
}

// grid (n_rows * group, d_v / 16), 256 threads: thread (sl, c) = (tid / 16,
// tid % 16) merges segments sl, sl + 16, ... for dim 16 blockIdx.y + c; the
// 16 segment lanes are then added (xor shuffles, then LDS across waves). The
// {m, l, o[d]} of a thread's first U segments are loaded together, before the
// block max, so up to 16 U segments cost one round trip to memory.
__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ part,
                                                           uint32_t n_seg, uint32_t group,
                                                           uint32_t d_v, float scale,
                                                           float* __restrict__ out) {
    const float sa = fabsf(scale);  // partial maxima are in t = score * sign(scale)
    constexpr uint32_t U = 8;
    __shared__ float red_a[4][16], red_l[4], red_m[4];
    __shared__ uint32_t red_n[4];
    const uint32_t qh = blockIdx.x, tid = threadIdx.x, wave = tid >> 6;
    const uint32_t c = tid & 15u, sl = tid >> 4;
    const uint32_t d = blockIdx.y * 16u + c;
    const uint32_t row = qh / group, j = qh % group;
    const size_t stride = (size_t)group * attn_partial_floats(d_v);  // one segment
    const float* p0 = part + ((size_t)row * n_seg * group + j) * attn_partial_floats(d_v);
    // Segment s = sl + 16 u, read at min(s, n_seg - 1) and masked (n_seg >= 1).
    float mu[U], lu[U], au[U];
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
        const uint32_t sg = sl + 16u * u;
        const float* ps = p0 + (size_t)(sg < n_seg ? sg : n_seg - 1u) * stride;
        mu[u] = ps[0], lu[u] = ps[1], au[u] = ps[4 + d];
    }
    float M = -INFINITY;
#pragma unroll
    for (uint32_t u = 0; u < U; ++u)
        if (sl + 16u * u < n_seg) M = fmaxf(M, mu[u]);
    for (uint32_t sg = sl + 16u * U; sg < n_seg; sg += 16u) M = fmaxf(M, p0[sg * stride]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
    if ((tid & 63u) == 0) red_m[wave] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
    float L = 0.0f, acc = 0.0f;
    bool nan = false;
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
        if (sl + 16u * u < n_seg) {
            const float f = __expf((mu[u] - M) * sa);
            nan = nan || isnan(lu[u]);
            L = fmaf(lu[u], f, L);
            acc = fmaf(au[u], f, acc);
        }
    }
    for (uint32_t sg = sl + 16u * U; sg < n_seg; sg += 16u) {  // more than 16 U segments
        const float* ps = p0 + sg * stride;
        const float f = __expf((ps[0] - M) * sa);
        nan = nan || isnan(ps[1]);
        L = fmaf(ps[1], f, L);
        acc = fmaf(ps[4 + d], f, acc);
    }
    uint32_t nn = nan ? 1u : 0u;
#pragma unroll
    for (int o = 16; o < 64; o <<= 1) {  // the 4 segment lanes of this wave
        L += __shfl_xor(L, o);
        acc += __shfl_xor(acc, o);
        nn |= (uint32_t)__shfl_xor((int)nn, o);
    }
    if ((tid & 63u) < 16u) red_a[wave][c] = acc;
    if ((tid & 63u) == 0) red_l[wave] = L, red_n[wave] = nn;
    __syncthreads();
    if (tid < 16u) {
        const float Lt = (red_l[0] + red_l[1]) + (red_l[2] + red_l[3]);
        const float At = (red_a[0][c] + red_a[1][c]) + (red_a[2][c] + red_a[3][c]);
        const bool bad = (red_n[0] | red_n[1] | red_n[2] | red_n[3]) != 0u || !(Lt > 0.0f);
        out[(size_t)qh * d_v + d] = bad ? 0.0f : At / Lt;
    }
}

// ---------------------------------------------------------------------------
// EventLog records (eventlog.rs:9-36): 144 bytes = u64 seq, u32 slot, u32
// checksum, the 128 tile bytes. The tile's in-memory bytes are already the
// little-endian serialisation of `tile_to_bytes` (eventlog.rs:82-100), so a
// record is the tile copied behind a 16-byte head. Version 2's checksum is
// FNV-1a 32 over seq || slot || tile (eventlog.rs:148-170); version 1 stores 0.

constexpr uint32_t kFnvOffset = 0x811C9DC5u, kFnvPrime = 0x01000193u;

__device__ __forceinline__ uint32_t fnv_word(uint32_t h, uint32_t w) {
#pragma unroll
    for (int b = 0; b < 4; ++b) h = (h ^ ((w >> (8 * b)) & 0xFFu)) * kFnvPrime;
    return h;
}

__device__ __forceinline__ uint32_t record_checksum(uint64_t seq, uint32_t slot, const uint4* t) {
    uint32_t h = fnv_word(kFnvOffset, (uint32_t)seq);
    h = fnv_word(h, (uint32_t)(seq >> 32));
    h = fnv_word(h, slot);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        h = fnv_word(h, t[j].x);
        h = fnv_word(h, t[j].y);
        h = fnv_word(h, t[j].z);
        h = fnv_word(h, t[j].w);
    }
    return h;
}

constexpr uint32_t kRecordQuads = 9;  // 144 B

// 256 records per workgroup: thread r gathers tile slots[r] (8 x 16-byte
// loads), hashes it and writes its record into LDS; the workgroup then stores
// its 36 KiB of records with consecutive 16-byte stores. (Gathering with 8
// lanes per tile instead needs a workgroup barrier before the hash and was
// 8 % slower.)
__global__ __launch_bounds__(256) void eventlog_pack_kernel(const uint4* __restrict__ arena,
                                                            const uint32_t* __restrict__ slots,
                                                            const uint64_t* __restrict__ seqs,
                                                            uint64_t n, uint32_t version,
                                                            uint4* __restrict__ records) {
    __shared__ uint4 rec[256 * kRecordQuads];
    __shared__ uint32_t s_slot[256];
    const uint64_t base = (uint64_t)blockIdx.x * 256u;
    const uint32_t tid = threadIdx.x;
    const uint32_t cnt = n - base < 256u ? (uint32_t)(n - base) : 256u;
    uint64_t seq = 0;
    uint32_t slot = 0;
    if (tid < cnt) {
        seq = seqs[base + tid];
        slot = slots[base + tid];
        s_slot[tid] = slot;
    }
    __syncthreads();
    // Tiles enter with 8 lanes per tile (lane quad tid % 8 of tile
    // tid / 8 + 32 k), so each load instruction reads whole 128-byte lines
    // rather than 16 bytes of 64 scattered tiles; thread r then checksums
    // record r from LDS.
    uint4 q[8];
#pragma unroll
    for (uint32_t k = 0; k < 8; ++k) {
        const uint32_t r = (tid >> 3) + 32u * k;
        q[k] = r < cnt ? arena[(size_t)s_slot[r] * 8 + (tid & 7u)] : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (uint32_t k = 0; k < 8; ++k) {
        const uint32_t r = (tid >> 3) + 32u * k;
        if (r < cnt) rec[r * kRecordQuads + 1u + (tid & 7u)] = q[k];
    }
    __syncthreads();
    if (tid < cnt) {
        uint4 t[8];
        uint4* r = rec + tid * kRecordQuads;
#pragma unroll
        for (int j = 0; j < 8; ++j) t[j] = r[1 + j];
        const uint32_t ck = version >= 2 ? record_checksum(seq, slot, t) : 0u;
        r[0] = make_uint4((uint32_t)seq, (uint32_t)(seq >> 32), slot, ck);
    }
    __syncthreads();
    uint4* out = records + base * kRecordQuads;
    for (uint32_t q = tid; q < cnt * kRecordQuads; q += 256u) out[q] = rec[q];
}

// The reverse: 256 records per workgroup are loaded with consecutive 16-byte
// loads into LDS; thread r checks record r's checksum (version 2) and writes
// status 0 (the tile is then written to slot dst[r]) or 1 (slot untouched).
// The tiles are then written with 8 consecutive lanes per tile, one whole
// 128-byte line per 8 lanes of a store (84 -> 64 us per 1 M records against
// one lane per tile).
__global__ __launch_bounds__(256) void eventlog_unpack_kernel(const uint4* __restrict__ records,
                                                              uint64_t n, uint32_t version,
                                                              const uint32_t* __restrict__ dst,
                                                              uint4* __restrict__ arena,
                                                              uint32_t* __restrict__ status) {
    __shared__ uint4 rec[256 * kRecordQuads];
    __shared__ uint32_t s_dst[256];
    __shared__ uint32_t s_ok[256];
    const uint64_t base = (uint64_t)blockIdx.x * 256u;
    const uint32_t tid = threadIdx.x;
    const uint32_t cnt = n - base < 256u ? (uint32_t)(n - base) : 256u;
    const uint4* in = records + base * kRecordQuads;
    for (uint32_t q = tid; q < cnt * kRecordQuads; q += 256u) rec[q] = in[q];
    const uint32_t d = tid < cnt ? dst[base + tid] : 0u;
    __syncthreads();
    if (tid < cnt) {
        const uint4* r = rec + tid * kRecordQuads;
        bool ok = true;
        if (version >= 2) {
            const uint4 head = r[0];
            uint4 t[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) t[j] = r[1 + j];
            const uint64_t seq = (uint64_t)head.x | ((uint64_t)head.y << 32);
            ok = record_checksum(seq, head.z, t) == head.w;
        }
        s_dst[tid] = d;
        s_ok[tid] = ok ? 1u : 0u;
        status[base + tid] = ok ? 0u : 1u;
    }
    __syncthreads();
    for (uint32_t q = tid; q < cnt * 8u; q += 256u) {
        const uint32_t r = q >> 3, j = q & 7u;
        if (s_ok[r]) arena[(size_t)s_dst[r] * 8 + j] = rec[r * kRecordQuads + 1 + j];
    }
}

// ---------------------------------------------------------------------------
// CCOS control plane over the device arena (ccos.rs)

// insert: tile i -> arena slot dst[i] with 8 lanes per tile, importance reset
// and, with a state array, the slot's state from the tile's FLAG_WARM (1 WARM,
// else 0 HOT; ccos.rs:226-247).
__global__ __launch_bounds__(256) void tile_scatter_kernel(const uint4* __restrict__ src,
                                                           const uint32_t* __restrict__ dst,
                                                           uint64_t n, uint4* __restrict__ arena,
                                                           float* __restrict__ importance,
                                                           uint8_t* __restrict__ state) {
    const uint64_t q = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (q >= n * 8) return;
    const uint64_t i = q >> 3;
    const uint32_t j = (uint32_t)(q & 7u);
    const uint32_t slot = dst[i];
    const uint4 v = src[q];
    arena[(size_t)slot * 8 + j] = v;
    if (j == 0 && importance) importance[slot] = 0.0f;
    if (j == 7 && state) state[slot] = ((v.y >> 16) & kFlagWarm) ? 1 : 0;  // flags @118
}

// observe_scores (ccos.rs:257-300) over the scores of slots [0, n), in two
// launches with fixed reduction orders (repeated calls agree bit for bit):
//   1. per workgroup: the online softmax statistics of its live scores,
//      (m, l) with l = sum exp((s - m) / T), and a flag (1: a non-finite live
//      score, 0: live scores, -1: none);
//   2. every workgroup merges the statistics in the same order into (M, L)
//      and, when the inputs are valid, adds exp((s - M) / T) * (1 / L) to the
//      importance of each live slot.
// L differs from the reference's sequential sum by rounding only (relative
// error a few f32 ulps). partial holds 3 * kObsBlocks floats.
constexpr uint32_t kObsBlocks = 512, kObsUnroll = 4;

struct SoftStat {
    float m, l;
};

__device__ __forceinline__ SoftStat soft_merge(SoftStat a, SoftStat b, float t) {
    const float m = fmaxf(a.m, b.m);
    if (m == -INFINITY) return {m, 0.0f};
    const float la = a.m == -INFINITY ? 0.0f : a.l * expf((a.m - m) / t);
    const float lb = b.m == -INFINITY ? 0.0f : b.l * expf((b.m - m) / t);
    return {m, la + lb};
}

__device__ __forceinline__ SoftStat block_soft(SoftStat x, float t, float (*tmp)[4]) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const SoftStat y = {__shfl_xor(x.m, o), __shfl_xor(x.l, o)};
        x = soft_merge(x, y, t);
    }
    __syncthreads();
    if ((threadIdx.x & 63u) == 0) tmp[0][threadIdx.x >> 6] = x.m, tmp[1][threadIdx.x >> 6] = x.l;
    __syncthreads();
    SoftStat r = {tmp[0][0], tmp[1][0]};
#pragma unroll
    for (int w = 1; w < 4; ++w) r = soft_merge(r, {tmp[0][w], tmp[1][w]}, t);
    return r;
}

__device__ __forceinline__ float block_max_f(float x, float* tmp) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
    __syncthreads();
    if ((threadIdx.x & 63u) == 0) tmp[threadIdx.x >> 6] = x;
    __syncthreads();
    return fmaxf(fmaxf(tmp[0], tmp[1]), fmaxf(tmp[2], tmp[3]));
}

// Slot groups: with VEC, group g is the 4 consecutive slots 4g .. 4g + 3
// (one 16-byte score load, one 4-byte state load; the caller checks the
// alignment) for g < n / 4, and the last n % 4 slots are a tail taken by
// thread 0 of workgroup 0; without VEC a group is one slot. Each thread takes
// kObsUnroll groups a grid-stride apart per iteration, loaded at an index
// clamped into range with no branch between the loads, then masked.
template <bool VEC>
struct ObsGroups {
    uint64_t full;  // groups loaded whole
    __device__ explicit ObsGroups(uint64_t n) : full(VEC ? n / 4 : n) {}
};

template <bool VEC>
__device__ __forceinline__ void load_group(const float* scores, const uint8_t* state, uint64_t g,
                                           float (&x)[4], uint32_t& st) {
    if constexpr (VEC) {
        const float4 v = *reinterpret_cast<const float4*>(scores + 4 * g);
        st = *reinterpret_cast<const uint32_t*>(state + 4 * g);
        x[0] = v.x, x[1] = v.y, x[2] = v.z, x[3] = v.w;
    } else {
        x[0] = scores[g];
        st = state[g] | 0x02020200u;  // slots 1..3 of a one-slot group read as COLD
        x[1] = x[2] = x[3] = 0.0f;
    }
}

// x / t for an exp argument x <= 0: quot<FQ>, except that an overflowing
// x yt (|x / t| beyond FLT_MAX, where the correction would give NaN) is
// returned as is; its exp is 0, as that of the division's -inf or -FLT_MAX.
template <bool FQ>
__device__ __forceinline__ float exp_arg(float x, float t, float yt) {
    if constexpr (FQ) {
        const float q0 = x * yt;
        return isinf(q0) ? q0 : quot<true>(x, t, yt);
    } else {
        return x / t;
    }
}

// Online softmax statistics of one slot (ccos.rs:257-300). Both branches of
// the update take exp of -|v - m| / t ((m - v) / t when v > m, else
// (v - m) / t: the same magnitude, as IEEE subtraction and division are
// sign-symmetric), so one exp serves either and the update is two selects
// instead of a divergent branch. The first finite slot of a thread gives
// l = 1, as l * e + 1 with l = 0 does. FQ: x / t by exp_arg from
// yt = RN(1 / t) (the launcher checks t's range), which gives the division's
// bits for |x / t| >= 2^-32 and, below that, an argument whose exp is 1.0f
// either way.
template <bool FQ>
__device__ __forceinline__ void soft_add(SoftStat& st, float& flag, float v, float t, float yt) {
    if (!isfinite(v)) {
        flag = 1.0f;
        return;
    }
    flag = fmaxf(flag, 0.0f);
    const bool first = st.m == -INFINITY, up = v > st.m;
    const float d = first ? 0.0f : fabsf(v - st.m);
    const float e = expf(exp_arg<FQ>(-d, t, yt));
    st.l = up ? (first ? 0.0f : st.l * e) + 1.0f : st.l + e;
    st.m = up ? v : st.m;
}

template <bool VEC, bool FQ>
__global__ __launch_bounds__(256) void observe_stats_kernel(const float* __restrict__ scores,
                                                            const uint8_t* __restrict__ state, uint64_t n,
                                                            float t, float yt, float* __restrict__ partial) {
    __shared__ float tmp[2][4];
    SoftStat st = {-INFINITY, 0.0f};
    float flag = -1.0f;
    const uint64_t full = ObsGroups<VEC>(n).full;
    const uint64_t stride = (uint64_t)gridDim.x * 256u;
    for (uint64_t g0 = (uint64_t)blockIdx.x * 256u + threadIdx.x; g0 < full; g0 += stride * kObsUnroll) {
        float x[kObsUnroll][4];
        uint32_t sb[kObsUnroll];
#pragma unroll
        for (uint32_t u = 0; u < kObsUnroll; ++u) {
            const uint64_t g = g0 + u * stride;
            load_group<VEC>(scores, state, g < full ? g : full - 1, x[u], sb[u]);
            if (g >= full) sb[u] = 0x02020202u;  // past the end: all COLD
        }
#pragma unroll
        for (uint32_t u = 0; u < kObsUnroll; ++u)
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (((sb[u] >> (8 * k)) & 0xFFu) != 2u) soft_add<FQ>(st, flag, x[u][k], t, yt);
    }
    if (VEC && blockIdx.x == 0 && threadIdx.x == 0)
        for (uint64_t s = 4 * full; s < n; ++s)
            if (state[s] != 2) soft_add<FQ>(st, flag, scores[s], t, yt);
    st = block_soft(st, t, tmp);
    flag = block_max_f(flag, tmp[0]);
    if (threadIdx.x == 0) {
        partial[blockIdx.x] = st.m;
        partial[kObsBlocks + blockIdx.x] = st.l;
        partial[2 * kObsBlocks + blockIdx.x] = flag;
    }
}

template <bool VEC, bool FQ>
__global__ __launch_bounds__(256) void observe_apply_kernel(const float* __restrict__ scores,
                                                            const uint8_t* __restrict__ state, uint64_t n,
                                                            float t, float yt, const float* __restrict__ partial,
                                                            float* __restrict__ importance) {
    __shared__ float tmp[2][4];
    SoftStat st = {-INFINITY, 0.0f};
    float flag = -1.0f;
    for (uint32_t k = threadIdx.x; k < gridDim.x; k += 256u) {
        st = soft_merge(st, {partial[k], partial[kObsBlocks + k]}, t);
        flag = fmaxf(flag, partial[2 * kObsBlocks + k]);
    }
    st = block_soft(st, t, tmp);
    flag = block_max_f(flag, tmp[0]);
    if (flag != 0.0f || !isfinite(st.l) || !(st.l > 0.0f)) return;
    const float M = st.m, inv = 1.0f / st.l;
    const uint64_t full = ObsGroups<VEC>(n).full;
    const uint64_t stride = (uint64_t)gridDim.x * 256u;
    for (uint64_t g0 = (uint64_t)blockIdx.x * 256u + threadIdx.x; g0 < full; g0 += stride * kObsUnroll) {
        float x[kObsUnroll][4], im[kObsUnroll][4];
        uint32_t sb[kObsUnroll];
#pragma unroll
        for (uint32_t u = 0; u < kObsUnroll; ++u) {
            const uint64_t g = g0 + u * stride, gc = g < full ? g : full - 1;
            load_group<VEC>(scores, state, gc, x[u], sb[u]);
            if constexpr (VEC) {
                const float4 v = *reinterpret_cast<const float4*>(importance + 4 * gc);
                im[u][0] = v.x, im[u][1] = v.y, im[u][2] = v.z, im[u][3] = v.w;
            } else {
                im[u][0] = importance[gc];
            }
        }
#pragma unroll
        for (uint32_t u = 0; u < kObsUnroll; ++u) {
            const uint64_t g = g0 + u * stride;
            if (g >= full) continue;
#pragma unroll
            for (int k = 0; k < (VEC ? 4 : 1); ++k)
                if (((sb[u] >> (8 * k)) & 0xFFu) != 2u)
                    im[u][k] += expf(exp_arg<FQ>(x[u][k] - M, t, yt)) * inv;
            if constexpr (VEC)
                *reinterpret_cast<float4*>(importance + 4 * g) = make_float4(im[u][0], im[u][1], im[u][2], im[u][3]);
            else
                importance[g] = im[u][0];
        }
    }
    if (VEC && blockIdx.x == 0 && threadIdx.x == 0)
        for (uint64_t s = ObsGroups<VEC>(n).full * 4; s < n; ++s)
            if (state[s] != 2) importance[s] += expf(exp_arg<FQ>(scores[s] - M, t, yt)) * inv;
}

// ---------------------------------------------------------------------------
// Launchers

size_t score_rows_workspace_bytes(uint32_t, uint32_t, bool, bool) { return 0; }

hipError_t launch_score_rows(const void* tiles, uint32_t n_rows, uint32_t n_tok, uint32_t group,
                             const float* qc, const uint64_t* qs, bool exact, float* scores,
                             uint32_t* ham, void* workspace, int codec_hint, hipStream_t s) {
    if (n_rows == 0 || n_tok == 0 || group == 0) return hipSuccess;
    dim3 grid((n_tok + 255) / 256, n_rows);
    const uint4* tp = static_cast<const uint4*>(tiles);
    const size_t smem =
        (!exact && !ham && group <= kMfmaMaxGroup) ? staging_bytes(staging_rows(group)) : 0;
    const uint32_t* qsw = reinterpret_cast<const uint32_t*>(qs);
    if (!exact && !ham && group <= kMfmaMaxGroup) {
        if (group <= 4 && codec_hint == kCodecInt4Single)
            score_rows_int4_kernel<<<grid, 256, 0, s>>>(tp, n_tok, group, qc, qsw, scores);
        else if (group <= 4 && codec_hint == kCodecNF4)
            score_rows_nf4_kernel<<<grid, 256, 0, s>>>(tp, n_tok, group, qc, qsw, scores);
        else if (group <= 4)
            score_rows_fast_kernel<4><<<grid, 256, 0, s>>>(tp, n_tok, group, qc, qsw, scores);
        else if (group <= kRegStageMaxGroup)
            score_rows_fast_kernel<16><<<grid, 256, 0, s>>>(tp, n_tok, group, qc, qsw, scores);
        else if (n_tok >= kWideMaxTok)
            score_rows_kernel<false, false><<<grid, 256, smem, s>>>(tp, n_tok, group, qc, qsw, scores, ham);
        else {
            // about four workgroups per CU over all rows (two resident at a
            // time), each looping over its row's 512-tile chunks; a
            // same-box sweep put 1 024 workgroups ahead of 512 and 2 048
            const uint32_t n_chunks = (n_tok + kWideChunk - 1) / kWideChunk;
            const uint32_t per_row = std::max(1u, std::min(n_chunks, (1024u + n_rows - 1) / n_rows));
            const dim3 wgrid(per_row, n_rows);
            if (group <= 32)
                score_rows_wide_kernel<1><<<wgrid, 512, wide_image_bytes(group), s>>>(tp, n_tok, group, qc,
                                                                                   qsw, scores);
            else
                score_rows_wide_kernel<2><<<wgrid, 512, wide_image_bytes(group), s>>>(tp, n_tok, group, qc,
                                                                                   qsw, scores);
        }
        return hipGetLastError();
    }
    if (exact) {
        if (ham)
            score_rows_kernel<true, true><<<grid, 256, smem, s>>>(tp, n_tok, group, qc, qsw, scores, ham);
        else
            score_rows_kernel<true, false><<<grid, 256, smem, s>>>(tp, n_tok, group, qc, qsw, scores, ham);
    } else {
        if (ham)
            score_rows_kernel<false, true><<<grid, 256, smem, s>>>(tp, n_tok, group, qc, qsw, scores, ham);
        else
            score_rows_kernel<false, false><<<grid, 256, smem, s>>>(tp, n_tok, group, qc, qsw, scores, ham);
    }
    return hipGetLastError();
}

hipError_t launch_score_paged_topk(const void* arena, uint32_t page_shift,
                                  const uint32_t* page_table, uint32_t max_pages,
                                  const uint32_t* seq_len, const uint64_t* score_base,
                                  uint32_t n_seq, uint32_t max_len, uint32_t n_kv, uint32_t group,
                                  const float* qc, const uint64_t* qs, float* scores, uint32_t k,
                                  uint32_t* topk_idx, float* topk_val, void* workspace,
                                  hipStream_t s) {
    if (n_seq == 0 || max_len == 0) return hipSuccess;
    const auto* base = reinterpret_cast<const unsigned long long*>(score_base);
    const dim3 grid((max_len + 255) / 256, n_seq * n_kv);
    const size_t smem = group <= kMfmaMaxGroup ? staging_bytes(staging_rows(group)) : 0;
    const uint4* ap = static_cast<const uint4*>(arena);
    const uint32_t* qsw = reinterpret_cast<const uint32_t*>(qs);
    if (page_shift >= 6 && group <= kMfmaMaxGroup) {
#define SLHA_PAGED(R, SMEM)                                                                     \
    score_paged_fast_kernel<R><<<grid, 256, SMEM, s>>>(ap, page_shift, page_table, max_pages,   \
                                                       seq_len, base, n_kv, group, qc, qsw, scores)
        if (group <= 4)
            SLHA_PAGED(4, 0);
        else if (group <= kRegStageMaxGroup)
            SLHA_PAGED(16, 0);
        else
            SLHA_PAGED(0, smem);
#undef SLHA_PAGED
    } else {
        score_paged_kernel<<<grid, 256, smem, s>>>(ap, page_shift, page_table, max_pages, seq_len,
                                                base, n_kv, group, qc, qsw, scores);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || k == 0) return e;
    const uint32_t hq = n_kv * group, rows = n_seq * hq;
    const uint32_t nseg = (max_len + kTopkSeg - 1) / kTopkSeg;
    if ((uint64_t)nseg * k > kTopkMaxCandidates) return hipErrorInvalidValue;  // checked by the ABI
    uint32_t* cand_key = static_cast<uint32_t*>(workspace);
    uint32_t* cand_idx = cand_key + (size_t)rows * nseg * k;
    // Rows along x: every row's first segment is dispatched before any
    // second segment, so the workgroups of short rows that have no work in
    // the later segments gather at the end of the grid instead of diluting
    // the occupancy throughout.
    topk_segment_kernel<<<dim3(rows, nseg), kSegThreads, 0, s>>>(scores, seq_len, base, hq, k, nseg,
                                                                 cand_key, cand_idx);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    topk_merge_kernel<<<rows, kMergeThreads, (size_t)nseg * k * 8, s>>>(
        cand_key, cand_idx, seq_len, hq, k, nseg, topk_idx, topk_val);
    return hipGetLastError();
}

size_t paged_topk_workspace_bytes(uint32_t n_seq, uint32_t max_len, uint32_t n_kv,
                                  uint32_t group, uint32_t k) {
    const size_t rows = (size_t)n_seq * n_kv * group;
    const size_t nseg = (max_len + kTopkSeg - 1) / kTopkSeg;
    return rows * nseg * k * 2 * sizeof(uint32_t);
}

// Paged scoring + top-k that allocates nothing: the top-k candidate lists
// live in `scratch`, a file-scope device array of kNoAllocScratchBytes that
// every GPU the library runs on holds until the process ends. Its device
// address is looked up once per device (hipGetSymbolAddress with that device
// current) and kept; the array's name is never passed to a kernel. The
// segment kernel writes every list entry the merge reads in the same call,
// so the array needs no clearing between calls. Calls that overlap on one GPU
// (two streams, two threads) share the array and race.
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kScratchMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kScratchMaxDevices];
}  // namespace

hipError_t noalloc_scratch(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kScratchMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return hipSuccess;
}

hipError_t launch_score_paged_topk_noalloc(const void* arena, uint32_t page_shift,
                                          const uint32_t* page_table, uint32_t max_pages,
                                          const uint32_t* seq_len, const uint64_t* score_base,
                                          uint32_t n_seq, uint32_t max_len, uint32_t n_kv,
                                          uint32_t group, const float* qc, const uint64_t* qs,
                                          float* scores, uint32_t k, uint32_t* topk_idx,
                                          float* topk_val, hipStream_t s) {
    void* ws = nullptr;
    if (k > 0 && n_seq > 0 && max_len > 0) {
        if (paged_topk_workspace_bytes(n_seq, max_len, n_kv, group, k) > kNoAllocScratchBytes)
            return hipErrorInvalidValue;  // checked by the ABI with its own message
        const hipError_t e = noalloc_scratch(&ws);
        if (e != hipSuccess) return e;
    }
    return launch_score_paged_topk(arena, page_shift, page_table, max_pages, seq_len, score_base, n_seq,
                                   max_len, n_kv, group, qc, qs, scores, k, topk_idx, topk_val, ws, s);
}

namespace {
uint16_t bf16_rne(float x) {  // finite x
    uint32_t u;
    std::memcpy(&u, &x, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
float bf16_to_float(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float x;
    std::memcpy(&x, &u, 4);
    return x;
}
}  // namespace

float build_projection_pack(const float* z, void* pack) {
    uint16_t* p = static_cast<uint16_t*>(pack);
    double zmax = 0.0;
    for (int s = 0; s < kDS; ++s) {
        double n2 = 0.0;
        for (int d = 0; d < kDC; ++d) n2 += (double)z[s * kDC + d] * (double)z[s * kDC + d];
        zmax = std::max(zmax, std::sqrt(n2));
    }
    for (int sb = 0; sb < 16; ++sb)
        for (int ks = 0; ks < 4; ++ks)
            for (int lane = 0; lane < 64; ++lane)
                for (int j = 0; j < 8; ++j) {
                    // Row m of row block sb is Z row 32 (sb / 2) + 8 (m / 4) +
                    // 4 (sb % 2) + m % 4: the MFMA hands rows 4 g .. 4 g + 3
                    // to lane group g, so each lane's projections of a key
                    // fill whole bytes (byte g) of the key's sketch words.
                    const int m = lane % 16;
                    const int s = 32 * (sb / 2) + 8 * (m / 4) + 4 * (sb % 2) + m % 4;
                    const int d = 32 * ks + 8 * (lane / 16) + j;
                    const float x = z[s * kDC + d];
                    const uint16_t hi = bf16_rne(x);
                    const uint16_t mid = bf16_rne(x - bf16_to_float(hi));
                    const size_t o = ((size_t)((sb * 4 + ks) * 2) * 64 + lane) * 8 + j;
                    p[o] = hi;
                    p[o + 64 * 8] = mid;
                }
    return (float)(kEncCertRel * zmax * (1.0 + 0x1p-20));
}

hipError_t launch_encode(const void* keys, int dtype, uint64_t n_keys, uint32_t n_tok,
                         uint32_t n_kv, uint32_t pos0, int codec, int residual_mode, int warm,
                         const float* z, const void* zpack, float cert_scale, const float* diag,
                         float lambda_c, float rht_inv, void* tiles, hipStream_t s) {
    if (n_keys == 0) return hipSuccess;
    const dim3 grid((unsigned)((n_keys + 255) / 256));
    uint4* tp = static_cast<uint4*>(tiles);
    const uint4* zp = static_cast<const uint4*>(zpack);
    const bool mfma = residual_mode == kResidualR && zp != nullptr;
#define SLHA_ENC(C)                                                                              \
    if (mfma)                                                                                    \
        encode_mfma_kernel<C><<<grid, 256, 0, s>>>(keys, dtype, n_keys, n_tok, n_kv, pos0, warm, \
                                                   z, zp, cert_scale, diag, lambda_c, rht_inv,  \
                                                   tp);                                          \
    else                                                                                         \
        encode_kernel<C><<<grid, 256, 0, s>>>(keys, dtype, n_keys, n_tok, n_kv, pos0,            \
                                              residual_mode, warm, z, diag, lambda_c, rht_inv, tp)
    switch (codec) {
        case kCodecInt4Single: SLHA_ENC(kCodecInt4Single); break;
        case kCodecInt4Grouped: SLHA_ENC(kCodecInt4Grouped); break;
        case kCodecNF4: SLHA_ENC(kCodecNF4); break;
        case kCodecMixed: SLHA_ENC(kCodecMixed); break;
        case kCodecTQ3: SLHA_ENC(kCodecTQ3); break;
        case kCodecMix3: SLHA_ENC(kCodecMix3); break;
        default: return hipErrorInvalidValue;
    }
#undef SLHA_ENC
    return hipGetLastError();
}

hipError_t launch_prepare_queries(const void* q, int dtype, uint64_t n_q, const float* z,
                                  const float* diag, float rht_inv, float* qc, uint64_t* qs,
                                  hipStream_t s) {
    if (n_q == 0) return hipSuccess;
    if (n_q > 0x7FFFFFFFu) return hipErrorInvalidValue;
    prepare_query_kernel<<<(unsigned)n_q, 256, 0, s>>>(q, dtype, z, diag, rht_inv, qc, qs);
    return hipGetLastError();
}

hipError_t launch_decode(const void* tiles, uint64_t n, const float* z_or_null, float sqrt_half_pi,
                         float* out, hipStream_t s) {
    if (n == 0) return hipSuccess;
    decode_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(static_cast<const uint4*>(tiles), n,
                                                             z_or_null, sqrt_half_pi, out);
    return hipGetLastError();
}

namespace {
LearnedArgs learned_args(const LearnedProjection& lp) {
    return LearnedArgs{lp.p, lp.z, lp.diag, reinterpret_cast<const float4*>(lp.p4),
                       reinterpret_cast<const float4*>(lp.z4), lp.d, lp.d_pad, lp.rht_inv};
}
unsigned learned_grid(uint64_t n) { return (unsigned)std::min<uint64_t>(n, 1u << 20); }
constexpr size_t kLdsMaxBytes = 160 * 1024;  // LDS per workgroup on gfx950

// Dynamic LDS above the default 64 KiB needs the kernel's opt-in.
template <typename K>
hipError_t allow_lds(K kernel, size_t bytes) {
    if (bytes <= 65536) return hipSuccess;
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}
}  // namespace

hipError_t launch_learned_encode(const void* keys, int dtype, uint64_t n_keys, uint32_t n_tok,
                                 uint32_t n_kv, uint32_t pos0, int codec, int warm,
                                 const LearnedProjection& lp, float lambda_c, void* tiles,
                                 hipStream_t s) {
    if (n_keys == 0) return hipSuccess;
    const size_t lds = learned_lds_bytes(lp.d, lp.d_pad);
    uint4* out = static_cast<uint4*>(tiles);
    const LearnedArgs a = learned_args(lp);
    // Four keys per workgroup when their vectors fit in LDS, else two.
    const size_t lds4 = learned_lds_bytes4(kLearnedKeysPerBlock, lp.d, lp.d_pad);
    const size_t lds2 = learned_lds_bytes2(lp.d, lp.d_pad);
    const bool quad = lds4 <= kLdsMaxBytes && n_keys >= 4;
    const bool pair = lds2 <= kLdsMaxBytes;
#define SLHA_LEARNED_ENC(C)                                                                        \
    {                                                                                              \
        if (quad) {                                                                                \
            const hipError_t e = allow_lds(learned_encode4_kernel<C>, lds4);                        \
            if (e != hipSuccess) return e;                                                         \
            learned_encode4_kernel<C><<<learned_grid((n_keys + 3) / 4), 256, lds4, s>>>(            \
                keys, dtype, n_keys, n_tok, n_kv, pos0, warm, a, lambda_c, out);                   \
            break;                                                                                 \
        }                                                                                          \
        if (pair) {                                                                                \
            const hipError_t e = allow_lds(learned_encode2_kernel<C>, lds2);                        \
            if (e != hipSuccess) return e;                                                         \
            learned_encode2_kernel<C><<<learned_grid((n_keys + 1) / 2), 256, lds2, s>>>(            \
                keys, dtype, n_keys, n_tok, n_kv, pos0, warm, a, lambda_c, out);                   \
            break;                                                                                 \
        }                                                                                          \
        const hipError_t e = allow_lds(learned_encode_kernel<C>, lds);                              \
        if (e != hipSuccess) return e;                                                             \
        learned_encode_kernel<C><<<learned_grid(n_keys), 256, lds, s>>>(keys, dtype, n_keys, n_tok, \
                                                                        n_kv, pos0, warm, a,       \
                                                                        lambda_c, out);            \
        break;                                                                                     \
    }
    switch (codec) {
        case kCodecInt4Single: SLHA_LEARNED_ENC(kCodecInt4Single)
        case kCodecInt4Grouped: SLHA_LEARNED_ENC(kCodecInt4Grouped)
        case kCodecNF4: SLHA_LEARNED_ENC(kCodecNF4)
        case kCodecMixed: SLHA_LEARNED_ENC(kCodecMixed)
        case kCodecTQ3: SLHA_LEARNED_ENC(kCodecTQ3)
        case kCodecMix3: SLHA_LEARNED_ENC(kCodecMix3)
        default: return hipErrorInvalidValue;
    }
#undef SLHA_LEARNED_ENC
    return hipGetLastError();
}

hipError_t launch_learned_prepare(const void* q, int dtype, uint64_t n_q, const LearnedProjection& lp,
                                  float* qc, uint64_t* qs, hipStream_t s) {
    if (n_q == 0) return hipSuccess;
    const size_t lds4 = (4 * ((size_t)lp.d + lp.d_pad) + 32) * 4;
    if (lds4 <= kLdsMaxBytes && n_q >= 4) {  // four queries per workgroup
        const hipError_t e = allow_lds(learned_prepare4_kernel, lds4);
        if (e != hipSuccess) return e;
        learned_prepare4_kernel<<<learned_grid((n_q + 3) / 4), 256, lds4, s>>>(q, dtype, n_q, learned_args(lp),
                                                                                qc, qs);
        return hipGetLastError();
    }
    const size_t lds2 = learned_lds_bytes2(lp.d, lp.d_pad);
    if (lds2 <= kLdsMaxBytes) {  // two queries per workgroup
        const hipError_t e = allow_lds(learned_prepare2_kernel, lds2);
        if (e != hipSuccess) return e;
        learned_prepare2_kernel<<<learned_grid((n_q + 1) / 2), 256, lds2, s>>>(q, dtype, n_q, learned_args(lp),
                                                                                qc, qs);
        return hipGetLastError();
    }
    const size_t lds = learned_lds_bytes(lp.d, lp.d_pad);
    const hipError_t e = allow_lds(learned_prepare_kernel, lds);
    if (e != hipSuccess) return e;
    learned_prepare_kernel<<<learned_grid(n_q), 256, lds, s>>>(q, dtype, n_q, learned_args(lp), qc, qs);
    return hipGetLastError();
}

hipError_t launch_learned_decode(const void* tiles, uint64_t n, const LearnedProjection& lp,
                                 int with_residual, float sqrt_half_pi, float* out, hipStream_t s) {
    if (n == 0) return hipSuccess;
    learned_decode_kernel<<<learned_grid((n + kDecTiles - 1) / kDecTiles), 256, kDecTiles * (128 + 32) * 4, s>>>(
        static_cast<const uint4*>(tiles), n, learned_args(lp), with_residual, sqrt_half_pi, out);
    return hipGetLastError();
}

namespace {
template <int VDT, int G>
hipError_t attn_partial_dv(dim3 grid, const float* scores, const void* vals, uint32_t n_tok,
                           uint32_t group, uint32_t d_v, float scale, float* part, hipStream_t s) {
#define SLHA_DV(DV)                                                                              \
    case DV:                                                                                     \
        attn_partial_kernel<VDT, G, DV><<<grid, 256, 0, s>>>(scores, vals, n_tok, group, scale, part); \
        break;
    switch (d_v) {
        SLHA_DV(32) SLHA_DV(64) SLHA_DV(128) SLHA_DV(256)
        default: return hipErrorInvalidValue;
    }
#undef SLHA_DV
    return hipGetLastError();
}
template <int VDT>
hipError_t attn_partial_g(dim3 grid, const float* scores, const void* vals, uint32_t n_tok,
                          uint32_t group, uint32_t d_v, float scale, float* part, hipStream_t s) {
    // attn_fused_ok(group, d_v) runs attn_fused_kernel instead
    if (group <= 8) return attn_partial_dv<VDT, 8>(grid, scores, vals, n_tok, group, d_v, scale, part, s);
    return attn_partial_dv<VDT, 16>(grid, scores, vals, n_tok, group, d_v, scale, part, s);
}
hipError_t attn_partial_dispatch(dim3 grid, const float* scores, const void* vals, int v_dtype,
                                 uint32_t n_tok, uint32_t group, uint32_t d_v, float scale,
                                 float* part, hipStream_t s) {
    return v_dtype == kDtypeBF16
               ? attn_partial_g<kDtypeBF16>(grid, scores, vals, n_tok, group, d_v, scale, part, s)
               : attn_partial_g<kDtypeF32>(grid, scores, vals, n_tok, group, d_v, scale, part, s);
}
}  // namespace

size_t decode_attention_workspace_bytes(uint32_t n_rows, uint32_t n_tok, uint32_t group,
                                        uint32_t d_v) {
    const size_t n_seg = (n_tok + kAttnSeg - 1) / kAttnSeg;
    const size_t part = (size_t)n_rows * n_seg * group * attn_partial_floats(d_v) * 4;
    if (attn_fused_ok(group, d_v)) return part;
    const size_t scores = (size_t)n_rows * group * n_tok * 4;
    const size_t wide = score_rows_workspace_bytes(n_rows, group, false, false);
    return ((part + 255) & ~(size_t)255) + ((scores + 255) & ~(size_t)255) + wide;
}

hipError_t launch_decode_attention(const void* tiles, const void* vals, int v_dtype,
                                   uint32_t n_rows, uint32_t n_tok, uint32_t group, uint32_t d_v,
                                   const float* qc, const uint64_t* qs, float scale, float* out,
                                   void* workspace, hipStream_t s) {
    if (n_rows == 0 || n_tok == 0 || group == 0) return hipSuccess;
    if (group > kAttnMaxGroup || d_v < 32 || d_v > 256 || (d_v & (d_v - 1)) != 0)
        return hipErrorInvalidValue;
    const uint32_t n_seg = (n_tok + kAttnSeg - 1) / kAttnSeg;
    // workspace: partials [n_rows][n_seg][group][d_v + 4], then (unfused
    // groups only) scores [n_rows * group][n_tok] and the scorer's workspace
    char* ws = static_cast<char*>(workspace);
    float* part = reinterpret_cast<float*>(ws);
    const size_t pb = ((size_t)n_rows * n_seg * group * attn_partial_floats(d_v) * 4 + 255) & ~(size_t)255;
    float* scores = reinterpret_cast<float*>(ws + pb);
    const size_t sb = ((size_t)n_rows * group * n_tok * 4 + 255) & ~(size_t)255;
    const uint4* tp = static_cast<const uint4*>(tiles);
    const uint32_t* qsw = reinterpret_cast<const uint32_t*>(qs);
    hipError_t e = hipSuccess;
    if (attn_fused_ok(group, d_v)) {  // scores stay in LDS
        const dim3 grid(n_seg, n_rows);
#define SLHA_FUSED(VDT, DV)                                                                         \
    (group <= 4 ? attn_fused_kernel<VDT, DV, 4><<<grid, 256, 0, s>>>(tp, n_tok, group, qc, qsw, vals, scale, part) \
                : attn_fused_kernel<VDT, DV, 8><<<grid, 256, 0, s>>>(tp, n_tok, group, qc, qsw, vals, scale, part))
#define SLHA_FUSED4(VDT, DV)                                                                        \
    attn_fused_kernel<VDT, DV, 4><<<grid, 256, 0, s>>>(tp, n_tok, group, qc, qsw, vals, scale, part)
        switch ((v_dtype == kDtypeBF16 ? 1000 : 0) + (int)d_v) {
            case 32: SLHA_FUSED(kDtypeF32, 32); break;
            case 64: SLHA_FUSED(kDtypeF32, 64); break;
            case 128: SLHA_FUSED(kDtypeF32, 128); break;
            case 256: SLHA_FUSED4(kDtypeF32, 256); break;
            case 1032: SLHA_FUSED(kDtypeBF16, 32); break;
            case 1064: SLHA_FUSED(kDtypeBF16, 64); break;
            case 1128: SLHA_FUSED(kDtypeBF16, 128); break;
            case 1256: SLHA_FUSED4(kDtypeBF16, 256); break;
            default: return hipErrorInvalidValue;
        }
#undef SLHA_FUSED4
#undef SLHA_FUSED
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        attn_combine_kernel<<<dim3(n_rows * group, d_v / 16), 256, 0, s>>>(part, n_seg, group, d_v, scale, out);
        return hipGetLastError();
    }
    e = launch_score_rows(tiles, n_rows, n_tok, group, qc, qs, false, scores, nullptr, ws + sb + pb, -1, s);
    if (e != hipSuccess) return e;
    const dim3 grid(n_seg, n_rows);
    e = attn_partial_dispatch(grid, scores, vals, v_dtype, n_tok, group, d_v, scale, part, s);
    if (e != hipSuccess) return e;
    attn_combine_kernel<<<dim3(n_rows * group, d_v / 16), 256, 0, s>>>(part, n_seg, group, d_v, scale, out);
    return hipGetLastError();
}

hipError_t launch_validate(const void* tiles, uint64_t n, uint64_t* status, hipStream_t s) {
    if (n == 0) return hipSuccess;
    validate_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(
        static_cast<const uint4*>(tiles), n, reinterpret_cast<unsigned long long*>(status));
    return hipGetLastError();
}

__global__ void fill_u64_kernel(uint64_t* p, uint64_t n, uint64_t value) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = value;
}

hipError_t launch_fill_u64(uint64_t* p, uint64_t n, uint64_t value, hipStream_t s) {
    if (n == 0) return hipSuccess;
    fill_u64_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(p, n, value);
    return hipGetLastError();
}

__global__ void fill_u32_kernel(uint32_t* p, uint64_t n, uint32_t value) {
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = value;
}

hipError_t launch_fill_u32(uint32_t* p, uint64_t n, uint32_t value, hipStream_t s) {
    if (n == 0) return hipSuccess;
    fill_u32_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(p, n, value);
    return hipGetLastError();
}

hipError_t launch_eventlog_pack(const void* arena, const uint32_t* slots, const uint64_t* seqs,
                                uint64_t n, uint32_t version, void* records, hipStream_t s) {
    if (n == 0) return hipSuccess;
    eventlog_pack_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(
        static_cast<const uint4*>(arena), slots, seqs, n, version, static_cast<uint4*>(records));
    return hipGetLastError();
}

hipError_t launch_eventlog_unpack(const void* records, uint64_t n, uint32_t version,
                                  const uint32_t* dst, void* arena, uint32_t* status, hipStream_t s) {
    if (n == 0) return hipSuccess;
    eventlog_unpack_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(
        static_cast<const uint4*>(records), n, version, dst, static_cast<uint4*>(arena), status);
    return hipGetLastError();
}

hipError_t launch_tile_scatter(const void* src, const uint32_t* dst, uint64_t n, void* arena,
                               float* importance, uint8_t* state, hipStream_t s) {
    if (n == 0) return hipSuccess;
    tile_scatter_kernel<<<(unsigned)((n * 8 + 255) / 256), 256, 0, s>>>(
        static_cast<const uint4*>(src), dst, n, static_cast<uint4*>(arena), importance, state);
    return hipGetLastError();
}

size_t observe_workspace_floats() { return 3 * (size_t)kObsBlocks; }

hipError_t launch_observe_scores(const float* scores, const uint8_t* state, uint64_t n, float temperature,
                                 float* importance, float* workspace, hipStream_t s) {
    if (n == 0) return hipSuccess;
    // 16-byte score loads when the three arrays allow them (importance and
    // state are the cache's own allocations).
    const bool vec = (reinterpret_cast<uintptr_t>(scores) | reinterpret_cast<uintptr_t>(importance)) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(state) % 4 == 0;
    const uint64_t groups = vec ? n / 4 : n;
    const uint64_t need = (groups + 256 * kObsUnroll - 1) / (256 * kObsUnroll);
    const unsigned blocks = (unsigned)(need == 0 ? 1 : need < kObsBlocks ? need : kObsBlocks);
    const float t = temperature;
    // The per-slot x / t as quot<true> from one reciprocal when t is in the
    // range where that equals the division (see quot); else the division.
    const bool fq = t >= 0x1p-71f && t <= 0x1p96f;
    const float yt = fq ? 1.0f / t : 0.0f;
#define SLHA_OBS(V, F)                                                                           \
    observe_stats_kernel<V, F><<<blocks, 256, 0, s>>>(scores, state, n, t, yt, workspace);        \
    observe_apply_kernel<V, F><<<blocks, 256, 0, s>>>(scores, state, n, t, yt, workspace, importance)
    if (vec) {
        if (fq) { SLHA_OBS(true, true); } else { SLHA_OBS(true, false); }
    } else {
        if (fq) { SLHA_OBS(false, true); } else { SLHA_OBS(false, false); }
    }
#undef SLHA_OBS
    return hipGetLastError();
}

hipError_t launch_ccos_apply(void* tiles, uint8_t* state, const uint32_t* slots, uint32_t slot0, uint64_t n,
                             int op, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (op < 0 || op > 2 || (!slots && n != 1)) return hipErrorInvalidValue;
    ccos_apply_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(static_cast<uint4*>(tiles), state, slots,
                                                                 slot0, n, op);
    return hipGetLastError();
}

}  // namespace slha
