/*
 * slha_oracle.c — TEST INFRASTRUCTURE ONLY. CPU restatement of the SLHA v2
 * reference's scalar tile path (Rust crate `scirust`), used as the checker for
 * the HIP implementation. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never does.
 *
 * Build: gcc -O2 -ffp-contract=off -fno-fast-math -fPIC -shared (slhav2_amd/build.py).
 * The -ffp-contract=off flag is load-bearing: Rust never fuses a*b+c.
 *
 * Pinning: every function is checked by tests/test_oracle.py against the
 * reference's own known-answer tests (basic_usage, decode_int4,
 * effective_scale, zero-point tiles), closed forms (Hadamard matrix,
 * brute-force Hamming, float64 dot products), brute-force nearest-level
 * searches and the reference's invariants (error bounds, negation, WARM).
 */
#include "slha_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

_Static_assert(sizeof(orc_tile) == 128, "tile must be 128 bytes");

static const float NF4_CODEBOOK[16] = {
    /* constants.rs:138-141 */
    -1.0f,   -0.7075f, -0.5421f, -0.4165f, -0.3108f, -0.2158f, -0.1272f, -0.0421f,
    0.0421f, 0.1272f,  0.2158f,  0.3108f,  0.4165f,  0.5421f,  0.7075f,  1.0f,
};

#define TQ3_CODE_BYTES 48
#define TQ3_HALF_RANGE 3.5f
#define TQ3_CORRECTION 0.25f
#define MIXED_HI_DIMS 8
#define MIXED_LO_DIMS 112
#define MIXED_DIMS 120
#define MIXED_LO_GROUPS 7
#define MIX3_CODES_OFF 8
#define MIX3_CORR_OFF 50

/* ---- Rust numeric semantics ------------------------------------------- */

/* `f as i32`: saturating, NaN -> 0. */
static int32_t rs_f32_to_i32(float f) {
    if (isnan(f)) return 0;
    if (f >= 2147483648.0f) return INT32_MAX;
    if (f <= -2147483648.0f) return INT32_MIN;
    return (int32_t)f;
}

/* `f as u8`: saturating, NaN -> 0. */
static uint8_t rs_f32_to_u8(float f) {
    if (isnan(f)) return 0;
    if (f >= 255.0f) return 255;
    if (f <= 0.0f) return 0;
    return (uint8_t)f;
}

/* f32::clamp: NaN passes through. */
static float rs_clamp_f32(float x, float lo, float hi) {
    if (x < lo) x = lo;
    if (x > hi) x = hi;
    return x;
}

static int32_t clamp_i32(int32_t x, int32_t lo, int32_t hi) {
    return x < lo ? lo : (x > hi ? hi : x);
}

/* ---- rng.rs ------------------------------------------------------------ */

void orc_rng_init(orc_rng* r, uint64_t seed) { r->state = seed ^ 0x9E3779B97F4A7C15ull; } /* rng.rs:13-18 */

uint64_t orc_rng_next_u64(orc_rng* r) { /* rng.rs:22-28 */
    r->state += 0x9E3779B97F4A7C15ull;
    uint64_t z = r->state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

float orc_rng_next_unit(orc_rng* r) { /* rng.rs:32-35 */
    return (float)(orc_rng_next_u64(r) >> 40) * (1.0f / 16777216.0f);
}

float orc_rng_next_gaussian(orc_rng* r) { /* rng.rs:39-44 */
    float u1 = fmaxf(orc_rng_next_unit(r), 1.0e-7f);
    float u2 = orc_rng_next_unit(r);
    float rr = sqrtf(-2.0f * logf(u1));
    return rr * cosf(2.0f * 3.14159265358979323846f * u2);
}

void orc_rng_fill_gaussian(orc_rng* r, float* out, size_t n) { /* rng.rs:47-51 */
    for (size_t i = 0; i < n; ++i) out[i] = orc_rng_next_gaussian(r);
}

/* ---- codec/{int4,...}.rs ----------------------------------------------------- */

static float absmax_range(const float* v, int lo, int hi) {
    float m = 0.0f;
    for (int d = lo; d < hi; ++d) m = fmaxf(m, fabsf(v[d]));
    return m;
}

static void put_nibble(uint8_t* out, int byte, int odd, uint8_t nib) {
    if (!odd)
        out[byte] = (uint8_t)((out[byte] & 0xF0) | nib);
    else
        out[byte] = (uint8_t)((out[byte] & 0x0F) | (uint8_t)(nib << 4));
}

/* Steps -> (global, gs) exactly as int4.rs:43-50 / nf4.rs:32-39 / mixed.rs:28-34. */
static float group_bytes(const float* steps, uint8_t* gs) {
    float global = 0.0f;
    for (int g = 0; g < ORC_N_GROUPS; ++g) global = fmaxf(global, steps[g]);
    if (!(global > 0.0f)) global = 1.0f;
    for (int g = 0; g < ORC_N_GROUPS; ++g) {
        float r = roundf(steps[g] / global * 255.0f);
        gs[g] = rs_f32_to_u8(rs_clamp_f32(r, 1.0f, 255.0f));
    }
    return global;
}

void orc_quantize_latent(const float* v, uint8_t* out, float* scale_out) { /* int4.rs:9-24 */
    float max_abs = absmax_range(v, 0, ORC_D_C);
    float scale = max_abs > 0.0f ? max_abs / 7.0f : 1.0f;
    memset(out, 0, ORC_LATENT_BYTES);
    for (int d = 0; d < ORC_D_C; ++d) {
        int32_t q = rs_f32_to_i32(roundf(v[d] / scale));
        uint8_t nib = (uint8_t)((clamp_i32(q, -8, 7) + 8) & 0x0F);
        put_nibble(out, d >> 1, d & 1, nib);
    }
    *scale_out = scale;
}

void orc_quantize_latent_grouped(const float* v, uint8_t* out, float* global_out,
                                 uint8_t* gs) { /* int4.rs:34-63 */
    float steps[ORC_N_GROUPS];
    for (int g = 0; g < ORC_N_GROUPS; ++g)
        steps[g] = absmax_range(v, g * ORC_GROUP_DIM, (g + 1) * ORC_GROUP_DIM) / 7.0f;
    float global = group_bytes(steps, gs);
    memset(out, 0, ORC_LATENT_BYTES);
    for (int d = 0; d < ORC_D_C; ++d) {
        float eff = global * ((float)gs[d / ORC_GROUP_DIM] / 255.0f);
        int32_t q = rs_f32_to_i32(roundf(v[d] / eff));
        uint8_t nib = (uint8_t)((clamp_i32(q, -8, 7) + 8) & 0x0F);
        put_nibble(out, d >> 1, d & 1, nib);
    }
    *global_out = global;
}

uint8_t orc_nf4_nearest(float t) { /* nf4.rs:7-18 — strict '<': ties keep the lower index */
    int best = 0;
    float best_d = INFINITY;
    for (int i = 0; i < 16; ++i) {
        float dd = fabsf(t - NF4_CODEBOOK[i]);
        if (dd < best_d) {
            best_d = dd;
            best = i;
        }
    }
    return (uint8_t)best;
}

void orc_quantize_latent_nf4(const float* v, uint8_t* out, float* global_out,
                             uint8_t* gs) { /* nf4.rs:23-57 */
    float steps[ORC_N_GROUPS];
    for (int g = 0; g < ORC_N_GROUPS; ++g)
        steps[g] = absmax_range(v, g * ORC_GROUP_DIM, (g + 1) * ORC_GROUP_DIM);
    float global = group_bytes(steps, gs);
    memset(out, 0, ORC_LATENT_BYTES);
    for (int d = 0; d < ORC_D_C; ++d) {
        float eff = global * ((float)gs[d / ORC_GROUP_DIM] / 255.0f);
        float t = eff > 0.0f ? rs_clamp_f32(v[d] / eff, -1.0f, 1.0f) : 0.0f;
        put_nibble(out, d >> 1, d & 1, orc_nf4_nearest(t));
    }
    *global_out = global;
}

void orc_quantize_latent_mixed(const float* v, uint8_t* out, float* global_out,
                               uint8_t* gs) { /* mixed.rs:13-57 */
    float steps[ORC_N_GROUPS];
    steps[0] = absmax_range(v, 0, MIXED_HI_DIMS) / 127.0f;
    for (int g = 0; g < MIXED_LO_GROUPS; ++g) {
        int base = MIXED_HI_DIMS + g * ORC_GROUP_DIM;
        steps[1 + g] = absmax_range(v, base, base + ORC_GROUP_DIM) / 7.0f;
    }
    float global = group_bytes(steps, gs);
    memset(out, 0, ORC_LATENT_BYTES);
    float eff_hi = global * ((float)gs[0] / 255.0f);
    for (int d = 0; d < MIXED_HI_DIMS; ++d) {
        int32_t q = rs_f32_to_i32(roundf(v[d] / eff_hi));
        out[d] = (uint8_t)(clamp_i32(q, -128, 127) + 128);
    }
    for (int ld = 0; ld < MIXED_LO_DIMS; ++ld) {
        int d = MIXED_HI_DIMS + ld;
        float eff = global * ((float)gs[1 + ld / ORC_GROUP_DIM] / 255.0f);
        int32_t q = rs_f32_to_i32(roundf(v[d] / eff));
        uint8_t nib = (uint8_t)((clamp_i32(q, -8, 7) + 8) & 0x0F);
        put_nibble(out, MIXED_HI_DIMS + (ld >> 1), ld & 1, nib);
    }
    *global_out = global;
}

/* One TQ3 grid code + correction bit, tq3.rs:31-46 / mix3.rs:44-58. */
static void tq3_put(uint8_t* out, int codes_off, int corr_off, int ld, float val, float eff) {
    float t = val / eff;
    uint8_t code = (uint8_t)clamp_i32(rs_f32_to_i32(roundf(t + TQ3_HALF_RANGE)), 0, 7);
    int bit = 3 * ld;
    int byte = codes_off + (bit >> 3);
    int shift = bit & 7;
    out[byte] |= (uint8_t)(code << shift);
    if (shift > 5) out[byte + 1] |= (uint8_t)(code >> (8 - shift));
    float level = (float)code - TQ3_HALF_RANGE;
    if (t - level > 0.0f) out[corr_off + (ld >> 3)] |= (uint8_t)(1u << (ld & 7));
}

void orc_quantize_latent_tq3(const float* v, uint8_t* out, float* global_out,
                             uint8_t* gs) { /* tq3.rs:10-49 */
    float steps[ORC_N_GROUPS];
    for (int g = 0; g < ORC_N_GROUPS; ++g)
        steps[g] = absmax_range(v, g * ORC_GROUP_DIM, (g + 1) * ORC_GROUP_DIM) / TQ3_HALF_RANGE;
    float global = group_bytes(steps, gs);
    memset(out, 0, ORC_LATENT_BYTES);
    for (int d = 0; d < ORC_D_C; ++d) {
        float eff = global * ((float)gs[d / ORC_GROUP_DIM] / 255.0f);
        tq3_put(out, 0, TQ3_CODE_BYTES, d, v[d], eff);
    }
    *global_out = global;
}

void orc_quantize_latent_mix3(const float* v, uint8_t* out, float* global_out,
                              uint8_t* gs) { /* mix3.rs:11-62 */
    float steps[ORC_N_GROUPS];
    steps[0] = absmax_range(v, 0, MIXED_HI_DIMS) / 127.0f;
    for (int g = 0; g < MIXED_LO_GROUPS; ++g) {
        int base = MIXED_HI_DIMS + g * ORC_GROUP_DIM;
        steps[1 + g] = absmax_range(v, base, base + ORC_GROUP_DIM) / TQ3_HALF_RANGE;
    }
    float global = group_bytes(steps, gs);
    memset(out, 0, ORC_LATENT_BYTES);
    float eff_hi = global * ((float)gs[0] / 255.0f);
    for (int d = 0; d < MIXED_HI_DIMS; ++d) {
        int32_t q = rs_f32_to_i32(roundf(v[d] / eff_hi));
        out[d] = (uint8_t)(clamp_i32(q, -128, 127) + 128);
    }
    for (int ld = 0; ld < MIXED_LO_DIMS; ++ld) {
        float eff = global * ((float)gs[1 + ld / ORC_GROUP_DIM] / 255.0f);
        tq3_put(out, MIX3_CODES_OFF, MIX3_CORR_OFF, ld, v[MIXED_HI_DIMS + ld], eff);
    }
    *global_out = global;
}

/* ---- tile.rs ----------------------------------------------------------- */

float orc_group_scale(const orc_tile* t, int d) { /* tile.rs:133-135 */
    return t->scale * ((float)t->group_scales[d / ORC_GROUP_DIM] / 255.0f);
}

/* Mixed/MIX3 sections scale as (scale * gs) / 255 — tile.rs:169,175,220,245. */
static float section_scale(const orc_tile* t, int g) {
    return t->scale * (float)t->group_scales[g] / 255.0f;
}

static float tq3_level(const uint8_t* lk, int codes_off, int codes_end, int corr_off, int ld,
                       int nocorr) {
    int bit = 3 * ld;
    int byte = codes_off + (bit >> 3);
    int shift = bit & 7;
    uint16_t lo = lk[byte];
    uint16_t hi = (byte + 1 < codes_end) ? (uint16_t)(lk[byte + 1] << 8) : 0;
    int code = ((lo | hi) >> shift) & 0x7;
    float level = (float)code - TQ3_HALF_RANGE;
    if (!nocorr) {
        int corr = (lk[corr_off + (ld >> 3)] >> (ld & 7)) & 1;
        float sign = corr == 1 ? 1.0f : -1.0f;
        level += sign * TQ3_CORRECTION;
    }
    return level;
}

float orc_dequant_at(const orc_tile* t, int d) { /* tile.rs:141-246 */
    const uint8_t* lk = t->latent_kv;
    int nocorr = (t->flags & ORC_FLAG_TQ3_NOCORR) != 0;
    if (t->flags & ORC_FLAG_MIXED) { /* :166-179 */
        if (d < MIXED_HI_DIMS) return (float)((int)lk[d] - 128) * section_scale(t, 0);
        if (d < MIXED_DIMS) {
            int ld = d - MIXED_HI_DIMS;
            uint8_t byte = lk[MIXED_HI_DIMS + (ld >> 1)];
            int nib = (ld & 1) == 0 ? (byte & 0x0F) : (byte >> 4);
            return (float)(nib - 8) * section_scale(t, 1 + ld / ORC_GROUP_DIM);
        }
        return 0.0f;
    }
    if (t->flags & ORC_FLAG_TQ3) /* :187-207 */
        return tq3_level(lk, 0, TQ3_CODE_BYTES, TQ3_CODE_BYTES, d, nocorr) * orc_group_scale(t, d);
    if (t->flags & ORC_FLAG_MIX3) { /* :217-246 */
        if (d < MIXED_HI_DIMS) return (float)((int)lk[d] - 128) * section_scale(t, 0);
        if (d >= MIXED_DIMS) return 0.0f;
        int ld = d - MIXED_HI_DIMS;
        float level = tq3_level(lk, MIX3_CODES_OFF, MIX3_CORR_OFF, MIX3_CORR_OFF, ld, nocorr);
        return level * section_scale(t, 1 + ld / ORC_GROUP_DIM);
    }
    uint8_t byte = lk[d >> 1];
    int nib = (d & 1) == 0 ? (byte & 0x0F) : (byte >> 4);
    float level = (t->flags & ORC_FLAG_NF4) ? NF4_CODEBOOK[nib] : (float)(nib - 8);
    return level * orc_group_scale(t, d);
}

void orc_dequant_latent(const orc_tile* t, float* out) { /* tile.rs:249-255 */
    for (int d = 0; d < ORC_D_C; ++d) out[d] = orc_dequant_at(t, d);
}

uint32_t orc_hamming(const uint64_t* a, const uint64_t* b) { /* simd.rs:1253-1259 */
    uint32_t h = 0;
    for (int w = 0; w < ORC_RESIDUAL_WORDS; ++w) h += (uint32_t)__builtin_popcountll(a[w] ^ b[w]);
    return h;
}

float orc_residual_term(const orc_tile* t, const uint64_t* q_sign) { /* tile.rs:261-264 */
    uint32_t ham = orc_hamming(q_sign, t->residual_bitmap);
    return t->dynamic_lambda * ((float)ORC_D_S - 2.0f * (float)ham);
}

float orc_compute_score_scalar(const orc_tile* t, const float* q, const uint64_t* qs) { /* tile.rs:267-281 */
    float k[ORC_D_C];
    orc_dequant_latent(t, k);
    float coarse = 0.0f;
    for (int d = 0; d < ORC_D_C; ++d) coarse += q[d] * k[d];
    if (t->flags & ORC_FLAG_WARM) return coarse;
    return coarse + orc_residual_term(t, qs);
}

/* ---- scenario.rs / learned.rs sign-LSH --------------------------------- */

void orc_projection_fill(float* z, size_t d_pad, uint64_t seed) { /* scenario.rs:59-64 */
    orc_rng r;
    orc_rng_init(&r, seed);
    orc_rng_fill_gaussian(&r, z, (size_t)ORC_D_S * d_pad);
}

void orc_sign_bits(const float* z, size_t d_pad, const float* v, uint64_t* out) { /* scenario.rs:70-83 */
    for (int w = 0; w < ORC_RESIDUAL_WORDS; ++w) out[w] = 0;
    for (int s = 0; s < ORC_D_S; ++s) {
        const float* row = z + (size_t)s * d_pad;
        float acc = 0.0f;
        for (size_t k = 0; k < d_pad; ++k) acc += row[k] * v[k];
        if (acc < 0.0f) out[s >> 6] |= 1ull << (s & 63);
    }
}

/* ---- incoherence.rs ---------------------------------------------------- */

size_t orc_next_pow2(size_t n) { /* :29-35 */
    size_t p = 1;
    while (p < n) p <<= 1;
    return p;
}

void orc_fwht_inplace(float* v, size_t n) { /* :45-70 */
    for (size_t h = 1; h < n; h <<= 1) {
        for (size_t i = 0; i < n; i += h << 1) {
            for (size_t j = i; j < i + h; ++j) {
                float a = v[j], b = v[j + h];
                v[j] = a + b;
                v[j + h] = a - b;
            }
        }
    }
    float inv = 1.0f / sqrtf((float)n);
    for (size_t i = 0; i < n; ++i) v[i] *= inv;
}

void orc_rht_diag(float* diag, size_t d_pad, uint64_t seed) { /* :89-98 */
    orc_rng r;
    orc_rng_init(&r, seed);
    for (size_t i = 0; i < d_pad; ++i) diag[i] = orc_rng_next_unit(&r) < 0.5f ? -1.0f : 1.0f;
}

void orc_rht_transform(const float* diag, size_t d, size_t d_pad, const float* v,
                       float* out) { /* :114-125 */
    for (size_t i = 0; i < d; ++i) out[i] = v[i];
    for (size_t i = d; i < d_pad; ++i) out[i] = 0.0f;
    for (size_t i = 0; i < d_pad; ++i) out[i] *= diag[i];
    orc_fwht_inplace(out, d_pad);
}

/* ---- metrics.rs / scenario.rs ------------------------------------------ */

float orc_rms(const float* v, size_t n) { /* metrics.rs:207-226 */
    if (n == 0) return 0.0f;
    for (size_t i = 0; i < n; ++i)
        if (!isfinite(v[i])) return NAN;
    double acc = 0.0;
    for (size_t i = 0; i < n; ++i) {
        double x = (double)v[i];
        acc += x * x;
    }
    return (float)sqrt(acc / (double)n);
}

float orc_analytic_lambda_c(void) { /* scenario.rs:30-32 */
    return sqrtf(3.14159265358979323846f / (2.0f * (float)ORC_D_S));
}

/* ---- head_dim-128 encode (build-defined composition of scenario.rs:95-114) */

int orc_encode_key(const float* key, int codec, int residual_mode, const float* z,
                   const float* rht_diag, uint32_t position, uint16_t head_id, int warm,
                   orc_tile* out) {
    orc_tile t;
    memset(&t, 0, sizeof t);
    uint16_t codec_flag = 0;
    switch (codec) { /* learned.rs:360-385 */
        case ORC_CODEC_INT4_SINGLE:
            orc_quantize_latent(key, t.latent_kv, &t.scale);
            memset(t.group_scales, 255, ORC_N_GROUPS);
            break;
        case ORC_CODEC_INT4_GROUPED:
            orc_quantize_latent_grouped(key, t.latent_kv, &t.scale, t.group_scales);
            break;
        case ORC_CODEC_NF4:
            orc_quantize_latent_nf4(key, t.latent_kv, &t.scale, t.group_scales);
            codec_flag = ORC_FLAG_NF4;
            break;
        case ORC_CODEC_MIXED:
            orc_quantize_latent_mixed(key, t.latent_kv, &t.scale, t.group_scales);
            codec_flag = ORC_FLAG_MIXED;
            break;
        case ORC_CODEC_TQ3:
            orc_quantize_latent_tq3(key, t.latent_kv, &t.scale, t.group_scales);
            codec_flag = ORC_FLAG_TQ3;
            break;
        case ORC_CODEC_MIX3:
            orc_quantize_latent_mix3(key, t.latent_kv, &t.scale, t.group_scales);
            codec_flag = ORC_FLAG_MIX3;
            break;
        default:
            return -4;
    }
    t.flags = (uint16_t)(codec_flag | (warm ? ORC_FLAG_WARM : 0));
    if (residual_mode == ORC_RESIDUAL_R) {
        float e[ORC_D_C], buf[ORC_D_C];
        for (int d = 0; d < ORC_D_C; ++d) e[d] = key[d] - orc_dequant_at(&t, d);
        if (rht_diag)
            orc_rht_transform(rht_diag, ORC_D_C, ORC_D_C, e, buf);
        else
            memcpy(buf, e, sizeof buf);
        orc_sign_bits(z, ORC_D_C, buf, t.residual_bitmap);
        t.residual_sigma = orc_rms(e, ORC_D_C);
        t.dynamic_lambda = t.residual_sigma * orc_analytic_lambda_c();
    } else if (residual_mode != ORC_RESIDUAL_Z) {
        return -3;
    }
    t.token_id = position;
    t.position = position;
    t.head_id = head_id;
    *out = t;
    return 0;
}

void orc_query_sign(const float* q, const float* z, const float* rht_diag, uint64_t* out) {
    float buf[ORC_D_C];
    if (rht_diag)
        orc_rht_transform(rht_diag, ORC_D_C, ORC_D_C, q, buf);
    else
        memcpy(buf, q, sizeof buf);
    orc_sign_bits(z, ORC_D_C, buf, out);
}

/* ---- learned.rs (d > 128, projection loaded from .slhw: scale_k = 1) ---- */

static float orc_evec_dot(const float* p, size_t d, int k, const float* v) { /* :257-265 */
    const float* row = p + (size_t)k * d;
    float acc = 0.0f;
    for (size_t i = 0; i < d; ++i) acc += row[i] * v[i];
    return acc;
}

void orc_learned_latent(const float* p, size_t d, const float* key, float* h) { /* :267-273 latent */
    for (int k = 0; k < ORC_D_C; ++k) h[k] = orc_evec_dot(p, d, k, key) / 1.0f;
}

void orc_learned_query_coarse(const float* p, size_t d, const float* q, float* out) { /* :267-273 */
    for (int k = 0; k < ORC_D_C; ++k) out[k] = orc_evec_dot(p, d, k, q) * 1.0f;
}

void orc_learned_reconstruct(const float* p, size_t d, const float* h, float* out) { /* :276-286 */
    for (size_t i = 0; i < d; ++i) out[i] = 0.0f;
    for (int k = 0; k < ORC_D_C; ++k) {
        const float w = h[k] * 1.0f;
        const float* row = p + (size_t)k * d;
        for (size_t i = 0; i < d; ++i) out[i] += w * row[i];
    }
}

/* sign_bits (:326-347): Z [256][d_pad] against RHT(v) or v itself. */
static void orc_learned_sign_bits(const float* z, const float* diag, size_t d, size_t d_pad,
                                  const float* v, uint64_t* out) {
    float* buf = (float*)malloc(d_pad * sizeof(float));
    if (diag)
        orc_rht_transform(diag, d, d_pad, v, buf);
    else
        memcpy(buf, v, d * sizeof(float));
    orc_sign_bits(z, d_pad, buf, out);
    free(buf);
}

void orc_learned_query(const float* p, const float* z, const float* diag, size_t d, size_t d_pad,
                       const float* q, float* q_coarse, uint64_t* q_sign) {
    orc_learned_query_coarse(p, d, q, q_coarse);
    orc_learned_sign_bits(z, diag, d, d_pad, q, q_sign);
}

int orc_learned_encode(const float* p, const float* z, const float* diag, size_t d, size_t d_pad,
                       const float* key, uint32_t position, int codec, int warm,
                       orc_tile* out) { /* encode_with, :353-408 */
    float h[ORC_D_C];
    orc_learned_latent(p, d, key, h);
    orc_tile t;
    /* codes, scale, gs and flags as the head_dim-128 encoder, mode Z */
    int rc = orc_encode_key(h, codec, ORC_RESIDUAL_Z, NULL, NULL, position, 0, warm, &t);
    if (rc) return rc;
    float* recon = (float*)malloc(d * sizeof(float));
    float* e = (float*)malloc(d * sizeof(float));
    orc_learned_reconstruct(p, d, h, recon); /* residual from the un-quantised latent */
    for (size_t i = 0; i < d; ++i) e[i] = key[i] - recon[i];
    orc_learned_sign_bits(z, diag, d, d_pad, e, t.residual_bitmap);
    float acc = 0.0f; /* sum::<f32>() of e_i * e_i, then / d, sqrt (f32) */
    for (size_t i = 0; i < d; ++i) acc += e[i] * e[i];
    t.residual_sigma = sqrtf(acc / (float)d);
    t.dynamic_lambda = t.residual_sigma * orc_analytic_lambda_c();
    free(recon);
    free(e);
    *out = t;
    return 0;
}

void orc_learned_decode(const float* p, const float* z, size_t d, size_t d_pad, int has_rht,
                        const orc_tile* t, int with_residual, float* out) { /* :276-320 */
    float h[ORC_D_C];
    orc_dequant_latent(t, h);
    orc_learned_reconstruct(p, d, h, out);
    if (!with_residual || has_rht) return;
    const float scale = t->residual_sigma * sqrtf(3.14159265358979323846f / 2.0f) / (float)ORC_D_S;
    for (int s = 0; s < ORC_D_S; ++s) {
        const float sign = ((t->residual_bitmap[s >> 6] >> (s & 63)) & 1) ? -1.0f : 1.0f;
        const float* row = z + (size_t)s * d_pad;
        for (size_t i = 0; i < d; ++i) out[i] += sign * scale * row[i];
    }
}

/* ---- metrics.rs:338-409 softmax_into; benchmark_decode.rs:29-38 aggregate_v */

void orc_softmax_into(const float* scores, size_t n, float scale, float* out) {
    if (n == 0) return;
    if (!isfinite(scale)) {
        for (size_t i = 0; i < n; ++i) out[i] = 0.0f;
        return;
    }
    const double sc = (double)scale;
    double maximum = -INFINITY;
    size_t pos_inf = 0;
    for (size_t i = 0; i < n; ++i) {
        const double logit = (double)scores[i] * sc;
        if (isnan(scores[i]) || isnan(logit)) {
            for (size_t k = 0; k < n; ++k) out[k] = 0.0f;
            return;
        }
        if (isinf(logit) && logit > 0.0) ++pos_inf;
        maximum = fmax(maximum, logit);
    }
    if (pos_inf > 0) {
        const float prob = 1.0f / (float)pos_inf;
        for (size_t i = 0; i < n; ++i) {
            const double logit = (double)scores[i] * sc;
            out[i] = (isinf(logit) && logit > 0.0) ? prob : 0.0f;
        }
        return;
    }
    if (isinf(maximum) && maximum < 0.0) {
        for (size_t i = 0; i < n; ++i) out[i] = 0.0f;
        return;
    }
    double sum = 0.0;
    for (size_t i = 0; i < n; ++i) {
        const double e = exp((double)scores[i] * sc - maximum);
        out[i] = (float)e;
        sum += e;
    }
    if (!isfinite(sum) || sum <= 0.0) {
        for (size_t i = 0; i < n; ++i) out[i] = 0.0f;
        return;
    }
    for (size_t i = 0; i < n; ++i) out[i] = (float)((double)out[i] / sum);
    double rounded = 0.0;
    for (size_t i = 0; i < n; ++i) rounded += (double)out[i];
    if (isfinite(rounded) && rounded > 0.0)
        for (size_t i = 0; i < n; ++i) out[i] = (float)((double)out[i] / rounded);
}

void orc_aggregate_v(const float* weights, const float* values, size_t n, size_t d_v, float* out) {
    for (size_t j = 0; j < d_v; ++j) out[j] = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        const float* row = values + i * d_v;
        for (size_t j = 0; j < d_v; ++j) out[j] += weights[i] * row[j];
    }
}

int orc_encode_batch(const float* keys, size_t n, int codec, int residual_mode, const float* z,
                     const float* rht_diag, uint32_t pos0, uint16_t head_id, orc_tile* out) {
    for (size_t i = 0; i < n; ++i) {
        int rc = orc_encode_key(keys + i * ORC_D_C, codec, residual_mode, z, rht_diag,
                                pos0 + (uint32_t)i, head_id, 0, out + i);
        if (rc) return rc;
    }
    return 0;
}

void orc_score_batch(const orc_tile* tiles, size_t n, const float* q, const uint64_t* qs,
                     float* scores, uint32_t* hamming) {
    for (size_t i = 0; i < n; ++i) {
        if (scores) scores[i] = orc_compute_score_scalar(tiles + i, q, qs);
        if (hamming) hamming[i] = orc_hamming(qs, tiles[i].residual_bitmap);
    }
}

/* ---- slha-c validation ------------------------------------------------- */

int orc_validate_tile(const orc_tile* t) { /* lib.rs:244-286 */
    const uint16_t known = ORC_FLAG_WARM | ORC_FLAG_NF4 | ORC_FLAG_MIXED | ORC_FLAG_TQ3 |
                           ORC_FLAG_TQ3_NOCORR | ORC_FLAG_MIX3;
    const uint16_t codecs = ORC_FLAG_NF4 | ORC_FLAG_MIXED | ORC_FLAG_TQ3 | ORC_FLAG_MIX3;
    if (t->flags & (uint16_t)~known) return -6;
    if (__builtin_popcount(t->flags & codecs) > 1) return -6;
    if ((t->flags & ORC_FLAG_TQ3_NOCORR) && !(t->flags & (ORC_FLAG_TQ3 | ORC_FLAG_MIX3))) return -6;
    if (!isfinite(t->scale) || !isfinite(t->dynamic_lambda) || !isfinite(t->residual_sigma))
        return -5;
    if (t->scale < 0.0f || t->dynamic_lambda < 0.0f || t->residual_sigma < 0.0f) return -6;
    return 0;
}

/* ---- ccos.rs ----------------------------------------------------------- */

void orc_page_out(orc_tile* t) { /* ccos.rs:369-378 */
    memset(t->residual_bitmap, 0, sizeof t->residual_bitmap);
    t->dynamic_lambda = 0.0f;
    t->flags |= ORC_FLAG_WARM;
}

int orc_drop_correction(orc_tile* t) { /* ccos.rs:386-397 */
    int n = (t->flags & ORC_FLAG_TQ3) ? 16 : ((t->flags & ORC_FLAG_MIX3) ? 14 : 0);
    if (n == 0 || (t->flags & ORC_FLAG_TQ3_NOCORR)) return 0;
    memset(t->latent_kv + ORC_LATENT_BYTES - n, 0, (size_t)n);
    t->flags |= ORC_FLAG_TQ3_NOCORR;
    return 1;
}

/* ---- top-k ------------------------------------------------------------- */

typedef struct {
    float v;
    uint32_t i;
} scored;

static int scored_cmp(const void* a, const void* b) {
    const scored* x = (const scored*)a;
    const scored* y = (const scored*)b;
    if (x->v > y->v) return -1;
    if (x->v < y->v) return 1;
    return x->i < y->i ? -1 : (x->i > y->i);
}

void orc_topk(const float* scores, size_t n, size_t k, uint32_t* idx_out, float* val_out) {
    scored* all = (scored*)malloc(n * sizeof(scored) + 1);
    for (size_t i = 0; i < n; ++i) {
        all[i].v = scores[i];
        all[i].i = (uint32_t)i;
    }
    qsort(all, n, sizeof(scored), scored_cmp);
    for (size_t j = 0; j < k; ++j) {
        if (j < n) {
            idx_out[j] = all[j].i;
            if (val_out) val_out[j] = all[j].v;
        } else {
            idx_out[j] = 0xFFFFFFFFu;
            if (val_out) val_out[j] = -INFINITY;
        }
    }
    free(all);
}

/* ------------------------------------------------------------------------ */
/* EventLog records (eventlog.rs:82-100, 148-170, 330-352). */

uint32_t orc_fnv1a(const uint8_t* p, size_t n) {
    uint32_t h = 0x811C9DC5u;
    for (size_t i = 0; i < n; ++i) {
        h ^= p[i];
        h *= 0x01000193u;
    }
    return h;
}

static void put_le(uint8_t* out, size_t* o, uint64_t v, int nbytes) {
    for (int b = 0; b < nbytes; ++b) out[(*o)++] = (uint8_t)(v >> (8 * b));
}

void orc_tile_to_bytes(const orc_tile* t, uint8_t* out) {
    size_t o = 0;
    for (int i = 0; i < ORC_LATENT_BYTES; ++i) out[o++] = t->latent_kv[i];
    for (int w = 0; w < ORC_RESIDUAL_WORDS; ++w) put_le(out, &o, t->residual_bitmap[w], 8);
    uint32_t u;
    memcpy(&u, &t->scale, 4);
    put_le(out, &o, u, 4);
    memcpy(&u, &t->dynamic_lambda, 4);
    put_le(out, &o, u, 4);
    memcpy(&u, &t->residual_sigma, 4);
    put_le(out, &o, u, 4);
    put_le(out, &o, t->token_id, 4);
    put_le(out, &o, t->position, 4);
    put_le(out, &o, t->head_id, 2);
    put_le(out, &o, t->flags, 2);
    for (int g = 0; g < ORC_N_GROUPS; ++g) out[o++] = t->group_scales[g];
}

uint32_t orc_record_checksum(uint64_t seq, uint32_t slot, const uint8_t* tile_bytes) {
    uint8_t buf[8 + 4 + 128];
    size_t o = 0;
    put_le(buf, &o, seq, 8);
    put_le(buf, &o, slot, 4);
    memcpy(buf + o, tile_bytes, 128);
    return orc_fnv1a(buf, sizeof buf);
}

void orc_eventlog_record(uint64_t seq, uint32_t slot, const orc_tile* t, uint32_t version,
                         uint8_t* out) {
    uint8_t tb[128];
    orc_tile_to_bytes(t, tb);
    size_t o = 0;
    put_le(out, &o, seq, 8);
    put_le(out, &o, slot, 4);
    put_le(out, &o, version == 2 ? orc_record_checksum(seq, slot, tb) : 0u, 4);
    memcpy(out + o, tb, 128);
}

/* ------------------------------------------------------------------------ */
/* CCOS observe_scores (ccos.rs:257-300), sequential f32 as the reference. */

void orc_observe_scores(const uint32_t* slots, const float* scores, size_t n, const uint8_t* live,
                        size_t n_slots, float temperature, float* importance) {
    if (n == 0 || !isfinite(temperature) || temperature <= 0.0f) return;
    size_t n_live = 0;
    float m = -INFINITY;
    for (size_t i = 0; i < n; ++i) {
        if (slots[i] >= n_slots || !live[slots[i]]) continue;
        if (!isfinite(scores[i])) return;
        ++n_live;
        m = fmaxf(m, scores[i]);
    }
    if (n_live == 0) return;
    float sum = 0.0f;
    float* w = (float*)malloc(n * sizeof(float));
    if (!w) return;
    for (size_t i = 0; i < n; ++i) {
        w[i] = 0.0f;
        if (slots[i] >= n_slots || !live[slots[i]]) continue;
        w[i] = expf((scores[i] - m) / temperature);
        sum += w[i];
    }
    if (isfinite(sum) && sum > 0.0f) {
        const float inv = 1.0f / sum;
        for (size_t i = 0; i < n; ++i)
            if (slots[i] < n_slots && live[slots[i]]) importance[slots[i]] += w[i] * inv;
    }
    free(w);
}
