/*
 * slha_oracle.h — CPU restatement of the SLHA v2 tile path, used ONLY as a
 * test checker (tests/, __graft_entry__.smoke(), bench.py's cpu_baseline leg).
 * Nothing in the product library links, loads or calls this code.
 *
 * Every function restates one function of the Rust reference (scirust) with
 * the reference's numeric semantics:
 *   - no FMA contraction (built with -ffp-contract=off), sequential f32 sums;
 *   - f32::round == roundf (half away from zero);
 *   - `as i32` / `as u8` saturate and map NaN to 0;
 *   - f32::max == fmaxf (the non-NaN operand wins);
 *   - correctly rounded '/' and sqrtf.
 */
#ifndef SLHA_ORACLE_H
#define SLHA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_D_C 128
#define ORC_D_S 256
#define ORC_LATENT_BYTES 64
#define ORC_RESIDUAL_WORDS 4
#define ORC_N_GROUPS 8
#define ORC_GROUP_DIM 16

/* constants.rs:22-48 */
#define ORC_FLAG_WARM 0x01u
#define ORC_FLAG_NF4 0x02u
#define ORC_FLAG_MIXED 0x04u
#define ORC_FLAG_TQ3 0x08u
#define ORC_FLAG_TQ3_NOCORR 0x10u
#define ORC_FLAG_MIX3 0x20u

/* slha.h:32-37 codec ids */
#define ORC_CODEC_INT4_SINGLE 0
#define ORC_CODEC_INT4_GROUPED 1
#define ORC_CODEC_NF4 2
#define ORC_CODEC_MIXED 3
#define ORC_CODEC_TQ3 4
#define ORC_CODEC_MIX3 5

/* tile.rs:52-77 — 128-byte tile, byte map latent@0 residual@64 scale@96
 * lambda@100 sigma@104 token@108 position@112 head@116 flags@118 gs@120. */
typedef struct __attribute__((aligned(64))) {
    uint8_t latent_kv[64];
    uint64_t residual_bitmap[4];
    float scale;
    float dynamic_lambda;
    float residual_sigma;
    uint32_t token_id;
    uint32_t position;
    uint16_t head_id;
    uint16_t flags;
    uint8_t group_scales[8];
} orc_tile;

/* rng.rs:7-52 — SplitMix64 + Box–Muller. */
typedef struct {
    uint64_t state;
} orc_rng;
void orc_rng_init(orc_rng* r, uint64_t seed);
uint64_t orc_rng_next_u64(orc_rng* r);
float orc_rng_next_unit(orc_rng* r);
float orc_rng_next_gaussian(orc_rng* r);
void orc_rng_fill_gaussian(orc_rng* r, float* out, size_t n);

/* codec/{int4,nf4,mixed,tq3,mix3}.rs — the six latent quantisers. */
void orc_quantize_latent(const float* v, uint8_t* out, float* scale);
void orc_quantize_latent_grouped(const float* v, uint8_t* out, float* global, uint8_t* gs);
uint8_t orc_nf4_nearest(float t);
void orc_quantize_latent_nf4(const float* v, uint8_t* out, float* global, uint8_t* gs);
void orc_quantize_latent_mixed(const float* v, uint8_t* out, float* global, uint8_t* gs);
void orc_quantize_latent_tq3(const float* v, uint8_t* out, float* global, uint8_t* gs);
void orc_quantize_latent_mix3(const float* v, uint8_t* out, float* global, uint8_t* gs);

/* tile.rs:133-281 — dequant and the scalar eq. 2.3 score. */
float orc_group_scale(const orc_tile* t, int d);
float orc_dequant_at(const orc_tile* t, int d);
void orc_dequant_latent(const orc_tile* t, float* out);
uint32_t orc_hamming(const uint64_t* a, const uint64_t* b);
float orc_residual_term(const orc_tile* t, const uint64_t* q_sign);
float orc_compute_score_scalar(const orc_tile* t, const float* q_coarse, const uint64_t* q_sign);

/* scenario.rs:54-84, learned.rs:326-347 — sign-LSH projection. */
void orc_projection_fill(float* z, size_t d_pad, uint64_t seed);
void orc_sign_bits(const float* z, size_t d_pad, const float* v, uint64_t* out);

/* incoherence.rs:29-126 — randomised Hadamard transform. */
size_t orc_next_pow2(size_t n);
void orc_fwht_inplace(float* v, size_t n);
void orc_rht_diag(float* diag, size_t d_pad, uint64_t seed);
void orc_rht_transform(const float* diag, size_t d, size_t d_pad, const float* v, float* out);

/* metrics.rs:207-226 and scenario.rs:30-32. */
float orc_rms(const float* v, size_t n);
float orc_analytic_lambda_c(void);

/* Head_dim-128 tile encode (mode R: e = k - dequant(k); mode Z: e = 0).
 * rht_diag == NULL disables the RHT. Returns 0 or a negative status. */
#define ORC_RESIDUAL_Z 0
#define ORC_RESIDUAL_R 1
int orc_encode_key(const float* key, int codec, int residual_mode, const float* z,
                   const float* rht_diag, uint32_t position, uint16_t head_id, int warm,
                   orc_tile* out);
void orc_query_sign(const float* q, const float* z, const float* rht_diag, uint64_t* out);

/* learned.rs:257-408 — LearnedModel with a loaded projection (d > 128):
 * P [128][d] row-major, per-component scale 1, Z [256][d_pad], RHT diagonal
 * [d_pad] or NULL. orc_learned_encode returns 0 or a negative status. */
void orc_learned_latent(const float* p, size_t d, const float* key, float* h);
void orc_learned_query_coarse(const float* p, size_t d, const float* q, float* out);
void orc_learned_reconstruct(const float* p, size_t d, const float* h, float* out);
void orc_learned_query(const float* p, const float* z, const float* diag, size_t d, size_t d_pad,
                       const float* q, float* q_coarse, uint64_t* q_sign);
int orc_learned_encode(const float* p, const float* z, const float* diag, size_t d, size_t d_pad,
                       const float* key, uint32_t position, int codec, int warm, orc_tile* out);
void orc_learned_decode(const float* p, const float* z, size_t d, size_t d_pad, int has_rht,
                        const orc_tile* t, int with_residual, float* out);

/* metrics.rs:338-409 — numerically stable softmax of scores * scale (f64),
 * with its contract: non-finite scale or a NaN score -> all zero; +inf logits
 * share the mass equally; all logits -inf -> all zero.
 * benchmark_decode.rs:29-38 — out[d] = sum_i w_i V[i][d] (f32, in order). */
void orc_softmax_into(const float* scores, size_t n, float scale, float* out);
void orc_aggregate_v(const float* weights, const float* values, size_t n, size_t d_v, float* out);

/* eventlog.rs:82-100 — tile_to_bytes: the fields in the byte map's order,
 * each little-endian. eventlog.rs:148-170 — FNV-1a 32 (offset 0x811C9DC5,
 * prime 0x01000193) over seq (8 LE bytes) || slot (4) || tile bytes (128).
 * orc_eventlog_record writes one 144-byte record (version 1: checksum 0). */
uint32_t orc_fnv1a(const uint8_t* p, size_t n);
void orc_tile_to_bytes(const orc_tile* t, uint8_t* out);
uint32_t orc_record_checksum(uint64_t seq, uint32_t slot, const uint8_t* tile_bytes);
void orc_eventlog_record(uint64_t seq, uint32_t slot, const orc_tile* t, uint32_t version,
                         uint8_t* out);

/* ccos.rs:257-300 — observe_scores: H2O importance from (slot, score) pairs.
 * live[slot] != 0 for a HOT/WARM slot; slots >= n_slots or not live are
 * skipped; no update when no pair is live, a live score is non-finite, the
 * temperature is non-finite or <= 0, or the f32 sum is not finite and > 0. */
void orc_observe_scores(const uint32_t* slots, const float* scores, size_t n, const uint8_t* live,
                        size_t n_slots, float temperature, float* importance);

/* Batched helpers for tests (row-major inputs, one tile per key). */
int orc_encode_batch(const float* keys, size_t n, int codec, int residual_mode, const float* z,
                     const float* rht_diag, uint32_t pos0, uint16_t head_id, orc_tile* out);
void orc_score_batch(const orc_tile* tiles, size_t n, const float* q_coarse,
                     const uint64_t* q_sign, float* scores, uint32_t* hamming);

/* slha-c/src/lib.rs:244-286 — tile validation; returns 0 / -5 / -6. */
int orc_validate_tile(const orc_tile* t);

/* ccos.rs:369-397 — HOT->WARM and correction-plane drop byte effects. */
void orc_page_out(orc_tile* t);
int orc_drop_correction(orc_tile* t);

/* Top-k of one score row: score descending, ties to the lower index. */
void orc_topk(const float* scores, size_t n, size_t k, uint32_t* idx_out, float* val_out);

#ifdef __cplusplus
}
#endif
#endif
