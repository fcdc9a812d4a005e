/*
 * slha_gpu.h — additive device-pointer API of the MI355X SLHA v2 library.
 *
 * The reference's GPU backend (slhav2-vram) scores one host-resident query
 * against tiles it uploads itself (GpuScoringPipeline::score_into,
 * slhav2-vram/src/pipeline.rs:177-230; CudaEngine::score_tiles_on_stream,
 * slhav2-vram/src/backends/cuda.rs:584-667). This API replaces that pipeline
 * for callers that keep tiles resident in HBM: every buffer argument named
 * *_dev is a device pointer, work is enqueued on `stream` (a hipStream_t;
 * NULL = the default stream) and the call returns without synchronising.
 * Status codes are those of slha.h plus SLHA_ERR_DEVICE for HIP failures;
 * the HIP error text goes to the same thread-local slha_last_error_message.
 */
#ifndef SLHA_GPU_H
#define SLHA_GPU_H

#include "slha.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Residual source of a head_dim-128 model. */
#define SLHA_RESIDUAL_Z 0 /* e = 0: residual bits 0, lambda = sigma = 0 */
#define SLHA_RESIDUAL_R 1 /* e = key - dequant(tile): the quantisation residual */

/* Element type of key / query arrays. */
#define SLHA_DTYPE_F32 0
#define SLHA_DTYPE_BF16 1

/* Score arithmetic. */
#define SLHA_SCORE_FAST 0  /* reassociated f32 (tolerance 1e-3*(1+|s|)) */
#define SLHA_SCORE_EXACT 1 /* tile.rs:267-281 order: bit-identical to the scalar path */

/*
 * Head_dim-128 projection model. The reference builds a model only from a
 * .slhw file with d > 128 (scirust/src/learned.rs:66, weights.rs:195); its
 * head_dim-128 benchmark path is the identity latent plus the sign-LSH
 * projection of scenario.rs:54-114. This constructor builds that model:
 * Z = 256x128 N(0,1) from SplitMix64(seed) (scenario.rs:59-64), optional RHT
 * diagonal from SplitMix64(seed ^ 0xA2A2A2A2A2A2A2A2) (learned.rs:158-165).
 * The handle works with every slha.h entry point taking a model (d = 128).
 */
SlhaModel* slha_model_new_raw128(uint64_t seed, int32_t rht, int32_t residual_mode);

/* Copy the model's Z (256 x d_pad floats, row-major) and RHT diagonal (d_pad
 * floats, may be NULL; all +1 when the model has no RHT) to host memory.
 * d_pad = slha_model_pad_dim(model): 128 for head_dim-128 models; for a
 * learned model next_pow2(d) with RHT, else d (learned.rs:233-245). */
int32_t slha_model_projection(const SlhaModel* model, float* z_out, float* rht_diag_out);
size_t slha_model_pad_dim(const SlhaModel* model);

/* Copy the latent projection P (128 x d floats, row-major) to host memory:
 * the .slhw payload of a learned model, the identity for head_dim 128. */
int32_t slha_model_latent_projection(const SlhaModel* model, float* p_out);

/*
 * Encode keys[n_rows][n_tok][d] (f32 or bf16, device; d = slha_model_dim)
 * into tiles_dev[n_rows][n_tok]. Row r gets head_id = r % n_kv_heads, token t
 * gets token_id = position = pos0 + t. warm != 0 sets FLAG_WARM. Bit-identical
 * to the oracle's encode: mode R / mode Z for head_dim-128 models,
 * LearnedModel::encode_with (learned.rs:353-408) for learned models (codes,
 * residual bits, sigma, lambda). Replaces slha_encode_key
 * (slha-c/src/lib.rs:708-752) for batches.
 */
int32_t slha_gpu_encode(const SlhaModel* model, const void* keys_dev, int32_t key_dtype,
                        size_t n_rows, size_t n_tok, size_t n_kv_heads, uint32_t pos0,
                        int32_t codec, int32_t warm, SciRustSlhaTile* tiles_dev, void* stream);

/*
 * Prepare n_q queries q_dev[n_q][d]: q_coarse_dev[n_q][128] = P q (the query
 * itself for head_dim-128 models; LearnedModel::query_coarse,
 * learned.rs:267-273, for learned ones) and q_sign_dev[n_q][4] = sign bits
 * of Z*RHT(q). Replaces slha_prepare_query (slha-c/src/lib.rs:420-463) for
 * batches.
 */
int32_t slha_gpu_prepare_queries(const SlhaModel* model, const void* q_dev, int32_t q_dtype,
                                 size_t n_q, float* q_coarse_dev, uint64_t* q_sign_dev,
                                 void* stream);

/*
 * GQA scoring (eq. 2.3, tile.rs:267-281). tiles_dev[n_rows][n_tok] where a
 * row is one (sequence, KV head); row r serves the `group` query heads
 * q_*_dev[r*group .. r*group+group). Each tile is read once for the whole
 * group. scores_dev[r*group + j][t]; hamming_dev (NULL to skip) receives the
 * per-pair Hamming distance in the same layout. `mode` is SLHA_SCORE_*.
 * Replaces slha_score_tiles (slha-c/src/lib.rs:527-585) and
 * GpuScoringPipeline::score_into (slhav2-vram/src/pipeline.rs:177-230).
 * Tiles are assumed valid (as produced by the encoders); use
 * slha_gpu_validate_tiles to check caller-supplied bytes. The call allocates
 * no device memory: for 16 < group <= 64 in SLHA_SCORE_FAST mode each
 * workgroup stages the row's queries in its own LDS.
 */
int32_t slha_gpu_score(const SciRustSlhaTile* tiles_dev, size_t n_rows, size_t n_tok,
                       const float* q_coarse_dev, const uint64_t* q_sign_dev, size_t group,
                       int32_t mode, float* scores_dev, uint32_t* hamming_dev, void* stream);

/*
 * slha_gpu_score with the codec the caller encoded the tiles with
 * (SLHA_CODEC_*, or -1 if unknown; slha_gpu_score passes -1). The hint picks
 * kernels only: tiles of another codec are still scored by their own codec,
 * only more slowly, and every kernel meets the fast-mode tolerance (results
 * may differ between kernels in the last bits). In SLHA_SCORE_FAST mode
 * with group <= 4: SLHA_CODEC_INT4 scores on the integer matrix cores
 * (queries carried to ~2^-23 relative); SLHA_CODEC_NF4 on f16 matrix cores
 * with each NF4 level carried as an f16 hi + lo pair (~2^-22).
 * No counterpart in the reference, which dispatches per tile on its flags
 * (simd.rs:23-84); an unknown hint is SLHA_ERR_CODEC.
 */
int32_t slha_gpu_score_codec(const SciRustSlhaTile* tiles_dev, size_t n_rows, size_t n_tok,
                             const float* q_coarse_dev, const uint64_t* q_sign_dev, size_t group,
                             int32_t mode, int32_t codec_hint, float* scores_dev,
                             uint32_t* hamming_dev, void* stream);

/*
 * Validate n tiles on the device (slha-c/src/lib.rs:244-286). status_dev[0]
 * receives 0, or the lowest failing tile index + 1 (u64); the failing status
 * (SLHA_ERR_NONFINITE / SLHA_ERR_INVALID_TILE) is status_dev[1].
 */
int32_t slha_gpu_validate_tiles(const SciRustSlhaTile* tiles_dev, size_t n, uint64_t* status_dev,
                                void* stream);

/*
 * Decode tiles to floats: out_dev[n][d] = reconstruct(dequant_latent)
 * (tile.rs:249-255, learned.rs:276-286; the identity for head_dim-128 models);
 * with_residual != 0 adds the sign-sketch residual estimate of
 * LearnedModel::reconstruct_from_tile (learned.rs:288-320) when the model has
 * no RHT.
 */
int32_t slha_gpu_decode(const SlhaModel* model, const SciRustSlhaTile* tiles_dev, size_t n,
                        int32_t with_residual, float* out_dev, void* stream);

/*
 * CCOS paged scoring with top-k (ElasticKvCache::score_all, ccos.rs:346-355,
 * over a paged arena). arena_dev holds pages of page_tiles tiles (a power of
 * two); page_table_dev[(s*n_kv_heads + h)*max_pages + p] is the physical page
 * of logical page p of (sequence s, KV head h). seq_len_dev[s] (u32) is the
 * token count of sequence s and max_len >= every seq_len. Scores of
 * (s, query head qh = h*group + j, token t) go to
 * scores_dev[score_base_dev[s] + qh*len(s) + t] (score_base_dev: u64 [n_seq]).
 * For each (s, qh) the k best tokens (score descending, ties to the lower
 * token index) go to topk_idx_dev / topk_score_dev[(s*n_kv_heads*group + qh)*k + i];
 * entries past len(s) are 0xFFFFFFFF / -inf. WARM tiles score coarse-only
 * (ccos.rs:320-355 via FLAG_WARM). 1 <= k <= 256 with
 * ceil(max_len / 16384) * k <= 8192 (k = 64: rows up to 2 097 152 tokens),
 * or k = 0 to skip top-k. The top-k stage keeps its candidate lists in a
 * device workspace the library allocates per (device, stream) on first use
 * and grows as needed: n_seq * n_kv_heads * group * ceil(max_len / 16384) *
 * k * 8 bytes.
 */
int32_t slha_gpu_score_paged_topk(const SciRustSlhaTile* arena_dev, size_t page_tiles,
                                  const uint32_t* page_table_dev, size_t max_pages,
                                  const uint32_t* seq_len_dev, const uint64_t* score_base_dev,
                                  size_t n_seq, size_t max_len, size_t n_kv_heads, size_t group,
                                  const float* q_coarse_dev, const uint64_t* q_sign_dev,
                                  float* scores_dev, size_t k, uint32_t* topk_idx_dev,
                                  float* topk_score_dev, void* stream);

/*
 * slha_gpu_score_paged_topk without any allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, checks and outputs as slha_gpu_score_paged_topk. The top-k
 * candidate lists (n_seq * n_kv_heads * group * ceil(max_len / 16384) * k * 8
 * bytes) live in a library-owned static device array of
 * SLHA_NOALLOC_SCRATCH_BYTES that each GPU holds until the process ends; a
 * call needing more returns SLHA_ERR_DIMENSION before any device work. Every
 * call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (other streams, other threads) race and must be serialised by the caller.
 */
#define SLHA_NOALLOC_SCRATCH_BYTES (16u << 20)
int32_t slha_gpu_score_paged_topk_noalloc(const SciRustSlhaTile* arena_dev, size_t page_tiles,
                                          const uint32_t* page_table_dev, size_t max_pages,
                                          const uint32_t* seq_len_dev, const uint64_t* score_base_dev,
                                          size_t n_seq, size_t max_len, size_t n_kv_heads, size_t group,
                                          const float* q_coarse_dev, const uint64_t* q_sign_dev,
                                          float* scores_dev, size_t k, uint32_t* topk_idx_dev,
                                          float* topk_score_dev, void* stream);

/*
 * Decode attention over compressed keys (the decode step of
 * scirust/examples/benchmark_decode.rs:29-90): for query head
 * qh = r*group + j of row r,
 *   w = softmax(s * scale) over the row's n_tok tiles, s the eq. 2.3 scores
 *       (SLHA_SCORE_FAST), with softmax_into's contract (metrics.rs:338-409:
 *       a NaN score or a non-finite scale gives zero weights);
 *   out_dev[qh][d] = sum_t w_t v_dev[r][t][d]   (aggregate_v, :29-38).
 * v_dev is [n_rows][n_tok][d_v], f32 or bf16; 1 <= group <= 16; d_v is 32,
 * 64, 128 or 256. The scores and per-segment partial sums live in a device workspace the
 * library allocates per (device, stream) on first use and grows as needed
 * (n_rows*group*(4*n_tok + (d_v+4)*4*ceil(n_tok/512)) bytes).
 */
int32_t slha_gpu_decode_attention(const SciRustSlhaTile* tiles_dev, const void* v_dev,
                                  int32_t v_dtype, size_t n_rows, size_t n_tok, size_t d_v,
                                  const float* q_coarse_dev, const uint64_t* q_sign_dev,
                                  size_t group, float scale, float* out_dev, void* stream);

/*
 * CCOS ladder steps on device-resident tiles (ccos.rs:369-397), applied to
 * the tiles whose index is listed in slots_dev[n]: op 0 = page_out
 * (HOT->WARM: residual := 0, lambda := 0, |FLAG_WARM), op 1 = drop_correction
 * (zero the TQ3/MIX3 correction plane, |FLAG_TQ3_NOCORR; no-op on other
 * codecs or when already dropped).
 */
int32_t slha_gpu_ccos_apply(SciRustSlhaTile* tiles_dev, const uint32_t* slots_dev, size_t n,
                            int32_t op, void* stream);

/* Synchronise the stream and report any pending HIP error. */
int32_t slha_gpu_synchronize(void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SLHA_GPU_H */
