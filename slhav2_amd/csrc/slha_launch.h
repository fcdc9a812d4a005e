// slha_launch.h — host-side launchers of the gfx950 kernels (internal; the
// public surface is include/slha.h and include/slha_gpu.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace slha {

// Codec ids (slha.h:32-37).
constexpr int kCodecInt4Single = 0, kCodecInt4Grouped = 1, kCodecNF4 = 2, kCodecMixed = 3,
              kCodecTQ3 = 4, kCodecMix3 = 5;
constexpr int kDtypeF32 = 0, kDtypeBF16 = 1;
constexpr int kResidualZ = 0, kResidualR = 1;
// Largest query group one scoring launch serves (LDS holds group*8 sums).
constexpr uint32_t kMaxGroup = 256;
// Largest k of the paged top-k.
constexpr uint32_t kMaxTopK = 256;
// The paged top-k selects per 16384-score segment, then merges at most
// kTopkMaxCandidates segment winners per row: ceil(max_len/16384) * k <= 8192.
constexpr uint32_t kTopkSeg = 16384;
constexpr uint32_t kTopkMaxCandidates = 8192;

// `workspace`: device memory of score_rows_workspace_bytes(), which no
// scoring path needs at present (0 bytes; may be null).
// `codec_hint`: the codec id the tiles were encoded with, or -1 if unknown;
// it selects kernels only (for group <= 4: kCodecInt4Single the integer
// INT4 path, kCodecNF4 the f16 NF4 path); every kernel meets the fast-mode
// tolerance, and tiles of another codec are still scored by their codec.
hipError_t launch_score_rows(const void* tiles, uint32_t n_rows, uint32_t n_tok, uint32_t group,
                             const float* qc, const uint64_t* qs, bool exact, float* scores,
                             uint32_t* ham, void* workspace, int codec_hint, hipStream_t s);
size_t score_rows_workspace_bytes(uint32_t n_rows, uint32_t group, bool exact, bool ham);
hipError_t launch_score_paged_topk(const void* arena, uint32_t page_shift,
                                  const uint32_t* page_table, uint32_t max_pages,
                                  const uint32_t* seq_len, const uint64_t* score_base,
                                  uint32_t n_seq, uint32_t max_len, uint32_t n_kv, uint32_t group,
                                  const float* qc, const uint64_t* qs, float* scores, uint32_t k,
                                  uint32_t* topk_idx, float* topk_val, void* workspace,
                                  hipStream_t s);
// Device bytes of the `workspace` launch_score_paged_topk needs (top-k candidates).
size_t paged_topk_workspace_bytes(uint32_t n_seq, uint32_t max_len, uint32_t n_kv,
                                  uint32_t group, uint32_t k);
// The same launch with the candidate lists in a file-scope device array of
// kNoAllocScratchBytes (16 MiB: C5, 2048 query rows of up to 131 072 tokens at
// k = 64, takes 8 MiB); nothing is allocated. hipErrorInvalidValue when
// paged_topk_workspace_bytes() exceeds it.
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
hipError_t launch_score_paged_topk_noalloc(const void* arena, uint32_t page_shift,
                                          const uint32_t* page_table, uint32_t max_pages,
                                          const uint32_t* seq_len, const uint64_t* score_base,
                                          uint32_t n_seq, uint32_t max_len, uint32_t n_kv,
                                          uint32_t group, const float* qc, const uint64_t* qs,
                                          float* scores, uint32_t k, uint32_t* topk_idx,
                                          float* topk_val, hipStream_t s);
// Mode R computes the sign sketch on MFMA when `zpack` (build_projection_pack)
// is given, else sequentially per lane; both give the reference's bits.
hipError_t launch_encode(const void* keys, int dtype, uint64_t n_keys, uint32_t n_tok,
                         uint32_t n_kv, uint32_t pos0, int codec, int residual_mode, int warm,
                         const float* z, const void* zpack, float cert_scale, const float* diag,
                         float lambda_c, float rht_inv, void* tiles, hipStream_t s);
// Bytes of Z's MFMA operand pack: a two-term bf16 split of [256][128].
constexpr size_t kZPackBytes = 256 * 128 * 2 * 2;
// Relative bound on |MFMA projection - sequential f32 projection| per unit
// ||z_s|| ||v|| (derivation at encode_mfma_kernel).
constexpr double kEncCertRel = 1.5e-4;
// Fills `pack` (kZPackBytes, host memory) from Z [256][128] and returns the
// certification scale kEncCertRel * max_s ||z_s|| the encode launch takes.
float build_projection_pack(const float* z, void* pack);
hipError_t launch_prepare_queries(const void* q, int dtype, uint64_t n_q, const float* z,
                                  const float* diag, float rht_inv, float* qc, uint64_t* qs,
                                  hipStream_t s);
// Learned (d > 128) models: P [128][d], Z [256][d_pad], RHT diagonal [d_pad]
// or null, d_pad = next_pow2(d) with RHT, else d. The kernels keep a vector
// and its padded residual in LDS: d_pad <= kLearnedMaxDPad.
struct LearnedProjection {
    const float* p = nullptr;
    const float* z = nullptr;
    const float* diag = nullptr;
    const float* p4 = nullptr;  // P interleaved by 4 columns, [ceil(d/4)][128][4]
    const float* z4 = nullptr;  // Z interleaved by 4 columns, [ceil(d_pad/4)][256][4]
    uint32_t d = 0, d_pad = 0;
    float rht_inv = 1.0f;
};
constexpr uint32_t kLearnedMaxDPad = 16384;
// keys [n_keys][d] (f32 or bf16) -> tiles, bit-exact with encode_with
// (learned.rs:353-408); key i: token_id = position = pos0 + i % n_tok,
// head_id = (i / n_tok) % n_kv.
hipError_t launch_learned_encode(const void* keys, int dtype, uint64_t n_keys, uint32_t n_tok,
                                 uint32_t n_kv, uint32_t pos0, int codec, int warm,
                                 const LearnedProjection& lp, float lambda_c, void* tiles,
                                 hipStream_t s);
// q [n_q][d] -> q_coarse [n_q][128], q_sign [n_q][4].
hipError_t launch_learned_prepare(const void* q, int dtype, uint64_t n_q, const LearnedProjection& lp,
                                  float* qc, uint64_t* qs, hipStream_t s);
// tiles [n] -> out [n][d] (reconstruct; with_residual adds the sign-sketch
// estimate when the model has no RHT).
hipError_t launch_learned_decode(const void* tiles, uint64_t n, const LearnedProjection& lp,
                                 int with_residual, float sqrt_half_pi, float* out, hipStream_t s);
// Decode attention over compressed keys: scores (fast mode), softmax of
// scores * scale, out[qh][d_v] = sum_t w_t V[row][t][:]. V is [n_rows][n_tok][d_v]
// (f32 or bf16), group <= 16, d_v is 32, 64, 128 or 256. `workspace` holds
// decode_attention_workspace_bytes().
hipError_t launch_decode_attention(const void* tiles, const void* vals, int v_dtype,
                                   uint32_t n_rows, uint32_t n_tok, uint32_t group, uint32_t d_v,
                                   const float* qc, const uint64_t* qs, float scale, float* out,
                                   void* workspace, hipStream_t s);
size_t decode_attention_workspace_bytes(uint32_t n_rows, uint32_t n_tok, uint32_t group,
                                        uint32_t d_v);
hipError_t launch_decode(const void* tiles, uint64_t n, const float* z_or_null, float sqrt_half_pi,
                         float* out, hipStream_t s);
hipError_t launch_validate(const void* tiles, uint64_t n, uint64_t* status, hipStream_t s);
// op 0 page_out, 1 drop_correction, 2 evict (state only) over slots[0, n), or
// over the one slot `slot0` when slots is NULL (n = 1); page_out and evict
// write the new state into `state` when it is non-NULL.
hipError_t launch_ccos_apply(void* tiles, uint8_t* state, const uint32_t* slots, uint32_t slot0, uint64_t n,
                             int op, hipStream_t s);
// EventLog records (144 B each, eventlog.rs:9-36); n < 2^31 * 256.
hipError_t launch_eventlog_pack(const void* arena, const uint32_t* slots, const uint64_t* seqs,
                                uint64_t n, uint32_t version, void* records, hipStream_t s);
hipError_t launch_eventlog_unpack(const void* records, uint64_t n, uint32_t version,
                                  const uint32_t* dst, void* arena, uint32_t* status, hipStream_t s);
// CCOS: tile i -> arena slot dst[i] (importance[dst[i]] = 0 and state[dst[i]]
// from the tile's FLAG_WARM, each when non-NULL);
// observe_scores over scores[0, n) with state (0 HOT, 1 WARM, 2 COLD) and a
// workspace of observe_workspace_floats() floats.
hipError_t launch_tile_scatter(const void* src, const uint32_t* dst, uint64_t n, void* arena,
                               float* importance, uint8_t* state, hipStream_t s);
size_t observe_workspace_floats();
hipError_t launch_observe_scores(const float* scores, const uint8_t* state, uint64_t n, float temperature,
                                 float* importance, float* workspace, hipStream_t s);
hipError_t launch_fill_u64(uint64_t* p, uint64_t n, uint64_t value, hipStream_t s);
hipError_t launch_fill_u32(uint32_t* p, uint64_t n, uint32_t value, hipStream_t s);

}  // namespace slha
