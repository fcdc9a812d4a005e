/*
 * slha.h — C ABI of the SLHA v2 tile library, MI355X (gfx950) build.
 *
 * Drop-in for the reference ABI slha-c/include/slha.h (ABI version 1): the
 * same 20 exported symbols, status codes, codec ids, tile flags and the same
 * 128-byte tile layout, so existing C callers (the llama.cpp shim,
 * integration/llama.cpp/shim/slha_llama.cpp) relink against libslha.so
 * without source changes. Compute behind these entry points runs on the GPU
 * through the hand-written HIP kernels of this library; host-pointer entry
 * points stage their buffers through device memory.
 *
 * Additive entry points (device pointers, batches, GQA, paged top-k) live in
 * slha_gpu.h.
 */
#ifndef SLHA_H
#define SLHA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* slha.h:11 — ABI revision. */
#define SLHA_ABI_VERSION 1u

/* slha.h:13-17 — tile geometry. */
#define SLHA_D_C 128u
#define SLHA_D_S 256u
#define SLHA_LATENT_BYTES 64u
#define SLHA_RESIDUAL_WORDS 4u
#define SLHA_N_GROUPS 8u

/* slha.h:20-29 — status codes (values are part of the ABI). */
#define SLHA_OK 0
#define SLHA_ERR_NULL (-1)
#define SLHA_ERR_PANIC (-2)
#define SLHA_ERR_DIMENSION (-3)
#define SLHA_ERR_CODEC (-4)
#define SLHA_ERR_NONFINITE (-5)
#define SLHA_ERR_INVALID_TILE (-6)
#define SLHA_ERR_INVALID_HANDLE (-7)
#define SLHA_ERR_IO (-8)
#define SLHA_ERR_UTF8 (-9)
/* Added by this build, after the reference's codes: a HIP runtime failure. */
#define SLHA_ERR_DEVICE (-10)

/* slha.h:32-37 — codec ids accepted by slha_encode_key. */
#define SLHA_CODEC_INT4_SINGLE 0
#define SLHA_CODEC_INT4_GROUPED 1
#define SLHA_CODEC_NF4 2
#define SLHA_CODEC_MIXED 3
#define SLHA_CODEC_TQ3 4
#define SLHA_CODEC_MIX3 5

/* slha.h:40-46 — tile flags (constants.rs:22-48). */
#define SLHA_FLAG_HOT 0u
#define SLHA_FLAG_WARM (1u << 0)
#define SLHA_FLAG_NF4 (1u << 1)
#define SLHA_FLAG_MIXED (1u << 2)
#define SLHA_FLAG_TQ3 (1u << 3)
#define SLHA_FLAG_TQ3_NOCORR (1u << 4)
#define SLHA_FLAG_MIX3 (1u << 5)

/*
 * slha.h:48-57 — tile alignment. 64 bytes by default. Define
 * SLHA_CACHE_LINE_128=1 when linking against a build of this library made
 * with the same definition (SLHA_CACHE_LINE_128=1 in the environment of
 * slhav2_amd/build.py), whose slha_tile_align() returns 128. The byte layout
 * and the 128-byte size are the same either way; only the alignment the
 * compiler assumes for a tile changes.
 */
#if defined(SLHA_CACHE_LINE_128) && SLHA_CACHE_LINE_128
#define SLHA_TILE_ALIGN 128u
#else
#define SLHA_TILE_ALIGN 64u
#endif

/*
 * slha.h:87-98 — the 128-byte tile (tile.rs:52-77). Byte map: latent 0..64,
 * residual 64..96 (4 little-endian u64), scale 96, lambda 100, sigma 104,
 * token_id 108, position 112, head_id 116, flags 118, group_scales 120..128.
 */
typedef struct __attribute__((aligned(SLHA_TILE_ALIGN))) {
    uint8_t latent_kv[SLHA_LATENT_BYTES];
    uint64_t residual_bitmap[SLHA_RESIDUAL_WORDS];
    float scale;
    float dynamic_lambda;
    float residual_sigma;
    uint32_t token_id;
    uint32_t position;
    uint16_t head_id;
    uint16_t flags;
    uint8_t group_scales[SLHA_N_GROUPS];
} SciRustSlhaTile;

#if defined(__cplusplus)
static_assert(sizeof(SciRustSlhaTile) == 128u, "tile is 128 bytes");
static_assert(offsetof(SciRustSlhaTile, residual_bitmap) == 64u, "residual offset");
static_assert(offsetof(SciRustSlhaTile, scale) == 96u, "scale offset");
static_assert(offsetof(SciRustSlhaTile, dynamic_lambda) == 100u, "lambda offset");
static_assert(offsetof(SciRustSlhaTile, residual_sigma) == 104u, "sigma offset");
static_assert(offsetof(SciRustSlhaTile, token_id) == 108u, "token offset");
static_assert(offsetof(SciRustSlhaTile, position) == 112u, "position offset");
static_assert(offsetof(SciRustSlhaTile, head_id) == 116u, "head offset");
static_assert(offsetof(SciRustSlhaTile, flags) == 118u, "flags offset");
static_assert(offsetof(SciRustSlhaTile, group_scales) == 120u, "group_scales offset");
static_assert(alignof(SciRustSlhaTile) == SLHA_TILE_ALIGN, "tile alignment");
#elif defined(__STDC_VERSION__) && __STDC_VERSION__ >= 201112L
_Static_assert(sizeof(SciRustSlhaTile) == 128u, "tile is 128 bytes");
_Static_assert(offsetof(SciRustSlhaTile, flags) == 118u, "flags offset");
_Static_assert(offsetof(SciRustSlhaTile, group_scales) == 120u, "group_scales offset");
_Static_assert(_Alignof(SciRustSlhaTile) == SLHA_TILE_ALIGN, "tile alignment");
#endif

typedef struct SlhaContext SlhaContext;
typedef struct SlhaModel SlhaModel;

/* slha.h:123-125 — ABI and layout introspection. */
uint32_t slha_abi_version(void);
size_t slha_tile_size(void);
size_t slha_tile_align(void);

/* slha.h:133-134 — thread-local last error (<= 511 bytes, library-owned). */
const char* slha_last_error_message(void);
void slha_clear_error(void);

/* slha.h:140,147 — process-wide context. Shutdown is a no-op, as in the
 * reference (lib.rs:331-360); device buffers the library caches live until
 * the process ends. */
SlhaContext* slha_init(void);
int32_t slha_shutdown(SlhaContext* context);

/* slha.h:153 — score one tile (eq. 2.3); score_out untouched on failure. */
int32_t slha_process_tile(const SciRustSlhaTile* tile, const float* q_coarse,
                          const uint64_t* q_sign, float* score_out);

/* slha.h:167 — q_coarse[128] and q_sign[4] from a d-dim query. */
int32_t slha_prepare_query(const SlhaModel* model, const float* q, size_t d, float* q_coarse,
                           uint64_t* q_sign);

/* slha.h:182 — slha_process_tile with a model-handle check. */
int32_t slha_score_tile(const SlhaModel* model, const SciRustSlhaTile* tile,
                        const float* q_coarse, const uint64_t* q_sign, float* score_out);

/* slha.h:197 — score n_tiles (<= 2^20) tiles against one prepared query.
 * Every tile is validated before any score is written. */
int32_t slha_score_tiles(const SlhaModel* model, const SciRustSlhaTile* tiles, size_t n_tiles,
                         const float* q_coarse, const uint64_t* q_sign, float* scores_out);

/* slha.h:210,213 — self-audit JSON; free with slha_free_string. */
char* slha_audit(void);
void slha_free_string(char* string);

/* slha.h:219,225 — projection models. slha_weights_load reads a .slhw v1/v2
 * learned projection (d > 128; scirust/src/weights.rs:8-31, 159-311) with the
 * reference's checks; its GPU kernels hold next_pow2(d) (with RHT, else d)
 * <= 16384 dimensions, and larger models are rejected with a message. */
SlhaModel* slha_weights_load(const char* path);
size_t slha_model_dim(const SlhaModel* model);

/* slha.h:233 — encode one d-dim key into a tile. */
int32_t slha_encode_key(const SlhaModel* model, const float* key, size_t d, uint32_t position,
                        int32_t codec, SciRustSlhaTile* out_tile);

/* slha.h:248,262 — decode a tile back to d floats (latent / latent + sketch). */
int32_t slha_decode_latent(const SlhaModel* model, const SciRustSlhaTile* tile, float* out,
                           size_t d);
int32_t slha_decode_key(const SlhaModel* model, const SciRustSlhaTile* tile, float* out,
                        size_t d);

/* slha.h:272,278 — release a model. */
int32_t slha_weights_release(SlhaModel* model);
void slha_weights_free(SlhaModel* model);

#ifdef __cplusplus
}
#endif

#endif /* SLHA_H */
