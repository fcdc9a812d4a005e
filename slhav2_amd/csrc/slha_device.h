// slha_device.h — register-level view of the 128-byte SLHA v2 tile and the
// per-codec decode used by every gfx950 kernel of this library.
//
// A tile lives in 32 VGPRs (w[0..31], little-endian u32 words):
//   w[0..15]  latent_kv (64 B)       w[16..23] residual_bitmap (4 x u64)
//   w[24] scale  w[25] dynamic_lambda  w[26] residual_sigma
//   w[27] token_id  w[28] position  w[29] head_id | flags << 16
//   w[30..31] group_scales[8]
// (tile.rs:52-77; slha.h byte map.)
//
// The *_exact helpers reproduce tile.rs's dequant arithmetic operation for
// operation (tile.rs:133-246). They are only bit-identical when the
// translation unit is compiled with -ffp-contract=off, which the build does;
// fast kernels opt back into contraction locally.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace slha {

constexpr int kDC = 128;
constexpr int kDS = 256;
constexpr uint32_t kFlagWarm = 0x01, kFlagNF4 = 0x02, kFlagMixed = 0x04, kFlagTQ3 = 0x08,
                   kFlagNoCorr = 0x10, kFlagMix3 = 0x20;
constexpr uint32_t kCodecFlags = kFlagNF4 | kFlagMixed | kFlagTQ3 | kFlagMix3;
constexpr uint32_t kKnownFlags = kFlagWarm | kCodecFlags | kFlagNoCorr;

// constants.rs:138-141
__device__ __forceinline__ float nf4_level(uint32_t nib) {
    // Select tree instead of a table so that a divergent index never leaves
    // registers. Values are the f32 literals of NF4_CODEBOOK.
    const float lo[8] = {-1.0f, -0.7075f, -0.5421f, -0.4165f, -0.3108f, -0.2158f, -0.1272f, -0.0421f};
    const float hi[8] = {0.0421f, 0.1272f, 0.2158f, 0.3108f, 0.4165f, 0.5421f, 0.7075f, 1.0f};
    uint32_t i = nib & 7u;
    float a = (i & 4u) ? ((i & 2u) ? ((i & 1u) ? lo[7] : lo[6]) : ((i & 1u) ? lo[5] : lo[4]))
                       : ((i & 2u) ? ((i & 1u) ? lo[3] : lo[2]) : ((i & 1u) ? lo[1] : lo[0]));
    float b = (i & 4u) ? ((i & 2u) ? ((i & 1u) ? hi[7] : hi[6]) : ((i & 1u) ? hi[5] : hi[4]))
                       : ((i & 2u) ? ((i & 1u) ? hi[3] : hi[2]) : ((i & 1u) ? hi[1] : hi[0]));
    return (nib & 8u) ? b : a;
}

__device__ __forceinline__ uint32_t nib_at(const uint32_t* lw, int n) {
    return (lw[n >> 3] >> (4 * (n & 7))) & 0xFu;
}
__device__ __forceinline__ uint32_t byte_at(const uint32_t* lw, int b) {
    return (lw[b >> 2] >> (8 * (b & 3))) & 0xFFu;
}
// 3 bits starting at absolute latent bit position p (TQ3/MIX3 code fields;
// a field never ends past its plane, so the tile.rs:194-198 window guard
// cannot change the extracted bits).
__device__ __forceinline__ uint32_t bits3_at(const uint32_t* lw, int p) {
    const int wi = p >> 5, sh = p & 31;
    uint32_t v = lw[wi] >> sh;
    if (sh > 29) v |= lw[wi + 1] << (32 - sh);
    return v & 7u;
}
__device__ __forceinline__ uint32_t bit_at(const uint32_t* lw, int p) {
    return (lw[p >> 5] >> (p & 31)) & 1u;
}
__device__ __forceinline__ float gs_at(const uint32_t* gw, int g) {
    return (float)((gw[g >> 2] >> (8 * (g & 3))) & 0xFFu);
}

// tile.rs:133-135 — scale * (gs/255).
__device__ __forceinline__ float group_scale_exact(float scale, float gsf) {
    return scale * (gsf / 255.0f);
}
// tile.rs:169,175,220,245 — (scale * gs) / 255.
__device__ __forceinline__ float section_scale_exact(float scale, float gsf) {
    return scale * gsf / 255.0f;
}

// TQ3 grid level of body dim ld (tile.rs:187-207, :217-246).
__device__ __forceinline__ float tq3_level_exact(const uint32_t* lw, int codes_bit0,
                                                 int corr_bit0, int ld, bool nocorr) {
    float level = (float)bits3_at(lw, codes_bit0 + 3 * ld) - 3.5f;
    if (!nocorr) {
        float sign = bit_at(lw, corr_bit0 + ld) ? 1.0f : -1.0f;
        level += sign * 0.25f;
    }
    return level;
}

// Dequantised latent k[0..127], tile.rs:141-255, operation for operation.
__device__ __forceinline__ void dequant_exact(const uint32_t* lw, const uint32_t* gw,
                                              float scale, uint32_t flags, float* k) {
    const bool nocorr = (flags & kFlagNoCorr) != 0;
    if (flags & kFlagMixed) {
#pragma unroll
        for (int d = 0; d < 8; ++d)
            k[d] = (float)((int)byte_at(lw, d) - 128) * section_scale_exact(scale, gs_at(gw, 0));
#pragma unroll
        for (int ld = 0; ld < 112; ++ld)
            k[8 + ld] = (float)((int)nib_at(lw, 16 + ld) - 8) *
                        section_scale_exact(scale, gs_at(gw, 1 + ld / 16));
#pragma unroll
        for (int d = 120; d < 128; ++d) k[d] = 0.0f;
    } else if (flags & kFlagTQ3) {
#pragma unroll
        for (int d = 0; d < 128; ++d)
            k[d] = tq3_level_exact(lw, 0, 384, d, nocorr) *
                   group_scale_exact(scale, gs_at(gw, d / 16));
    } else if (flags & kFlagMix3) {
#pragma unroll
        for (int d = 0; d < 8; ++d)
            k[d] = (float)((int)byte_at(lw, d) - 128) * section_scale_exact(scale, gs_at(gw, 0));
#pragma unroll
        for (int ld = 0; ld < 112; ++ld)
            k[8 + ld] = tq3_level_exact(lw, 64, 400, ld, nocorr) *
                        section_scale_exact(scale, gs_at(gw, 1 + ld / 16));
#pragma unroll
        for (int d = 120; d < 128; ++d) k[d] = 0.0f;
    } else if (flags & kFlagNF4) {
#pragma unroll
        for (int d = 0; d < 128; ++d)
            k[d] = nf4_level(nib_at(lw, d)) * group_scale_exact(scale, gs_at(gw, d / 16));
    } else {
#pragma unroll
        for (int d = 0; d < 128; ++d)
            k[d] = (float)((int)nib_at(lw, d) - 8) * group_scale_exact(scale, gs_at(gw, d / 16));
    }
}

__device__ __forceinline__ uint32_t hamming_words(const uint32_t* r, const uint32_t* qs) {
    uint32_t h = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) h += __popc(r[i] ^ qs[i]);
    return h;
}

}  // namespace slha
