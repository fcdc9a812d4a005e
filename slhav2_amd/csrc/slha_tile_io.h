// slha_tile_io.h — how the gfx950 scoring kernels move tiles and scores:
// a wave's 64 consecutive tiles go HBM -> LDS by direct (LDS DMA) buffer
// loads, are read back one tile per lane, and scores leave with
// non-temporal stores. Shared by the product kernels and the bench's
// read-then-store floor kernel, so that the floor moves bytes exactly as the
// product does.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace slha {

// Scores and Hamming distances are written once and not read again by the
// scoring kernels: non-temporal stores stream them out of L2 as they are
// written instead of leaving 4 B per pair dirty there. At the C2 size
// (4 MiB of scores per launch) this took the launch from ~9.5 to ~8.9 us.
template <typename T>
__device__ __forceinline__ void store_out(T* p, T v) {
    __builtin_nontemporal_store(v, p);
}

// LDS byte address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_byte_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// Coalesced direct-to-LDS fetch of a wave's 64 consecutive tiles (8 KiB)
// into its LDS region. buffer_load_dwordx4 ... lds writes lane l of load j to
// region + 1024 j + 16 l; each lane picks the global chunk that belongs in
// that slot under the swizzle "chunk c of tile u at uint4 slot
// 8u + (c ^ (u & 7))", so every load instruction reads 1 KiB of contiguous
// HBM (8 lanes per 128-B tile, chunks permuted inside the tile) and no VGPRs
// hold the data in flight. The buffer's range ends at the last valid tile:
// slots of tiles at or past n_valid read as zero. The compiler waits for
// these loads (vmcnt) before the region is read back.
// Cache policy of the tile loads: nt (streaming). A launch reads each tile
// once; at C2 this took the launch from ~8.9 to ~8.7 us.
constexpr int kCachePolicyNT = 2;

__device__ __forceinline__ void fetch_tiles_lds(const uint4* wave_base, uint32_t n_valid,
                                                uint4* region) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t in_tile = (lane & 0x38u) + ((lane & 7u) ^ (lane >> 3));
    // readfirstlane: the range is wave-uniform, and a descriptor built from
    // VGPRs would be legalised into a loop over lanes.
    const uint32_t bytes = __builtin_amdgcn_readfirstlane((n_valid < 64u ? n_valid : 64u) * 128u);
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint4*>(wave_base), 0, bytes, 0x00020000);
    // The whole offset in the VGPR operand: the range check of a raw buffer
    // load covers it but not the SGPR offset.
#pragma unroll
    for (int j = 0; j < 8; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rsrc, (__attribute__((address_space(3))) void*)(region + 64 * j), 16,
            1024u * j + in_tile * 16u, 0, 0, kCachePolicyNT);
}

// fetch_tiles_lds with the wave's tiles dealt into four 2 KiB blocks: block
// k (DMA loads 2k, 2k + 1) holds tiles 4c + k, c = 0..15, tile 4c + k at
// local position c (chunk ch at uint4 slot 128 k + 8 c + (ch ^ (c & 7))).
// Each load still reads whole 128-byte tiles (8 of them, 512 bytes apart),
// and tiles at or past n_valid read as zero. A lane that scores local tile c
// of every block ends with four consecutive tokens 4c .. 4c + 3.
__device__ __forceinline__ void fetch_tiles_lds_dealt(const uint4* wave_base, uint32_t n_valid,
                                                      uint4* region) {
    const uint32_t lane = threadIdx.x & 63u;
    // load j = 2k + half: lane l holds chunk (l & 7) ^ (l >> 3) of local tile
    // c = 8 half + (l >> 3), i.e. of tile 4c + k
    const uint32_t in_tile = 512u * (lane >> 3) + 16u * ((lane & 7u) ^ (lane >> 3));
    const uint32_t bytes = __builtin_amdgcn_readfirstlane((n_valid < 64u ? n_valid : 64u) * 128u);
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint4*>(wave_base), 0, bytes, 0x00020000);
#pragma unroll
    for (int j = 0; j < 8; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rsrc, (__attribute__((address_space(3))) void*)(region + 64 * j), 16,
            4096u * (j & 1) + 128u * (j >> 1) + in_tile, 0, 0, kCachePolicyNT);
}

// Lane l reads tile l back from a region filled by fetch_tiles_lds_dealt.
__device__ __forceinline__ void fetch_tiles_readback_dealt(const uint4* region, uint32_t* w) {
    const uint32_t lane = threadIdx.x & 63u, c = lane >> 2;
    const uint4* t = region + 128u * (lane & 3u) + 8u * c;
#pragma unroll
    for (int ch = 0; ch < 8; ++ch) {
        const uint4 x = t[ch ^ (c & 7u)];
        w[4 * ch + 0] = x.x;
        w[4 * ch + 1] = x.y;
        w[4 * ch + 2] = x.z;
        w[4 * ch + 3] = x.w;
    }
}

// Lane l reads tile l back from a region filled by fetch_tiles_lds; the XOR
// swizzle keeps these reads free of bank conflicts. Only lanes of one wave
// touch the region, so no barrier is needed.
__device__ __forceinline__ void fetch_tiles_readback(const uint4* region, uint32_t* w) {
    const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const uint4 x = region[8u * lane + (c ^ (lane & 7u))];
        w[4 * c + 0] = x.x;
        w[4 * c + 1] = x.y;
        w[4 * c + 2] = x.z;
        w[4 * c + 3] = x.w;
    }
}

}  // namespace slha
