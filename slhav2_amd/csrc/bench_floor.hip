// bench_floor.hip — the measured floor of the C2 score launch (bench.py).
//
// stream_floor_kernel reads every tile once and writes one f32 per (query,
// tile) pair exactly as score_rows_int4_kernel / score_rows_fast_kernel do:
// the same grid (256-thread workgroups over 256 consecutive tokens of one
// row), the same LDS-DMA tile fetch, read-back and non-temporal score
// stores, and no scoring arithmetic. Its time per launch is the cost of
// moving the launch's bytes with this grid, the bar the score kernel is held
// against. Not part of the product library (libslha.so).
#include "slha_tile_io.h"

namespace slha {

__global__ __launch_bounds__(256) void stream_floor_kernel(const uint4* __restrict__ tiles,
                                                           uint32_t n_tok, uint32_t group,
                                                           float* __restrict__ scores) {
    __shared__ uint4 tile_lds[4][512];
    const uint32_t row = blockIdx.y;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t wave0 = blockIdx.x * blockDim.x + 64u * wave;
    const uint32_t n_valid = wave0 < n_tok ? n_tok - wave0 : 0u;
    fetch_tiles_lds(tiles + ((size_t)row * n_tok + wave0) * 8, n_valid, tile_lds[wave]);
    uint32_t w[32];
    fetch_tiles_readback(tile_lds[wave], w);
    uint32_t x = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) x ^= w[i];
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    float* out = scores + (size_t)row * group * n_tok;
    if (t < n_tok)
        for (uint32_t j = 0; j < group; ++j) store_out(out + (size_t)j * n_tok + t, __uint_as_float(x + j));
}

}  // namespace slha

extern "C" int32_t slha_bench_stream_floor(const void* tiles, uint32_t n_rows, uint32_t n_tok,
                                           uint32_t group, float* scores, void* stream) {
    if (n_rows == 0 || n_tok == 0 || group == 0) return 0;
    slha::stream_floor_kernel<<<dim3((n_tok + 255) / 256, n_rows), 256, 0,
                                static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint4*>(tiles), n_tok, group, scores);
    return hipGetLastError() == hipSuccess ? 0 : -10;
}
