// Internal launcher interface between the C ABI (awq_api.hip) and the kernel
// translation units.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "awq_device.h"

namespace awq {

struct GemmArgs {
    const half_t* x;         // [M, K]
    const uint32_t* qweight; // [K, N/8]
    const uint32_t* qzeros;  // [K/128, N/8]
    const half_t* scales;    // [K/128, N]
    half_t* out;             // [M, N]
    float* partials;         // [split_k, M, N] when split_k > 1
    int M, N, K;
};

struct SkinnyConfig {
    int m_blocks;            // 16-row MFMA blocks of x: 1, 2 or 4
    int rows_per_wave;       // K rows per wave: 32, 64 or a multiple of 128
    int kw_count;            // waves per workgroup along K (partials added in LDS): 1, 2 or 4
    int split_k;             // workgroups along K: ceil(K / (rows_per_wave * kw_count))
};

struct TileConfig {
    int variant;             // tile kernel variant
    int tile_m, tile_n;
};

hipError_t launch_dequant(const uint32_t* qweight, const uint32_t* qzeros, const half_t* scales,
                          half_t* w, int N, int K, hipStream_t stream);

hipError_t launch_skinny(const GemmArgs& a, const SkinnyConfig& cfg, hipStream_t stream);
size_t skinny_lds_bytes(int M, int m_blocks, int kw_count);
int64_t skinny_blocks(int N, int K, int rows_per_wave, int kw_count);

hipError_t launch_splitk_reduce(const float* partials, half_t* out, int64_t mn, int split_k,
                                hipStream_t stream);

hipError_t launch_tile(const GemmArgs& a, const TileConfig& cfg, hipStream_t stream);

// Output columns per skinny wave.
constexpr int kSkinnyCols = 128;

}  // namespace awq
