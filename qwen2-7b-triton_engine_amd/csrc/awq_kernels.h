// Internal launcher interface between the C ABI (awq_api.hip) and the kernel
// translation units.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/awq_w4a16.h"
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
    const half_t* bias = nullptr;      // [N] added to every row (epilogue), or null
    const half_t* residual = nullptr;  // [M, N] added after the bias (epilogue), or null; may alias out
};

struct SkinnyConfig {
    int m_blocks;            // 16-row MFMA blocks of x: 1, 2 or 4
    int rows_per_wave;       // K rows per wave: 32, 64 or a multiple of 128
    int kw_count;            // waves per workgroup along K (partials added in LDS): 1, 2 or 4
    int split_k;             // workgroups along K: ceil(K / (rows_per_wave * kw_count))
    int variant;             // main loop: 1 chunked software pipeline, 2 plain loop
    bool factored;           // scale applied to group sums (true) or to each weight (false)
};

struct GemvConfig {
    int variant;             // 2: K-streaming, one group per chunk; 5: column quads with MFMA
                             // column sums, fixed-point split-K finish
    int rows_per_wave;       // variant 2: K rows per wave, 16 or 32
    int kw_count;            // waves per workgroup along K: 1 .. 8 (variant 2: 128 / rows_per_wave)
    int split_k;             // workgroups along K
    int chunks_per_split;    // variant 2: 128-row groups per workgroup
    int depth;               // variant 2: chunk buffers in flight (2, 3 or 4; 4 only for 16 rows per wave)
    int cw;                  // variant 5: packed columns per lane, 4 (512-column strips) or 2 (256)
};

// Tile variants 6 .. 9, 13, 14, 15: weights dequantised into MFMA registers,
// every load a direct global->LDS load into a ring (x rows per tile, stages).
// Variants 13, 14: the hybrid of variants 6 (128 rows) and 8 (64 rows) --
// whole tiles on every CU, the leftover tiles split along K.  Variant 15:
// variant 7 with eight waves on 512-column tiles, one workgroup per CU.
// Numbers 10 - 12 (retired k-half pair tiles) name no kernel.
constexpr int tile5_rows(int variant) { return (variant == 8 || variant == 14) ? 64 : variant == 9 ? 32 : 128; }
constexpr int tile5_cols(int variant) { return variant == 15 ? 512 : 256; }
constexpr int tile5_threads(int variant) { return variant == 15 ? 512 : 256; }
constexpr bool tile_hybrid(int variant) { return variant == 13 || variant == 14; }
// Whether a tile variant number names a kernel.
constexpr bool tile_variant_served(int variant) {
    return (variant >= 6 && variant <= 9) || variant == 13 || variant == 14 || variant == 15;
}

struct TileConfig {
    int variant;             // 6 .. 9, 13, 14, 15: register dequant, N tile 256 (15: 512)
    int tile_m, tile_n;
    int split_k;             // workgroups along K per tile (hybrid: per leftover tile)
    int k_per_split;         // K rows per split (a multiple of the 128-row group)
    int64_t grid;            // workgroups (the hybrid's: whole tiles + leftover tiles x split_k)
};

// out[M, N] = x[M, K] @ w[N, K]^T, fp16 weights (the output projection), one
// MFMA per 16 weight rows x 32 k; M <= 8, K % 8 == 0, K <= fp16_gemv_max_k()
// (x staged in LDS: at most 8 x 4104 x 2 bytes); grids sized for `cus`
// compute units.
hipError_t launch_fp16_gemv(const half_t* x, const half_t* w, half_t* out, int M, int N, int K, int cus,
                            hipStream_t stream);
int fp16_gemv_max_k();

// out[m, i] = fp16(silu(gate_up[m, i]) * gate_up[m, I + i]); I % 8 == 0.
hipError_t launch_silu_mul(const half_t* gate_up, half_t* out, int M, int I, hipStream_t stream);

hipError_t launch_dequant(const uint32_t* qweight, const uint32_t* qzeros, const half_t* scales,
                          half_t* w, int N, int K, hipStream_t stream);

// counters: skinny_counter_bytes() of zero-filled uint32 arrival counters
// (left zero on return); a.partials: split_k * M * N floats (split_k > 1),
// at kPartialsOffset in the workspace.
hipError_t launch_skinny(const GemmArgs& a, const SkinnyConfig& cfg, uint32_t* counters, hipStream_t stream);
size_t skinny_lds_bytes(int M, int m_blocks, int kw_count);
int64_t skinny_pairs(int N);
int64_t skinny_blocks(int N, int K, int rows_per_wave, int kw_count);
size_t skinny_counter_bytes();

// Same workspace contract as launch_skinny (counters, then partials).
// Variants 4 and 5: the workspace after the counter block holds M * N zeroed
// 64-bit fixed-point slots (left zero on return) instead of partials.
hipError_t launch_gemv(const GemmArgs& a, const GemvConfig& cfg, uint32_t* counters, hipStream_t stream);
int64_t gemv_strips(int N);
int64_t gemv_strips_cw(int N, int cw);
size_t gemv_quad_lds_bytes(int M, int K, int split_k, int k_waves, int cw);
int64_t gemv_quad_max_groups(int K, int split_k);
bool gemv_quad_fits(int M, int K, int split_k, int k_waves, int cw);

// Stream path (M <= 16, N % 32 == 0, split_k <= K / 128).  layout:
// kStreamRowLayout (M <= 8; 16-row chunks, k_waves waves) or
// kStreamHalfLayout (32-row chunks, k_waves wave pairs).  depth: chunk
// buffers per wave: row layout 2 (k_waves 1, 2, 4 or 8); half layout 2
// (k_waves <= 4), 4 or 6 (k_waves <= 2).  finish 0: the workspace after the
// counter block holds M * N zeroed 64-bit fixed-point slots; 1: fp32
// partials [split_k, M, N] and one arrival counter per strip; 2: fp32
// partials added by a second kernel launch.  The counter block and the slots
// are left zero on return.
constexpr int kStreamHalfLayout = 32;  // rows per chunk
constexpr int kStreamRowLayout = 16;
// awq_splitk_reduce_kernel over a.partials [split_k][M][N] fp32 -> a.out.
hipError_t splitk_reduce_launch(const GemmArgs& a, int split_k, hipStream_t stream);
hipError_t launch_stream(const GemmArgs& a, int split_k, int k_waves, int depth, int layout, int finish,
                         uint32_t* counters, hipStream_t stream);
size_t stream_lds_bytes(int M, int K, int split_k, int k_waves, int layout);
bool stream_fits(int M, int K, int split_k, int k_waves, int layout);
int64_t stream_threads(int layout, int k_waves);

// split_k > 1 uses the same workspace contract as launch_skinny (counters:
// one per tile).  Variants 7, 8, 9 keep fragment-native partials
// (tile_partials_bytes of them at kPartialsOffset: one 16 KB unit per split,
// 16-row block and 256-column tile) and add them in a second launch of
// awq_tile_reduce_kernel on the same stream.
hipError_t launch_tile(const GemmArgs& a, const TileConfig& cfg, uint32_t* counters, hipStream_t stream);
int64_t tile_tiles(int M, int N, int variant);
uint64_t tile_partials_bytes(int64_t split_k, int64_t M, int64_t N);
// Threads that share one output piece in the reduce launches (enough that
// each adds at most eight splits; eight from 12 splits up).
int stream_reduce_parts(int split_k);

// Output columns per skinny wave.
constexpr int kSkinnyCols = 128;
// Arrival-counter block at the start of a split-K workspace: one uint32 per
// pair of 128-column tiles, so N up to kCounterBytes / 4 * 256 columns.
constexpr size_t kCounterBytes = 16384;
constexpr int64_t kMaxN = (int64_t)(kCounterBytes / 4) * 2 * kSkinnyCols;
// Workspace of a split-K plan: [arrival counters: kCounterBytes]
// [64-bit fixed-point slots: up to kSlotBytes] [fp32 partials].  Counters
// and slots are zero between calls (every call leaves them zero); the
// partials region keeps whatever the last call wrote -- each call writes
// every partial it reads, so it is never cleared.  Fixed-point plans need
// M * N * 8 <= kSlotBytes.
constexpr size_t kSlotBytes = AWQ_W4A16_SLOT_BYTES;
constexpr size_t kPartialsOffset = kCounterBytes + kSlotBytes;

}  // namespace awq
