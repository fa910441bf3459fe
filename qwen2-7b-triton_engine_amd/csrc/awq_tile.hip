// Prefill W4A16 AWQ GEMM (large M) for gfx950: LDS-tiled MFMA kernels
// (awq_tile_kernel, tile variants 6 .. 9, 13, 14, 15): 256 output columns per
// tile (512 for variant 15),
// weights dequantised straight into MFMA operand registers, every operand
// streamed into LDS rings by direct global->LDS loads, the reference's exact
// fp16 weight fp16((q - z) * s) formed next to the load.
#include "awq_kernels.h"

namespace awq {

// ---------------------------------------------------------------------------
// Tile variants 6 .. 9, 13, 14: 256 output columns per tile, four waves of 64
// columns x 32, 64 or 128 x rows (variant 15: eight such waves, 512 columns
// x 128 rows), weights dequantised straight into MFMA A
// registers (never written back to LDS), every global load a direct
// global->LDS load issued two k-steps ahead into a 3-stage ring.  No VGPR
// holds data in flight and the compiler sees no global load inside the main
// loop, so nothing waits on a load before the step that consumes it: the
// kernel waits itself, once per k-step (vmcnt = the loads issued since).
//
// A stage holds one k-step (64 rows):
//   * x: BM rows of 128 B, XOR-swizzled: 16-byte chunk p of row r holds
//     k-chunk p ^ (r & 7), so the MFMA fragment reads of 8 consecutive rows
//     hit 8 distinct chunk positions (all banks once); rows beyond M read as
//     zeros (buffer range check); a wave's dwordx4 load writes 8 rows.
//   * packed weights, 64 rows x 8 packed columns a wave: wave w's 2 KB holds its
//     packed columns 8 w .. + 7 row-major (32 B a row, the two 16-byte halves
//     of row r swapped when bit 3 of r is set), loaded by two dwordx4 loads
//     and read back column-wise with LDS transpose reads.
//   * per wave, the group's 8 zero words and 64 scales of its columns (160 B;
//     loaded with the first k-step of each 128-row group only).
// Each k-step runs in two phases that overlap the dequantisation of the next
// k-half with the MFMAs of the current one (see the main loop).
// FM: 16-row blocks per wave (8: 128 x rows per wave; 4: 64; 2: 32).
// Variant 6 = FM 8: 128 x 256 tiles, two workgroups per CU, last-arriver
// split-K finish; 7, 8, 9 = FM 8, 4, 2: 128, 64 and 32 x 256 tiles (two,
// three, four workgroups per CU) with the reduce-launch finish -- the smaller
// tiles for small M, where the larger ones would leave MFMA rows idle or the
// CUs short of work.  (Variants 10 - 12, tiles with a second wave per SIMD
// taking every other k-half, are retired: slower than these everywhere.)
namespace {
constexpr int T5_BK = 64;
constexpr int T5_BN = 256;
constexpr int T5_ZS_WAVE = 160;               // one wave's 8 zero words + 64 scales
constexpr int T5_GM = 4;
constexpr int T5_STAGES = 3;

template <int FM, int NW = 4>
struct T5Layout {
    static constexpr int S = T5_STAGES;
    static constexpr int BM = 16 * FM;  // x rows per tile (every wave reads all of them)
    static constexpr int BN = 64 * NW;  // columns per tile: 64 a wave
    static constexpr int X_BYTES = BM * T5_BK * 2;
    static constexpr int W_BYTES = 2048 * NW;  // packed weights of one k-step
    static constexpr int ZS_BYTES = NW * T5_ZS_WAVE;
    static constexpr int STAGE = X_BYTES + W_BYTES + ZS_BYTES;
    static constexpr int WAVES = NW;
    // The ring, or the staged fp16 tile (rows BN x 2 + 32 bytes apart) if larger.
    static constexpr int SMEM = S * STAGE > BM * (BN * 2 + 32) ? S * STAGE : BM * (BN * 2 + 32);
    static constexpr int X_LOADS = X_BYTES / 1024 / WAVES;  // dwordx4 loads per wave per stage (FM / 2)
    // Workgroups per CU: by registers (accumulators 4 * FM float4 per lane)
    // and by LDS (S stages).
    static constexpr int PER_CU_REG = NW == 8 ? 1 : (FM >= 8 ? 2 : (FM >= 4 ? 3 : 4));
    static constexpr int PER_CU_LDS = (160 * 1024) / (SMEM + 64);
    static constexpr int PER_CU = PER_CU_REG < PER_CU_LDS ? PER_CU_REG : PER_CU_LDS;
    static constexpr int W_LOADS = 2;  // dwordx4 packed-weight loads per wave per stage (its own 2 KB)
    // Loads a wave issues per stage: an even k-step's (the first of its
    // 128-row group) and an odd one's, which brings no zero words or scales.
    static constexpr int LOADS = X_LOADS + W_LOADS + 2;
    static constexpr int LOADS_NZ = X_LOADS + W_LOADS;
};
template <bool B>
struct Parity {
    static constexpr bool value = B;
};
}  // namespace

// Hybrid tiles: bands per leftover tile whose partials are added by helpers
// -- the largest power of two up to 8 with n_sk x bands whole-tile
// workgroups to help (d of them) and bands of at least 16 rows.
__device__ __forceinline__ int hy_bands(int n_sk, int d, int bm) {
    int h = 1;
    while (h < 8 && n_sk * 2 * h <= d && bm / (2 * h) >= 16) h *= 2;
    return h;
}

// FIN (split_k > 1): 0 -- the last workgroup of a tile to arrive adds the
// partials; 1 -- fragment-native partials (whole-kilobyte stores of the
// accumulator registers), summed by a second launch of
// awq_tile_reduce_kernel over the whole device (for small tiles, whose last
// arrivers would each read split x tile bytes alone).
// HY (hybrid, FIN 0): workgroups 0 .. D-1 each take one whole tile, the last
// L tiles of the order are split split_k ways along K, one piece per
// remaining workgroup (grid = D + L split_k, so L = (grid - tiles) /
// (split_k - 1)).  With D a whole number of workgroups per CU and L split_k at
// most one more per CU, every CU holds its whole tiles plus at most one short
// piece, instead of some CUs holding a whole tile more than the others; the
// pieces finish early, so their last arrivers add the partials while the
// whole tiles still run.  The pieces' partials are compact: [split_k][L][BM
// rows][256 columns] fp32.
//
// NW: waves per workgroup, each owning 64 of the tile's 64 NW columns (4:
// 256-column tiles, two workgroups per CU for 128 rows; 8: 512-column tiles,
// one workgroup per CU, FIN 1 and no hybrid only -- variant 15).  The x rows
// of a k-step are loaded once for all of the workgroup's columns.
template <int FM, int FIN, bool HY = false, int NW = 4>
__global__ __launch_bounds__(64 * NW, (T5Layout<FM, NW>::PER_CU)) void awq_tile_kernel(GemmArgs a, int split_k,
                                                                              int k_per_split,
                                                                              uint32_t* counters) {
    using L = T5Layout<FM, NW>;
    constexpr int BN = L::BN;
    constexpr int BM = L::BM;
    constexpr int S = L::S;
    static_assert((S - 2) * L::LOADS <= 63, "vmcnt holds 6 bits");
    static_assert(FM % 2 == 0 && L::X_LOADS >= 1, "a wave loads whole 8-row blocks of x");
    static_assert(L::PER_CU >= 1 && L::PER_CU * L::SMEM <= 160 * 1024, "LDS per CU");
    static_assert(NW == 4 || (NW == 8 && FIN == 1 && !HY), "eight waves: reduce-launch finish only");
    __shared__ __attribute__((aligned(16))) unsigned char smem[L::SMEM];
    __shared__ int last_flag;
    __shared__ int last_band[8];
    floatx4* fin = reinterpret_cast<floatx4*>(smem);  // split-K finish, after the main loop

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave;
    const int n16 = lane & 15;
    const int kb = lane >> 4;

    // ---- work item: XCD-aware grouped tile order (groups of T5_GM row tiles) ----
    const int m_tiles = (a.M + BM - 1) / BM;
    const int n_tiles = (a.N + BN - 1) / BN;
    // Position of workgroup b among `total` consecutive ones in XCD order:
    // the workgroups one XCD runs (b % 8 == x) get consecutive positions.
    auto xcd_order = [](int b, int total) {
        const int xcd = b & 7, xi = b >> 3, per = (total + 7) >> 3, rem = total & 7;
        return (rem == 0 || xcd < rem) ? xcd * per + xi : rem * per + (xcd - rem) * (per - 1) + xi;
    };
    int tile, split, ks = split_k, sk_tile = 0, n_sk = 0;  // ks: splits of this workgroup's tile
    if constexpr (HY) {
        const int T = m_tiles * n_tiles;
        n_sk = ((int)gridDim.x - T) / (split_k - 1);
        const int D = T - n_sk;
        if ((int)blockIdx.x < D) {
            tile = xcd_order((int)blockIdx.x, D);
            split = 0;
            ks = 1;
        } else {
            const int w = xcd_order((int)blockIdx.x - D, (int)gridDim.x - D);
            sk_tile = w / split_k;
            tile = D + sk_tile;
            split = w - sk_tile * split_k;
        }
    } else if (FIN == 1 && split_k > 1 && a.K >= 8192) {
        // Split-major for long K (grid = tiles x split_k): the workgroups of
        // one XCD hold neighbouring K ranges of every tile, so each x and
        // weight byte is fetched into one XCD's L2 only, where tile-major
        // order fetches a K range of x into every XCD holding one of its
        // tiles.  The reduce launch sums the splits in split order, so the
        // outputs are the same in either order.  Measured 1 - 3 % faster on
        // K = 18944 (down_proj) at M = 96 - 2048, and 2 - 3 % slower on K =
        // 3584, hence the bound.
        const int T = m_tiles * n_tiles;
        const int w = xcd_order((int)blockIdx.x, (int)gridDim.x);
        split = w / T;
        tile = w - split * T;
    } else {
        const int w = xcd_order((int)blockIdx.x, (int)gridDim.x);
        tile = w / split_k;
        split = w - tile * split_k;
    }
    const int in_group = T5_GM * n_tiles;
    // Tile t's first row and column (tiles in groups of T5_GM row tiles).
    auto tile_origin = [&](int t, int& tm0, int& tn0) {
        const int first_m = (t / in_group) * T5_GM;
        const int gm = min(m_tiles - first_m, T5_GM);
        tm0 = (first_m + (t % in_group) % gm) * BM;
        tn0 = ((t % in_group) / gm) * BN;
    };
    int m0, n0;
    tile_origin(tile, m0, n0);
    const int pn = a.N >> 3;
    const int k_begin = ks == 1 ? 0 : split * k_per_split;
    const int k_end = ks == 1 ? a.K : min(a.K, k_begin + k_per_split);
    const int KT = (k_end - k_begin) / T5_BK;  // even: whole groups

    const u32x4 rx = raw_rsrc(a.x, (uint32_t)((size_t)a.M * a.K * 2));
    const u32x4 rw = raw_rsrc(a.qweight, (uint32_t)((size_t)a.K * pn * 4));
    const u32x4 rz = raw_rsrc(a.qzeros, (uint32_t)((size_t)(a.K / kGroup) * pn * 4));
    const u32x4 rs = raw_rsrc(a.scales, (uint32_t)((size_t)(a.K / kGroup) * a.N * 2));
    const uint32_t lds0 = lds_addr(smem);

    // x: load i of wave w writes rows 8 (X_LOADS w + i) .. + 7; lane l brings
    // row 8 b + l / 8, k-chunk (l % 8) ^ (l / 8) to LDS chunk position l % 8.
    // A row at or beyond M has an offset at or beyond the buffer's M x K x 2
    // bytes, so the range check zeroes it; load i's offset is load 0's plus
    // 8 i rows.
    const uint32_t x_voff =
        (uint32_t)(((size_t)(m0 + 8 * L::X_LOADS * wave + (lane >> 3)) * a.K + 8 * ((lane & 7) ^ (lane >> 3))) * 2);
    // Packed weights: wave w loads only its own packed columns 8 w .. 8 w + 7,
    // row-major (32 B a row): dwordx4 load i covers rows 32 i .. + 31, lane
    // l bringing the 16-byte slot (l % 2) ^ sw(r) (packed columns 4 s .. + 3)
    // of row r = 32 i + l / 2, sw(r) = bit 3 of r.  A transpose read below
    // takes 8 bytes at one offset from each of the 64 rows, 32 lanes (rows
    // r, r + 8, r + 32, r + 40 for each r < 8) through the 64 banks at a
    // time; a row's banks repeat every 8 rows, so swapping the slots on bit
    // 3 splits those four rows into two pairs -- a 2-way conflict, the least
    // 16-byte slots allow (bit 2, which the four rows share, left it 4-way).
    // Load 1 uses load 0's offset, its rows 32 further down through the
    // scalar offset.
    const int w_row = lane >> 1;
    const int w_jc = (n0 >> 3) + 8 * wave + 4 * ((lane & 1) ^ ((w_row >> 3) & 1));
    const uint32_t w_voff = w_jc < pn ? (uint32_t)((w_row * pn + w_jc) * 4) : 0x80000000u;
    // Zero words and scales: every wave loads the scales of its 64 columns
    // (lanes 0..31) and the zero words of its 8 packed columns (lanes
    // 32..39, whose LDS slots the load's base, 128 B lower, puts on the
    // 32-byte zero area); the other lanes are masked off and write nothing.
    // One offset register serves both.
    uint32_t zs_voff;
    if (lane < 32) {
        const int s_col = n0 + 64 * wave + 2 * lane;
        zs_voff = s_col < a.N ? (uint32_t)s_col * 2u : 0x80000000u;
    } else {
        const int z_jc = (n0 >> 3) + 8 * wave + (lane & 7);
        zs_voff = z_jc < pn ? (uint32_t)z_jc * 4u : 0x80000000u;
    }

    auto issue = [&](int kt, int stage) {
        const uint32_t base = lds0 + (uint32_t)(stage * L::STAGE);
        const int k0 = k_begin + kt * T5_BK;
        const int g = k0 / kGroup;
        // Zero words and scales with the first k-step of each group only
        // (k-steps are 64 rows, groups 128, and every K range starts on a
        // group).  Partial-wave loads: the lanes left out write no LDS (never
        // all of them, so both loads issue and count in vmcnt).
        if ((kt & 1) == 0) {
            const uint32_t zb = base + L::X_BYTES + L::W_BYTES + (uint32_t)(T5_ZS_WAVE * wave);
            if (lane >= 32 && lane < 40)
                buffer_load_lds_x1(rz, zs_voff, __builtin_amdgcn_readfirstlane((uint32_t)g * (uint32_t)pn * 4u),
                                   zb - 128u);
            if (lane < 32)
                buffer_load_lds_x1(rs, zs_voff, __builtin_amdgcn_readfirstlane((uint32_t)g * (uint32_t)a.N * 2u),
                                   zb + 32u);
        }
#pragma unroll
        for (int i = 0; i < L::X_LOADS; ++i)
            buffer_load_lds_x4(rx, x_voff + (uint32_t)(16 * i) * (uint32_t)a.K, __builtin_amdgcn_readfirstlane((uint32_t)k0 * 2u),
                               base + 1024u * (uint32_t)(L::X_LOADS * wave + i));
#pragma unroll
        for (int i = 0; i < L::W_LOADS; ++i)
            buffer_load_lds_x4(rw, w_voff, __builtin_amdgcn_readfirstlane((uint32_t)(k0 + 32 * i) * (uint32_t)pn * 4u),
                               base + L::X_BYTES + 2048u * (uint32_t)wave + 1024u * (uint32_t)i);
    };

    const uint32_t magic = magic_vgpr();        // for one v_and_or_b32 per k-pair
    const uint32_t magic_hi = magic_hi_vgpr();  // (nibbles cut in place)

    floatx4 acc[4][FM];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int f = 0; f < FM; ++f) acc[c][f] = floatx4{0.f, 0.f, 0.f, 0.f};

    {
        // Pipelined across k-steps.  Step kt runs in two phases of FM
        // chunks; chunk f issues the 4 MFMAs of x rows 16 f .. + 15 against
        // the phase's k-half, the read of the B fragment two chunks ahead,
        // and a share of the dequantisation the next phase needs:
        //   phase 0 (k-half 0): forms k-half 1's A fragments from weight
        //     nibbles already in registers;
        //   phase 1 (k-half 1): reads step kt + 1's weight nibbles, zero
        //     words and scales and forms its k-half 0 A fragments.  The wave
        //     loaded those itself, so its own vmcnt wait before the phase is
        //     all they need.
        // The dequantisation thus runs between the MFMAs of the same wave,
        // and each B fragment has two chunks of MFMAs to land.  The barrier
        // ending step kt publishes step kt + 1's x rows (every wave waited
        // for its own loads of that step) and frees stage kt, which the loads
        // of step kt + 3, issued after it, overwrite.
        //
        // Weights reach the A fragments through transpose reads
        // (ds_read_b64_tr_b4: within each 16-lane group, lane j receives
        // nibble j of the 8-byte row slices the group's 16 lanes address).
        // A fragment c (MFMA row n = lane % 16) is the 16-column chunk c of
        // the wave's 64 columns: packed columns 2 c and 2 c + 1, nibble n of
        // the 8-byte slice, i.e. logical column 8 (2 c + n / 8) +
        // 2 (n % 4) + (n % 8) / 4 (the AWQ nibble order).  Lane 16 kb + p
        // addresses row 32 (p / 8) + 8 kb + SIG(p % 8), SIG = 0 2 4 6 1 3 5 7,
        // so of the 64 bits each lane receives, the low dword holds k-half
        // 0's rows 8 kb .. + 7 in SIG order and the high dword k-half 1's:
        // masking 0x000F000F then gives rows (8 kb, 8 kb + 1) in one half
        // pair, 0x00F000F0 (the nibble in place, read with the 64.0 magic)
        // rows + 2, + 3, and the same on the dword shifted by 8 rows + 4 ..
        // + 7: the A fragment in k order, every column the exact q - z and
        // one fp16 rounding of (q - z) * s.
        static_assert(S == 3, "two steps in flight");
        const int sgi = n16 & 7;
        const int tr_row = 32 * (n16 >> 3) + 8 * kb + 2 * (sgi & 3) + (sgi >> 2);
        const int tr_sw = (tr_row >> 3) & 1;
        // Stage byte offsets of the lane's reads: transpose slices of chunks
        // 0, 1 at tr_lo + 8 c and 2, 3 at tr_hi + 8 (c - 2); B fragment of
        // (k-half h, rows 16 f ..) at x_rd[h] + 2048 f; zero word of packed
        // column 2 c + n16 / 8 at z_rd + 8 c; its scale at s_rd + 32 c.
        const uint32_t w_rd = (uint32_t)L::X_BYTES + 2048u * (uint32_t)wn + 32u * (uint32_t)tr_row;
        const uint32_t tr_lo = w_rd + 16u * (uint32_t)tr_sw;  // w_rd is 32-aligned: tr_hi = tr_lo ^ 16
        const uint32_t z_base = (uint32_t)(L::X_BYTES + L::W_BYTES + T5_ZS_WAVE * wn);
        const uint32_t z_rd = z_base + 4u * (uint32_t)(n16 >> 3);
        const uint32_t s_rd = z_base + 32u + 16u * (uint32_t)(n16 >> 3) + 2u * (uint32_t)(2 * (sgi & 3) + (sgi >> 2));
        const uint32_t zsh = 4u * (uint32_t)sgi;
        // k-half 1's chunk is k-half 0's with bit 2 flipped ((4 + kb) ^ c8 =
        // (kb ^ c8) ^ 4): its byte offset is x_rd ^ 64.
        const uint32_t x_rd = 128u * (uint32_t)n16 + 16u * (uint32_t)(kb ^ (n16 & 7));
        auto bfrag = [&](const unsigned char* st, int h, int f) {
            return *reinterpret_cast<const half8_t*>(st + (h ? x_rd ^ 64u : x_rd) + 2048 * f);
        };
        // The 64 transposed bits of chunk c: [0] k-half 0, [1] k-half 1.
        auto trread = [&](const unsigned char* st, int c) {
            typedef int v2i __attribute__((ext_vector_type(2)));
            const unsigned char* ptr = st + (c < 2 ? tr_lo : tr_lo ^ 16u) + 8 * (c & 1);
            const v2i v = __builtin_amdgcn_ds_read_tr4_b64_v2i32(
                (__attribute__((address_space(3))) v2i*)(ptr));
            return v;
        };
        // Zero splats (1024 + z and, for the in-place nibbles, 64 + z) and
        // the scale pair of the lane's column in each chunk.
        auto splats = [&](const unsigned char* st, uint32_t (&zl)[4], uint32_t (&zh)[4], uint32_t (&ss)[4]) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint32_t zw = *reinterpret_cast<const uint32_t*>(st + z_rd + 8 * c);
                const uint32_t sv = *reinterpret_cast<const uint16_t*>(st + s_rd + 32 * c);
                const uint32_t z = __builtin_amdgcn_ubfe(zw, zsh, 4);
                zl[c] = z * 0x00010001u + kMagic2;
                zh[c] = z * 0x00100010u + kMagic2Hi;
                ss[c] = sv | (sv << 16);
            }
        };
        // Dequantisation unit u (0 .. 7) of a k-half: chunk c = u / 2, words
        // 2 (u % 2) and 2 (u % 2) + 1 of its A fragment, from the chunk's
        // transposed dword d of that k-half.
        auto dq = [&](const uint32_t (&d)[4], const uint32_t (&zl)[4], const uint32_t (&zh)[4],
                      const uint32_t (&ss)[4], u32x4 (&af)[4], int u) {
            const int c = u >> 1, part = u & 1;
            const uint32_t v = part ? d[c] >> 8 : d[c];
            const uint32_t lo = and_or(v, 0x000F000Fu, magic), hi = and_or(v, 0x00F000F0u, magic_hi);
            af[c][2 * part] = as_u32((as_h2(lo) - as_h2(zl[c])) * as_h2(ss[c]));
            af[c][2 * part + 1] = as_u32((as_h2(hi) - as_h2(zh[c])) * as_h2(ss[c]));
        };
        // Phase 1 starts its dequantisation at chunk C0, once the reads it
        // issued in chunk 0 have had time to land.
        constexpr int C0 = FM >= 8 ? 2 : 1;
        // KT is even (whole groups), so steps come in (even, odd) pairs: the
        // even step's loads bring the group's zero words and scales, and the
        // odd step's phase 1 forms the next group's splats.
        if (KT > 0) {
            issue(0, 0);
            if (KT > 1) issue(1, 1);
            wait_batches<L::LOADS_NZ, 1>(min(1, KT - 1));
            uint32_t d1[4];                  // k-half 1 nibbles of the current step
            u32x4 afa[4], afb[4];            // A fragments of k-half 0 and 1
            uint32_t zl[4], zh[4], ss[4];    // splats of the current step's group
            {
                uint32_t d0[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const auto v = trread(smem, c);
                    d0[c] = (uint32_t)v[0];
                    d1[c] = (uint32_t)v[1];
                }
                splats(smem, zl, zh, ss);
#pragma unroll
                for (int u = 0; u < 8; ++u) dq(d0, zl, zh, ss, afa, u);
            }
            __syncthreads();
            int stage = 0;
            auto step = [&](int kt, auto odd_c) {
                constexpr bool ODD = decltype(odd_c)::value;
                if (kt + 2 < KT) issue(kt + 2, stage == 0 ? 2 : stage - 1);
                const unsigned char* st = smem + stage * L::STAGE;
                const int nstage = stage == 2 ? 0 : stage + 1;
                const unsigned char* sn = smem + nstage * L::STAGE;
                half8_t bq[3];  // B fragment i (h = i / FM, rows 16 (i % FM) ..) in bq[i % 3]
                __builtin_amdgcn_sched_barrier(0);
                bq[0] = bfrag(st, 0, 0);
                bq[1] = bfrag(st, 0, 1);
#pragma unroll
                for (int f = 0; f < FM; ++f) {
                    const int i = f + 2;
                    bq[i % 3] = bfrag(st, i / FM, i % FM);
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        acc[c][f] = mfma16x16x32(__builtin_bit_cast(half8_t, afa[c]), bq[f % 3], acc[c][f]);
#pragma unroll
                    for (int u = 8 * f / FM; u < 8 * (f + 1) / FM; ++u) dq(d1, zl, zh, ss, afb, u);
                    __builtin_amdgcn_sched_barrier(0);
                }
                // k-half 1's A fragments are formed here, under phase 0's
                // MFMAs: the empty asm uses them, so the compiler cannot sink
                // their dequantisation past the wait's branch into phase 1.
#pragma unroll
                for (int c = 0; c < 4; ++c) asm volatile("" ::"v"(afb[c]));
                // This wave's loads of step kt + 1 must have landed; those of
                // step kt + 2 (an even step's with the zero words and scales)
                // stay in flight.
                wait_batches<ODD ? L::LOADS_NZ : L::LOADS, 1>(max(0, min(1, KT - 2 - kt)));
                uint32_t d0[4];
#pragma unroll
                for (int f = 0; f < FM; ++f) {
                    const int i = FM + f + 2;
                    if (i < 2 * FM) bq[i % 3] = bfrag(st, 1, i - FM);
                    if (f == 0) {
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            const auto v = trread(sn, c);
                            d0[c] = (uint32_t)v[0];
                            d1[c] = (uint32_t)v[1];
                        }
                    }
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        acc[c][f] = mfma16x16x32(__builtin_bit_cast(half8_t, afb[c]), bq[(FM + f) % 3], acc[c][f]);
                    if constexpr (ODD) {
                        if (f == C0) splats(sn, zl, zh, ss);  // step kt + 1 starts a group
                    }
                    if (f >= C0) {
#pragma unroll
                        for (int u = 8 * (f - C0) / (FM - C0); u < 8 * (f - C0 + 1) / (FM - C0); ++u)
                            dq(d0, zl, zh, ss, afa, u);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                // Likewise step kt + 1's k-half 0 fragments, formed under
                // phase 1's MFMAs, not after the barrier.
#pragma unroll
                for (int c = 0; c < 4; ++c) asm volatile("" ::"v"(afa[c]));
                __syncthreads();
                stage = nstage;
            };
            for (int kt = 0; kt < KT; kt += 2) {
                step(kt, Parity<false>{});
                step(kt + 1, Parity<true>{});
            }
        }
    }

    // Output quads: acc[c][f] lane value r is column 64 wn + 16 c + 8 (kb >>
    // 1) + 2 r + (kb & 1) of tile row 16 f + n16 (the transposed fragments);
    // lanes l and l ^ 16 trade two values so that acc[c][f] holds the 4
    // consecutive columns 64 wn + 16 c + 8 (kb >> 1) + 4 (kb & 1) .. + 3.
    // The lane's indices are formed again here, the lane number counted
    // afresh (mbcnt): values shared with the code before the main loop would
    // otherwise stay in registers across it.
    const uint32_t eln = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    const int e16 = (int)(eln & 15u), ekb = (int)(eln >> 4);
    if constexpr (FIN == 1) {
        if (ks > 1) {
            // Split-K partials for the reduce launch, fragment-native: the
            // accumulator registers as they are, each store one whole
            // kilobyte (a wave's 64 lanes x 16 bytes), no exchange.  Unit
            // (split, 16-row block rb, 256-column tile tn) is 16 KB at
            // ((split x RB + rb) x NT + tn) x 16 KB, holding fragment (wave,
            // c) at (4 wave + c) KB; lane l's value r is output (16 rb + l %
            // 16, 256 tn + 64 wave + 16 c + 8 (kb >> 1) + 2 r + (kb & 1)), kb
            // = l / 16.  Blocks of rows at or beyond M are not written (nor
            // read by the reduce launch).
            // A 512-column tile (eight waves) writes two such units, waves
            // 4 .. 7 the second (none where it lies beyond N).
            const int RB = (a.M + 15) >> 4, NT = (a.N + T5_BN - 1) / T5_BN;
            const __amdgpu_buffer_rsrc_t rp = make_rsrc(a.partials, (uint32_t)((size_t)split_k * RB * NT * 16384));
            const int tn = n0 / T5_BN + (NW == 8 ? (wn >> 2) : 0);
            const int wq = NW == 8 ? (wn & 3) : wn;
            if (NW == 8 && tn >= NT) return;
#pragma unroll
            for (int f = 0; f < FM; ++f) {
                if (m0 + 16 * f >= a.M) break;
                const uint32_t unit = (uint32_t)(((split * RB + (m0 >> 4) + f) * NT + tn));
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    buf_store_f4_device(acc[c][f], rp, unit * 16384u + (uint32_t)((4 * wq + c) * 1024) + eln * 16u);
            }
            return;
        }
    }
    {
        const bool odd = ekb & 1;
        const int src = (int)((eln ^ 16u) << 2);
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int f = 0; f < FM; ++f) {
                const floatx4 v = acc[c][f];
                const float r0 = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(odd ? v[0] : v[2])));
                const float r1 = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(odd ? v[1] : v[3])));
                acc[c][f] = odd ? floatx4{r0, v[2], r1, v[3]} : floatx4{v[0], r0, v[1], r1};
            }
    }
    const int qcol = 64 * wn + 8 * (ekb >> 1) + 4 * (ekb & 1);  // + 16 c: the quad's first column in the tile
    // Hybrids: add the split_k pieces' partials of band h (of hb) of leftover
    // tile t ([split_k][n_sk][BM][256] fp32), write fp16, reset the band's
    // counter.  Called by the whole workgroup.
    auto hy_finish_band = [&](int t, int h, int hb) {
        if constexpr (HY) {
            int tm0, tn0;
            tile_origin(n_tiles * m_tiles - n_sk + t, tm0, tn0);
            const int br = BM / hb;
            const int row0 = tm0 + h * br;
            const uint32_t tile_bytes = (uint32_t)(BM * BN * 4);
            const PartLayout bp{(uint32_t)t * tile_bytes + (uint32_t)(h * br) * (uint32_t)(BN * 4),
                                (uint32_t)(BN * 4), (uint32_t)n_sk * tile_bytes};
            const __amdgpu_buffer_rsrc_t rpb = make_rsrc(a.partials, (uint32_t)split_k * bp.split_stride);
            const int rows = min(br, a.M - row0);
            if (rows > 0)
                splitk_finish<(FM >= 8 ? 16 : 8)>(rpb, a.out, a.bias, a.residual, a.M, a.N, row0, rows, tn0,
                                                  min(BN, a.N - tn0), split_k, fin, bp);
            if (tid == 0)
                __hip_atomic_store(&counters[t * hb + h], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    };
    if (ks == 1) {
        // The fp16 tile goes through LDS and leaves as whole rows: each
        // thread stores 16 bytes, 32 threads a 512-byte row, instead of every
        // store instruction writing 32 bytes into each of 16 rows.  Staged
        // rows are 544 bytes apart, so the 16 rows of a wave's 8-byte writes
        // start 8 banks apart.  The ring is free: every wave has passed the
        // last step's barrier, after which no load is in flight.
        constexpr int ROW = BN * 2 + 32;
        static_assert(BM * ROW <= L::SMEM, "the staged tile fits");
        typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
        typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
#pragma unroll
        for (int f = 0; f < FM; ++f)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const h4_t h = {(half_t)acc[c][f][0], (half_t)acc[c][f][1], (half_t)acc[c][f][2], (half_t)acc[c][f][3]};
                *reinterpret_cast<h4_t*>(smem + (16 * f + e16) * ROW + 2 * (qcol + 16 * c)) = h;
            }
        __syncthreads();
        const bool epi = a.bias || a.residual;
        const __amdgpu_buffer_rsrc_t ro = make_rsrc(a.out, (uint32_t)((size_t)a.M * a.N * 2));
#pragma unroll
        for (int p = tid; p < BM * (BN / 8); p += 64 * NW) {
            const int r = (int)((unsigned)p / (BN / 8)), c8 = 8 * (int)((unsigned)p % (BN / 8));
            const int m = m0 + r, n = n0 + c8;
            if (m >= a.M || n >= a.N) continue;
            h8_t h = *reinterpret_cast<const h8_t*>(smem + r * ROW + 2 * c8);
            const size_t o = (size_t)m * a.N + n;
            if (epi) {
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    h[i] = epi_round_vals((float)h[i], a.bias != nullptr, a.bias ? a.bias[n + i] : (half_t)0,
                                          a.residual != nullptr, a.residual ? a.residual[o + i] : (half_t)0);
            }
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, h), ro, (uint32_t)(o * 2), 0, kCpolSC1);
        }
        if constexpr (HY) {
            // Whole-tile workgroup b < n_sk * H helps finish band b % H of
            // leftover tile b / H (below).
            const int hb = hy_bands(n_sk, (int)gridDim.x - n_sk * split_k, BM);
            if ((int)blockIdx.x < n_sk * hb) {
                __syncthreads();  // the staged tile's reads are done: the LDS becomes `fin`
                if (tid == 0)
                    last_flag = __hip_atomic_fetch_add(&counters[blockIdx.x], 1u, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)split_k;
                __syncthreads();
                if (last_flag) hy_finish_band((int)blockIdx.x / hb, (int)blockIdx.x % hb, hb);
            }
        }
        return;
    }

    if constexpr (FIN == 1) return;  // split_k > 1 returned above
    // FIN 0 (the last-arriver finish).  Partials of this workgroup's split:
    // [split_k, M, N], or for the hybrid's pieces [split_k][n_sk][BM][256]
    // (PartLayout: byte base + r row_stride + 4 c + split split_stride for
    // output (m0 + r, n0 + c)).
    const PartLayout pl = HY ? PartLayout{(uint32_t)sk_tile * (uint32_t)(BM * BN * 4), (uint32_t)(BN * 4),
                                          (uint32_t)n_sk * (uint32_t)(BM * BN * 4)}
                             : full_parts(a.M, a.N, m0, n0);
    const uint32_t part_bytes = HY ? (uint32_t)split_k * pl.split_stride : (uint32_t)((size_t)split_k * a.M * a.N * 4);
    const __amdgpu_buffer_rsrc_t rp_ = make_rsrc(a.partials, part_bytes);
#pragma unroll
    for (int f = 0; f < FM; ++f) {
        const int m = m0 + 16 * f + e16;
        if (m >= a.M) continue;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int col = qcol + 16 * c;
            if (n0 + col >= a.N) continue;
            const uint32_t off = pl.base + (uint32_t)(16 * f + e16) * pl.row_stride + (uint32_t)col * 4u +
                                 (uint32_t)split * pl.split_stride;
            buf_store_f4_device(acc[c][f], rp_, off);
        }
    }
    wait_vm_stores();
    __syncthreads();
    if constexpr (HY) {
        // Band h of this leftover tile has a counter of its own that its
        // split_k pieces and one helper (a whole-tile workgroup, after its
        // own tile) each add 1 to; whoever brings it to split_k + 1 adds the
        // band's partials.  The helpers run late, so usually they do, spread
        // over many workgroups instead of one last piece per tile.
        const int hb = hy_bands(n_sk, (int)gridDim.x - n_sk * split_k, BM);
        if (tid < hb)
            last_band[tid] = __hip_atomic_fetch_add(&counters[sk_tile * hb + tid], 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)split_k;
        __syncthreads();
        for (int h = 0; h < hb; ++h)
            if (last_band[h]) hy_finish_band(sk_tile, h, hb);
        return;
    }
    if (tid == 0)
        last_flag = __hip_atomic_fetch_add(&counters[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                    (uint32_t)(split_k - 1);
    __syncthreads();
    if (!last_flag) return;
    // Quads per thread in flight while summing: 16 fit the 128-row tile's
    // registers; the 64-row tile (three workgroups per CU, 168 VGPRs) takes
    // 8 so that nothing spills.
    splitk_finish<(FM >= 8 ? 16 : 8)>(rp_, a.out, a.bias, a.residual, a.M, a.N, m0, min(BM, a.M - m0), n0,
                                      min(BN, a.N - n0), split_k, fin, pl);
    if (tid == 0) __hip_atomic_store(&counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Second launch of tile variants 7, 8, 9 with split_k > 1: out = fp16(sum
// over the splits of the fragment-native partials), each output summed in
// split order (deterministic), with the bias / residual epilogue.  A thread
// takes 8 consecutive columns of one output row: lanes 32 j + n and 32 j +
// 16 + n of a fragment (k-blocks 2 j and 2 j + 1) hold them interleaved
// (even and odd columns).  P threads share such a piece (splits p, p + P,
// ...; at most eight splits each) and combine
// through LDS in part order.  32 consecutive threads read one kilobyte.
__global__ __launch_bounds__(256) void awq_tile_reduce_kernel(const float* __restrict__ partials, half_t* __restrict__ out,
                                                             const half_t* bias, const half_t* residual, int M, int N,
                                                             int split_k, int P) {
    __shared__ floatx4 fin[2][256];
    const int per_wg = 256 / P;  // pieces per workgroup
    const int t = threadIdx.x;
    const int part = t / per_wg;
    const int RB = (M + 15) >> 4, NT = (N + T5_BN - 1) / T5_BN;
    const int piece = blockIdx.x * per_wg + t % per_wg;
    const int u = piece >> 9, in = piece & 511;     // unit rb x NT + tn; 512 pieces a unit
    const int wc = in >> 5, j = (in >> 4) & 1, n16 = in & 15;
    const int rb = u / NT, tn = u - rb * NT;
    const int m = 16 * rb + n16;
    const int n = T5_BN * tn + 64 * (wc >> 2) + 16 * (wc & 3) + 8 * j;
    const bool valid = u < RB * NT && m < M && n < N;
    floatx4 sa = {0.f, 0.f, 0.f, 0.f}, sb = {0.f, 0.f, 0.f, 0.f};
    if (valid) {
        // In float4: a unit is 1024, a fragment 64, lane 32 j + n16.
        const floatx4* p = reinterpret_cast<const floatx4*>(partials) + (size_t)u * 1024 + 64 * wc + 32 * j + n16;
        const size_t step = (size_t)RB * NT * 1024;  // one split
#pragma unroll 4
        for (int sp = part; sp < split_k; sp += P) {
            sa += __builtin_nontemporal_load(p + (size_t)sp * step);
            sb += __builtin_nontemporal_load(p + (size_t)sp * step + 16);
        }
    }
    fin[0][t] = sa;
    fin[1][t] = sb;
    __syncthreads();
    if (valid && part == 0) {
        for (int i = 1; i < P; ++i) {
            sa += fin[0][i * per_wg + t];
            sb += fin[1][i * per_wg + t];
        }
        const float y[8] = {sa[0], sb[0], sa[1], sb[1], sa[2], sb[2], sa[3], sb[3]};
        store_out<8>(out, bias, residual, N, m, n, y);
    }
}

int64_t tile_reduce_blocks(int M, int N, int split_k) {
    const int64_t pieces = (int64_t)((M + 15) / 16) * ((N + T5_BN - 1) / T5_BN) * 512;
    const int64_t per_wg = 256 / stream_reduce_parts(split_k);
    return (pieces + per_wg - 1) / per_wg;
}

uint64_t tile_partials_bytes(int64_t split_k, int64_t M, int64_t N) {
    return (uint64_t)split_k * (uint64_t)((M + 15) / 16) * (uint64_t)((N + T5_BN - 1) / T5_BN) * 16384u;
}

int64_t tile_tiles(int M, int N, int variant) {
    const int bm = tile5_rows(variant), bn = tile5_cols(variant);
    return (int64_t)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
}

hipError_t launch_tile(const GemmArgs& a, const TileConfig& cfg, uint32_t* counters, hipStream_t stream) {
    if (tile_variant_served(cfg.variant)) {
        const int64_t blocks = tile_hybrid(cfg.variant) ? cfg.grid : tile_tiles(a.M, a.N, cfg.variant) * cfg.split_k;
        if (blocks == 0) return hipSuccess;
        const dim3 grid((unsigned)blocks);
        bool reduce = false;
        switch (cfg.variant) {
            case 6: hipLaunchKernelGGL((awq_tile_kernel<8, 0>), grid, dim3(256), 0, stream, a, cfg.split_k, cfg.k_per_split, counters); break;
            case 7: hipLaunchKernelGGL((awq_tile_kernel<8, 1>), grid, dim3(256), 0, stream, a, cfg.split_k, cfg.k_per_split, counters); reduce = true; break;
            case 8: hipLaunchKernelGGL((awq_tile_kernel<4, 1>), grid, dim3(256), 0, stream, a, cfg.split_k, cfg.k_per_split, counters); reduce = true; break;
            case 9: hipLaunchKernelGGL((awq_tile_kernel<2, 1>), grid, dim3(256), 0, stream, a, cfg.split_k, cfg.k_per_split, counters); reduce = true; break;
            case 15: hipLaunchKernelGGL((awq_tile_kernel<8, 1, false, 8>), grid, dim3(512), 0, stream, a, cfg.split_k, cfg.k_per_split, counters); reduce = true; break;
            case 13: hipLaunchKernelGGL((awq_tile_kernel<8, 0, true>), grid, dim3(256), 0, stream, a, cfg.split_k, cfg.k_per_split, counters); break;
            case 14: hipLaunchKernelGGL((awq_tile_kernel<4, 0, true>), grid, dim3(256), 0, stream, a, cfg.split_k, cfg.k_per_split, counters); break;
            default: return hipErrorInvalidValue;
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess || !reduce || cfg.split_k <= 1) return e;
        hipLaunchKernelGGL(awq_tile_reduce_kernel, dim3((unsigned)tile_reduce_blocks(a.M, a.N, cfg.split_k)), dim3(256),
                           0, stream, a.partials, a.out, a.bias, a.residual, a.M, a.N, cfg.split_k,
                           stream_reduce_parts(cfg.split_k));
        return hipGetLastError();
    }
    return hipErrorInvalidValue;
}

}  // namespace awq
