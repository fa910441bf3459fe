// C ABI of the W4A16 AWQ GEMM library: validation, shape dispatch, launches.
// Declarations and the reference interfaces they replace: include/awq_w4a16.h.
#include <limits.h>
#include <stdint.h>

#include <atomic>
#include <mutex>

#include "../../include/awq_w4a16.h"
#include "awq_kernels.h"

using namespace awq;

namespace {

// Largest M the skinny path serves (4 MFMA blocks of 16 rows).
constexpr int64_t kSkinnyMaxM = 64;
// LDS the skinny dispatcher allows one workgroup for its K reduction.
constexpr uint64_t kSkinnyLdsBudget = 64 * 1024;

// Compute units of an MI355X: the planner's count where no device answers
// (a host without a GPU that plans ahead).
constexpr int64_t kDefaultCUs = 256;
constexpr int kMaxDevices = 64;
std::atomic<int> g_cus[kMaxDevices];  // per device, 0 until looked up
// Compute units of the current device, looked up once per device: every grid
// and split count below is sized by it, so a partitioned or smaller device
// gets grids for its own CU count.
int64_t cus() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return kDefaultCUs;
    int n = g_cus[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        n = (int)kDefaultCUs;
    g_cus[dev].store(n, std::memory_order_relaxed);
    return n;
}
// Largest M awq_fp16_linear serves (decode: the last position's logits).
constexpr int64_t kFp16LinearMaxM = 8;

constexpr int64_t kIndexLimit = (int64_t)1 << 30;
// K bound that keeps every 32-bit buffer offset in range, including the rows
// past M that a tile reads as zeros: (M + 256) * K * 2 < 2^32 (tiles hold at
// most 128 rows; the bound keeps a margin).
constexpr int64_t kMaxK = (int64_t)1 << 22;
// Byte-size limit of any one operand (buffer descriptors carry 32-bit sizes).
constexpr int64_t kBytesLimit = ((int64_t)1 << 31) - 1;

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int check_dims(int64_t M, int64_t N, int64_t K, int32_t G) {
    if (G != kGroup) return AWQ_ERR_GROUP_SIZE;
    if (M < 0 || N <= 0 || K <= 0 || N % 8 != 0 || K % G != 0) return AWQ_ERR_BAD_DIMS;
    if (M > kIndexLimit || N > kMaxN || K > kMaxK) return AWQ_ERR_TOO_LARGE;
    if (K * (N / 2) > kBytesLimit || M * K * 2 > kBytesLimit || M * N * 2 > kBytesLimit)
        return AWQ_ERR_TOO_LARGE;
    return AWQ_OK;
}

// Workspace bytes of a plan that keeps fp32 partials [split, M, N].
uint64_t partials_workspace(int64_t split, int64_t M, int64_t N) {
    return kPartialsOffset + (uint64_t)split * (uint64_t)M * (uint64_t)N * 4u;
}

bool valid_rows_per_wave(int64_t r, int64_t K) {
    if (r == 32 || r == 64) return true;
    return r > 0 && r % kGroup == 0 && r <= K;
}

int m_blocks_for(int64_t M) { return M <= 16 ? 1 : (M <= 32 ? 2 : 4); }

// Fills every field of a skinny plan from its tuning values.
int fill_skinny(int64_t M, int64_t N, int64_t K, int64_t rows_per_wave, int64_t k_waves, int64_t variant,
                int64_t factored, awq_w4a16_plan* p) {
    if (M > kSkinnyMaxM) return AWQ_ERR_PATH;
    if (!valid_rows_per_wave(rows_per_wave, K)) return AWQ_ERR_PATH;
    if (!(k_waves == 1 || k_waves == 2 || k_waves == 4)) return AWQ_ERR_PATH;
    const int mb = m_blocks_for(M);
    // Kernel instances that exist: see launch_skinny.
    if (variant == 1) {
        if (mb != 1) return AWQ_ERR_PATH;
    } else if (variant == 2) {
        if (mb == 4 && factored) return AWQ_ERR_PATH;
    } else {
        return AWQ_ERR_PATH;
    }
    if (factored != 0 && factored != 1) return AWQ_ERR_PATH;
    const int64_t rows_per_block = rows_per_wave * k_waves;
    p->path = AWQ_PATH_SKINNY;
    p->variant = (int32_t)variant;
    p->tile_m = 16 * mb;
    p->tile_n = kSkinnyCols;
    p->rows_per_wave = (int32_t)rows_per_wave;
    p->k_waves = (int32_t)k_waves;
    p->split_k = (int32_t)((K + rows_per_block - 1) / rows_per_block);
    p->block_threads = (int32_t)(128 * k_waves);
    p->factored_scale = (int32_t)factored;
    p->depth = 0;
    p->grid = skinny_blocks((int)N, (int)K, (int)rows_per_wave, (int)k_waves);
    p->workspace_bytes = p->split_k > 1 ? partials_workspace(p->split_k, M, N) : 0u;
    p->lds_bytes = skinny_lds_bytes((int)M, mb, (int)k_waves);
    if (p->lds_bytes > kSkinnyLdsBudget) return AWQ_ERR_PATH;
    if (p->workspace_bytes > (uint64_t)kBytesLimit) return AWQ_ERR_TOO_LARGE;
    return AWQ_OK;
}

// Defaults measured on MI355X (K range per wave x waves per workgroup x main
// loop swept over the Qwen2-7B shapes at M = 4 and 16).  K rows per split
// (rows_per_wave x waves): wide N (>= 64 column-tile pairs) -- 1024 rows for
// M <= 4, all of K above (the split-K partials grow with M); narrow N --
// 512 rows for K <= 8192, else 1024 (M <= 4) or 2048.  Four waves along K
// for narrow N, two for wide N (fewer waves, more workgroups), fewer when
// the LDS reduction would not fit; the chunk-pipelined main loop for K
// ranges of 512 rows per wave and more, the plain loop otherwise.
int skinny_plan(int64_t M, int64_t N, int64_t K, awq_w4a16_plan* p) {
    if (M > kSkinnyMaxM) return AWQ_ERR_PATH;
    const int mb = m_blocks_for(M);
    const bool wide = skinny_pairs((int)N) >= 64;
    int64_t kw = wide ? 2 : 4;
    while (kw > 1 && skinny_lds_bytes((int)M, mb, (int)kw) > kSkinnyLdsBudget) kw /= 2;
    int64_t rows_per_split;
    if (wide) rows_per_split = M <= 4 ? 1024 : K;
    else if (K > 8192) rows_per_split = M <= 4 ? 1024 : 2048;
    else rows_per_split = 512;
    const int64_t want = (rows_per_split + kw - 1) / kw;
    int64_t r = want <= 32 ? 32 : (want <= 64 ? 64 : (want + kGroup - 1) / kGroup * kGroup);
    if (r > K) r = K;
    const int64_t variant = (mb == 1 && r >= 512) ? 1 : 2;
    return fill_skinny(M, N, K, r, kw, variant, mb == 4 ? 0 : 1, p);
}

// AUTO takes the skinny kernel up to M = 16 (where the stream path does not
// serve); above, the tile planner's 32- and 64-row tiles are faster on every
// Qwen2-7B shape (measured at M = 32 and 64).
bool auto_skinny(int64_t M, int64_t /*N*/) { return M <= 16; }

// Largest M the GEMV path serves.
constexpr int64_t kGemvMaxM = 2;
constexpr int64_t kGemvPairMaxM = 8;
constexpr int64_t kGemvSingleMaxM = 8;
// LDS the column-quad GEMV may stage per workgroup.
constexpr uint64_t kQuadLdsBudget = 96 * 1024;

// 512-column strips (tile_n = 512).  Variant 2: k_waves = 128 /
// rows_per_wave, split_k in 1 .. K/128 with each split a whole number of
// groups, depth 2 .. 4 chunk buffers (3 at most for 32 rows).  Variant 5:
// see below.
int fill_gemv(int64_t M, int64_t N, int64_t K, int64_t variant, int64_t tile_n, int64_t rows_per_wave,
              int64_t k_waves, int64_t split_k, int64_t depth, awq_w4a16_plan* p) {
    // Column pairs and singles (variant 5 with 256- and 128-column strips)
    // carry up to 4 and 8 rows of x; variant 6 (singles with fp32 partials
    // and the reduce launch) 9 .. 16.
    const bool red = variant == 6;
    const bool pairs = (variant == 5 || red) && (tile_n == 256 || tile_n == 128);
    // Rows of x: 2 for the quads, 4 for pairs, 8 for singles, 16 for variant 6.
    const int64_t max_m = red ? 16 : (pairs ? (tile_n == 128 ? kGemvPairMaxM : 4) : kGemvMaxM);
    if (red && (tile_n != 128 || M < 9)) return AWQ_ERR_PATH;
    if (M > max_m) return AWQ_ERR_PATH;
    p->path = AWQ_PATH_GEMV;
    p->variant = (int32_t)variant;
    p->tile_m = (int32_t)max_m;
    p->tile_n = (int32_t)tile_n;
    p->rows_per_wave = (int32_t)rows_per_wave;
    p->k_waves = (int32_t)k_waves;
    p->block_threads = (int32_t)(64 * k_waves);
    p->factored_scale = 1;
    p->depth = 0;
    if (tile_n != 512 && !pairs) return AWQ_ERR_PATH;
    if (variant == 5 || variant == 6) {
        // Column quads (512-column strips, M <= 2) or column pairs (256-column
        // strips, M <= 4) with MFMA column sums: N % 32 == 0; rows_per_wave 0;
        // depth 2 .. 4 chunk buffers per wave (2 .. 3 for pairs; each strip's
        // K/32 chunks are divided evenly over split_k workgroups of k_waves
        // waves); split_k <= min(K/32, kFixMaxSplit); the groups and x rows a
        // workgroup stages must fit its prologue loads, and the staged data
        // its LDS.
        const int cw = (int)(tile_n / 128);
        if (N % 32 != 0 || rows_per_wave != 0 || depth < 2 || depth > (pairs ? 3 : 4)) return AWQ_ERR_PATH;
        if (k_waves < 1 || k_waves > 8 || split_k < 1 || split_k > K / 32 || split_k > kFixMaxSplit)
            return AWQ_ERR_PATH;
        if (!gemv_quad_fits((int)M, (int)K, (int)split_k, (int)k_waves, cw)) return AWQ_ERR_PATH;
        p->split_k = (int32_t)split_k;
        p->depth = (int32_t)depth;
        p->grid = gemv_strips_cw((int)N, cw) * split_k;
        if (red) {
            if (depth != 2) return AWQ_ERR_PATH;
            p->workspace_bytes = split_k > 1 ? partials_workspace(split_k, M, N) : 0u;
        } else {
            if (split_k > 1 && (uint64_t)M * (uint64_t)N * 8u > kSlotBytes) return AWQ_ERR_PATH;
            p->workspace_bytes = split_k > 1 ? kCounterBytes + (uint64_t)M * (uint64_t)N * 8u : 0u;
        }
        p->lds_bytes = gemv_quad_lds_bytes((int)M, (int)K, (int)split_k, (int)k_waves, cw);
        if (p->lds_bytes > kQuadLdsBudget) return AWQ_ERR_PATH;
        if (p->workspace_bytes > (uint64_t)kBytesLimit) return AWQ_ERR_TOO_LARGE;
        return AWQ_OK;
    }
    if (variant == 2) {
        if (!(rows_per_wave == 16 || rows_per_wave == 32) || k_waves * rows_per_wave != kGroup) return AWQ_ERR_PATH;
        if (depth < 2 || depth > (rows_per_wave == 16 ? 4 : 3)) return AWQ_ERR_PATH;
        p->depth = (int32_t)depth;
        const int64_t groups = K / kGroup;
        if (split_k < 1 || split_k > groups) return AWQ_ERR_PATH;
        const int64_t per = (groups + split_k - 1) / split_k;
        if ((groups + per - 1) / per != split_k) return AWQ_ERR_PATH;
        if (split_k > 1 && gemv_strips((int)N) * 4 > (int64_t)kCounterBytes) return AWQ_ERR_PATH;
        p->split_k = (int32_t)split_k;
        p->grid = gemv_strips((int)N) * split_k;
    } else {
        return AWQ_ERR_PATH;
    }
    p->workspace_bytes = p->split_k > 1 ? partials_workspace(p->split_k, M, N) : 0u;
    p->lds_bytes = 0;
    if (p->workspace_bytes > (uint64_t)kBytesLimit) return AWQ_ERR_TOO_LARGE;
    return AWQ_OK;
}

// Measured default (MI355X, Qwen2-7B shapes): the K-streaming variant, 16
// rows per wave (8 waves), 3 chunks in flight, and as many K splits as keep
// the grid within one workgroup per CU (more workgroups than CUs leaves some
// CUs with twice the work), at least 2 chunks per split.
int64_t stream_split(int64_t N, int64_t K);

// Column-quad GEMV (variant 5) shape: as many K splits as keep the grid
// within one workgroup per CU (a CU holding two workgroups finishes last),
// four waves per workgroup (measured: interleaved chunks of four waves
// stream faster than eight), fewer when a workgroup has fewer chunks; more
// splits or waves when the staged consts would not fit.
int quad_plan(int64_t M, int64_t N, int64_t K, awq_w4a16_plan* p) {
    const int64_t strips = gemv_strips((int)N);
    const int64_t C = K / 32;
    int64_t split = cus() / strips;
    if (split > C) split = C;
    if (split > kFixMaxSplit) split = kFixMaxSplit;
    if (split < 1) split = 1;
    // Waves: one per chunk of the split, rounded up, four at most (3584 x 3584
    // at 36 splits of 3 - 4 chunks: 6.9 us with four waves, 7.1 with three).
    int64_t w = (C + split - 1) / split;
    if (w > 4) w = 4;
    if (w < 1) w = 1;
    while (!gemv_quad_fits((int)M, (int)K, (int)split, (int)w, 4) ||
           gemv_quad_lds_bytes((int)M, (int)K, (int)split, (int)w, 4) > kQuadLdsBudget) {
        if (w < 8) ++w;
        else if (split < C && split < kFixMaxSplit) ++split;
        else break;
    }
    return fill_gemv(M, N, K, 5, 512, 0, w, split, 2, p);
}

// Column singles (128-column strips, up to 4 rows of x) on narrow weights
// (fewer than 16 strips of 512 columns): four times the strips of the
// quads, so one workgroup per CU needs a quarter of the K splits, and the
// fixed-point finish a quarter of the atomics.  Two strips share each
// 128-byte line; the kernel's XCD-ordered work items keep them on one L2.
// Measured against the previous AUTO plans (graphs over >= 640 MB of
// weights; us), M = 1 / 2 / 3 / 4:
//   3584 x 4608 (four waves): singles 5.77 / 6.44 / 7.36 / 7.56, pairs (256
//     columns) 5.89 / - / - / -, before 7.47 / 8.13 / 9.06 / 9.51;
//   3584 x 3584 (four waves): singles 5.59 / 6.26 / 7.18 / 7.31, pairs 5.72,
//     before 6.79 / 7.96 / 8.82 / 9.22;
//   18944 x 3584 (eight waves): singles 10.98 / 11.50 / 12.46 / 12.56, pairs
//     11.03 / 12.12, before 12.28 / 12.92 / 13.75 / 14.67;
//   3584 x 37888: the quads (M = 1) and stream kernels (M >= 2) stay ahead
//     (unsplit singles and pairs stream too long a K range per workgroup).
// At M = 5 .. 8 (eight rows of x, eight waves): 3584 x 4608 9.07 / 9.14 /
// 9.34 us at M = 5 / 6 / 8 against 9.4 - 9.5 for the 32-row tile; 3584 x 3584
// 8.83 / 8.91 / 9.12 against 9.3 - 9.45; 18944 x 3584 14.5 / 14.2 / 14.45
// against 15.9 - 16.1 for the stream kernel with its reduce launch.
bool auto_pairs(int64_t M, int64_t N, int64_t K) {
    // Measured on 3584 - 4608 columns (28 - 36 strips of 128); narrower
    // weights keep the plans measured for them.
    if (N % 32 != 0 || gemv_strips((int)N) >= 16 || gemv_strips_cw((int)N, 2) < 8) return false;
    return M <= kGemvSingleMaxM;
}

int pair_plan(int64_t M, int64_t N, int64_t K, awq_w4a16_plan* p) {
    const int cw = 1;
    const int64_t strips = gemv_strips_cw((int)N, cw);
    const int64_t C = K / 32;
    int64_t split = cus() / strips;
    if (split > C) split = C;
    if (split > kFixMaxSplit) split = kFixMaxSplit;
    if (split < 1) split = 1;
    int64_t w = (K >= 8192 || M > 4) ? 8 : 4;
    while (!gemv_quad_fits((int)M, (int)K, (int)split, (int)w, cw) ||
           gemv_quad_lds_bytes((int)M, (int)K, (int)split, (int)w, cw) > kQuadLdsBudget) {
        if (w < 8) ++w;
        else if (split < C && split < kFixMaxSplit) ++split;
        else return AWQ_ERR_PATH;
    }
    return fill_gemv(M, N, K, 5, 128 * cw, 0, w, split, 2, p);
}

// Two more width classes for the column pairs and singles, from sweeps of
// every strip width, split, wave count and depth against the previous AUTO
// (graphs over >= 400 MB of weights; us):
//  * slim weights (256 <= N < 2048: 1 - 7 strips of 256 columns; 2048 <= K <
//    8192):
//    singles with two waves, four 32-row chunks per workgroup, at M <= 8 --
//    3584 x 512 at M = 1 / 2 / 4 / 8: 4.56 / 5.04 / 5.79 / 7.41 against 8.14 /
//    7.63 / 8.67 / 10.36 for the quads split 112 ways (112 fixed-point atomics
//    on each output) and the stream and skinny kernels on 18 and 14
//    workgroups; at M = 9 .. 16 the 16-row singles (variant 6, eight waves)
//    with one workgroup per CU: 9.51 against 12.84 at M = 16.
//  * wide, shallow weights (>= 16 strips of 512 columns, K < 8192) whose
//    256-column strips leave at least three splits per CU: pairs at M <= 2,
//    singles at M = 3 .. 8, split CUs / strips of 256 -- 3584 x 18944 at M = 1
//    / 2 / 4 / 8: 10.61 / 11.89 / 13.64 / 16.02 against 12.30 / 13.09 / 14.46 /
//    16.88 for the quads and the stream kernel.  3584 x 37888 (1.7 splits per
//    CU) keeps those: its best pair plans were 3 % faster at M <= 2 and 6 - 42 %
//    slower at M = 4 - 8.
constexpr int64_t kSlimMinN = 256;
constexpr int64_t kSlimMinK = 2048;

int strip_fit(int64_t M, int64_t N, int64_t K, int variant, int cw, int64_t split, int64_t w,
              awq_w4a16_plan* p) {
    const int64_t C = K / 32;
    if (split > C) split = C;
    if (split > kFixMaxSplit) split = kFixMaxSplit;
    if (split < 1) split = 1;
    while (!gemv_quad_fits((int)M, (int)K, (int)split, (int)w, cw) ||
           gemv_quad_lds_bytes((int)M, (int)K, (int)split, (int)w, cw) > kQuadLdsBudget) {
        if (w < 8) ++w;
        else if (split < C && split < kFixMaxSplit) ++split;
        else return AWQ_ERR_PATH;
    }
    awq_w4a16_plan q;
    if (fill_gemv(M, N, K, variant, 128 * cw, 0, w, split, 2, &q) != AWQ_OK) return AWQ_ERR_PATH;
    *p = q;
    return AWQ_OK;
}

int strip_class_plan(int64_t M, int64_t N, int64_t K, awq_w4a16_plan* p) {
    if (N % 32 != 0 || M > 16) return AWQ_ERR_PATH;
    const int64_t s128 = gemv_strips_cw((int)N, 1), s256 = gemv_strips_cw((int)N, 2);
    if (N >= kSlimMinN && s256 < 8 && K >= kSlimMinK && K < 8192) {
        const int64_t four_chunks = (K / 32) / 4, fill = cus() / s128;
        if (M <= kGemvSingleMaxM) return strip_fit(M, N, K, 5, 1, four_chunks < fill ? four_chunks : fill, 2, p);
        if (M >= 9) return strip_fit(M, N, K, 6, 1, fill, 8, p);
        return AWQ_ERR_PATH;
    }
    if (gemv_strips((int)N) >= 16 && K < 8192 && cus() / s256 >= 3 && M <= kGemvSingleMaxM) {
        if (M <= 2) return strip_fit(M, N, K, 5, 2, cus() / s256, M == 1 ? 4 : 8, p);
        return strip_fit(M, N, K, 5, 1, cus() / s256, 4, p);
    }
    return AWQ_ERR_PATH;
}

// Column quads while their fixed-point slots (M x N x 8 bytes) fit the slot
// region; else (and for N % 32 != 0) the K-streaming variant 2, whose fp32
// partials have no such limit.
int gemv_plan(int64_t M, int64_t N, int64_t K, awq_w4a16_plan* p) {
    if (N % 32 == 0 && quad_plan(M, N, K, p) == AWQ_OK) return AWQ_OK;
    return fill_gemv(M, N, K, 2, 512, 16, 8, stream_split(N, K), 3, p);
}

// Split count of the K-streaming kernels: as many K splits as keep the grid
// within one workgroup per CU, at least 2 groups per split.
int64_t stream_split(int64_t N, int64_t K) {
    const int64_t groups = K / kGroup;
    const int64_t strips = gemv_strips((int)N);
    int64_t split = cus() / strips;
    if (split > groups / 2) split = groups / 2;
    if (split < 1) split = 1;
    const int64_t per = (groups + split - 1) / split;
    return (groups + per - 1) / per;
}

// Stream path (M <= 16): 16x16x32 MFMA, zero/scale folded once per 128-row
// group; row layout (M <= 8, whole 256-byte row segments per load) or
// half-strip layout (M <= 16).
constexpr int64_t kStreamMaxM = 16;
constexpr uint64_t kStreamLdsBudget = 160 * 1024 - 64;

// rows_per_wave: kStreamRowLayout (16) or kStreamHalfLayout (32).  variant 1:
// fixed-point split-K finish; 2: fp32 partials, last-arriving workgroup per
// strip; 3: fp32 partials added by a second launch.
int fill_stream(int64_t M, int64_t N, int64_t K, int64_t rows_per_wave, int64_t variant, int64_t k_waves,
                int64_t split_k, int64_t depth, awq_w4a16_plan* p) {
    if (M > kStreamMaxM || N % 32 != 0 || variant < 1 || variant > 3) return AWQ_ERR_PATH;
    const bool row = rows_per_wave == kStreamRowLayout;
    if (!row && rows_per_wave != kStreamHalfLayout) return AWQ_ERR_PATH;
    if (row && M > 8) return AWQ_ERR_PATH;
    if (row ? !((depth == 2 && (k_waves == 1 || k_waves == 2 || k_waves == 4 || k_waves == 8)) ||
                (depth == 1 && (k_waves == 4 || k_waves == 8)))
            : !((depth == 2 && k_waves <= 4) || ((depth == 4 || depth == 6) && k_waves <= 2)))
        return AWQ_ERR_PATH;
    if (variant == 2 && split_k > 1 && gemv_strips((int)N) * 4 > (int64_t)kCounterBytes) return AWQ_ERR_PATH;
    if (variant == 1 && split_k > kFixMaxSplit) return AWQ_ERR_PATH;
    if (variant == 1 && split_k > 1 && (uint64_t)M * (uint64_t)N * 8u > kSlotBytes) return AWQ_ERR_PATH;
    if (k_waves < 1 || split_k < 1) return AWQ_ERR_PATH;
    if (!stream_fits((int)M, (int)K, (int)split_k, (int)k_waves, (int)rows_per_wave)) return AWQ_ERR_PATH;
    p->path = AWQ_PATH_STREAM;
    p->variant = (int32_t)variant;
    p->tile_m = row ? 8 : 16;
    p->tile_n = 512;
    p->rows_per_wave = (int32_t)rows_per_wave;
    p->k_waves = (int32_t)k_waves;
    p->split_k = (int32_t)split_k;
    p->block_threads = (int32_t)stream_threads((int)rows_per_wave, (int)k_waves);
    p->factored_scale = 1;
    p->depth = (int32_t)depth;
    p->grid = gemv_strips((int)N) * split_k;
    p->workspace_bytes = split_k <= 1 ? 0u
                         : variant == 1 ? kCounterBytes + (uint64_t)M * (uint64_t)N * 8u
                                        : partials_workspace(split_k, M, N);
    p->lds_bytes = stream_lds_bytes((int)M, (int)K, (int)split_k, (int)k_waves, (int)rows_per_wave);
    if (p->lds_bytes > kStreamLdsBudget) return AWQ_ERR_PATH;
    if (p->workspace_bytes > (uint64_t)kBytesLimit) return AWQ_ERR_TOO_LARGE;
    return AWQ_OK;
}

// Stream plan (measured on the Qwen2-7B shapes at M = 2 .. 16, every layout,
// finish, wave count and split of 3 .. 36): split K into groups so that the
// grid fills the device with one workgroup per CU, keeping about 1.5 groups
// per workgroup or more (2 x groups / 3 splits at most: 18 on K = 3584,
// 3 - 4 % faster than 14 at M = 3 and 4).  Layouts:
//   M <= 2: half-strip layout with two wave pairs where a split holds at
//     most two groups (K = 3584: 8.3 us against 9.7 for the column-quad
//     GEMV), else the row layout with four waves and two chunk buffers
//     (18944 x 3584: 13.0 us against 15.0);
//   M <= 8: row layout, eight waves sharing every group, one chunk buffer;
//     at M >= 5 with more than 8 splits, four waves and two buffers
//     (18944 x 3584: 16.3 us against 17.4 at M = 5, 16.7 against 17.5 at 8);
//   M <= 16: half-strip layout, four wave pairs, two buffers.
// Finish: fixed-point atomics for M <= 4 (one atomic per output element and
// split: cheapest while M * N * split stays a few hundred thousand) while
// their slots fit; above, the last-arriving workgroup of a strip while the
// partials it reads stay small (M * split <= 32), else a second launch that
// adds the partials over the whole device.
int stream_plan(int64_t M, int64_t N, int64_t K, awq_w4a16_plan* p) {
    if (M > kStreamMaxM || N % 32 != 0) return AWQ_ERR_PATH;
    const int64_t strips = gemv_strips((int)N);
    const int64_t groups = K / kGroup;
    int64_t split = cus() / strips;
    if (split > (2 * groups) / 3) split = (2 * groups) / 3;
    if (split < 1) split = 1;
    const int64_t per = (groups + split - 1) / split;
    bool row = M <= 8;
    int64_t kw = row ? 8 : 4;
    int64_t depth = row ? 1 : 2;
    if (M <= 2 && per <= 2) {
        row = false;
        kw = 2;
        depth = 2;
    } else if (M <= 2 || (M >= 5 && row && split > 8)) {
        kw = 4;
        depth = 2;
    }
    const int64_t layout = row ? kStreamRowLayout : kStreamHalfLayout;
    while (split < groups && (!stream_fits((int)M, (int)K, (int)split, (int)kw, (int)layout) ||
                              stream_lds_bytes((int)M, (int)K, (int)split, (int)kw, (int)layout) > kStreamLdsBudget))
        ++split;
    int64_t variant = 1;
    if (split > 1 && M > 4) variant = M * split <= 32 ? 2 : 3;
    if (variant == 1 && split > 1 && (split > kFixMaxSplit || (uint64_t)M * (uint64_t)N * 8u > kSlotBytes))
        variant = M * split <= 32 ? 2 : 3;
    if (M > 8 && split > 1) {
        // Half layout (9 <= M <= 16), measured on 3584 x 37888 (split 3) and
        // 18944 x 3584 (split 36) at M = 9, 12, 16: fewer wave pairs per
        // workgroup -- two for a few splits, three for many -- and the reduce
        // launch as the finish, 0.7 - 1.4 us faster than four pairs.
        const int64_t kw_half = split <= 8 ? 2 : 3;
        if (stream_fits((int)M, (int)K, (int)split, (int)kw_half, (int)layout) &&
            stream_lds_bytes((int)M, (int)K, (int)split, (int)kw_half, (int)layout) <= kStreamLdsBudget &&
            fill_stream(M, N, K, layout, 3, kw_half, split, depth, p) == AWQ_OK)
            return AWQ_OK;
    }
    return fill_stream(M, N, K, layout, variant, kw, split, depth, p);
}

// AUTO between the stream path and skinny for 2 <= M <= 16 (measured on the
// Qwen2-7B shapes): the stream path for M <= 4 on every shape; above, where
// the weight is wide (at least 16 strips of 512 columns) or deep (K >= 8192),
// whose splits keep the partial sums small against the weight stream.
bool auto_stream(int64_t M, int64_t N, int64_t K) {
    if (M > kStreamMaxM || N % 32 != 0) return false;
    if (M <= 4) return true;
    return gemv_strips((int)N) >= 16 || K >= 8192;
}

int fill_tile(int64_t M, int64_t N, int64_t K, int64_t variant, int64_t split_k, awq_w4a16_plan* p) {
    p->path = AWQ_PATH_TILE;
    p->variant = (int32_t)variant;
    p->tile_m = 128;
    p->tile_n = 128;
    p->rows_per_wave = 0;
    p->k_waves = 1;
    p->block_threads = 256;
    p->factored_scale = 0;
    p->depth = 0;
    p->lds_bytes = 0;
    if (!tile_variant_served((int)variant) || split_k < 1) return AWQ_ERR_PATH;
    p->tile_m = tile5_rows((int)variant);
    p->tile_n = tile5_cols((int)variant);
    p->block_threads = tile5_threads((int)variant);
    const int64_t tiles = tile_tiles((int)M, (int)N, (int)variant);
    // K range per split: whole 128-row groups (two 64-row k-steps).
    const int64_t unit = kGroup;
    const int64_t steps = K / unit;
    const int64_t per = (steps + split_k - 1) / split_k;
    const int64_t s = (steps + per - 1) / per;
    if (s != split_k) return AWQ_ERR_PATH;
    if (split_k > 1 && tiles * 4 > (int64_t)kCounterBytes) return AWQ_ERR_PATH;
    p->split_k = (int32_t)split_k;
    p->rows_per_wave = (int32_t)(per * unit);  // K rows per split
    p->grid = tiles * split_k;
    // Variant 6 (last-arriver finish): partials [split, M, N]; 7, 8, 9, 15
    // (reduce launch): fragment-native units of 16 rows x 256 columns.
    p->workspace_bytes = split_k <= 1 ? 0u
                         : variant == 6 ? partials_workspace(split_k, M, N)
                                        : kPartialsOffset + tile_partials_bytes(split_k, M, N);
    if (tile_hybrid((int)variant)) {
        // Whole tiles: `full` per CU on every CU (fewer than the workgroups a
        // CU holds: 2 for 128 rows, 3 for 64); the L leftover tiles split
        // split_k ways, at most one piece per CU; compact partials.
        const int64_t C = cus();
        const int64_t per_cu = variant == 13 ? 2 : 3;
        const int64_t full = tiles / C;
        const int64_t L = tiles - full * C;
        if (split_k < 2 || full < 1 || full > per_cu - 1 || L < 1 || L * split_k > C) return AWQ_ERR_PATH;
        p->grid = full * C + L * split_k;
        p->workspace_bytes = kPartialsOffset + (uint64_t)split_k * (uint64_t)L * (uint64_t)p->tile_m * 256u * 4u;
    }
    if (p->workspace_bytes > (uint64_t)kBytesLimit) return AWQ_ERR_TOO_LARGE;
    return AWQ_OK;
}

// Register-dequant tile variants (tile rows, workgroups per CU, a lone
// workgroup's time per k-step in microseconds, slowdown per further
// workgroup on the CU, finish: 1 reduce launch / 0 last arriver).  Only the
// one-wave-per-SIMD tiles with the reduce finish: variant 7 computes exactly
// what variant 6 does and measured 1 - 5 % faster at every split (split 1
// included), and the k-half pair tiles (10 - 12) were slower than these on
// every measured shape.
struct TileModel {
    int variant, rows, per_cu;
    double t1, eta;
    int reduce;
};
constexpr TileModel kTileModels[] = {
    {7, 128, 2, 0.920, 0.243, 1},
    {8, 64, 3, 0.896, 0.073, 1},
    {9, 32, 4, 0.768, 0.219, 1},
};

// 9 <= M <= 16 on deep, narrow weights (K >= 8192, fewer than 16 strips of
// 512 columns): the 32-row tile (variant 9) with five 128-row groups per
// split, where that grid covers every CU and fits two workgroups per CU;
// else AWQ_ERR_PATH.
// 18944 x 3584 (down_proj): 16.9 / 17.4 / 17.6 us at M = 9 / 12 / 16
// against 17.2 / 17.9 / 18.8 for the half-strip stream kernel with its
// reduce launch; at M = 5 - 8 the stream row kernel stays ahead (16.2 - 16.6
// against 16.6 - 16.8).  Other splits of the same tile measured slower at
// every M (17 splits 18.3 - 18.9, 25 splits 18.4 - 19.1, 37 splits 18.6 -
// 20.0).
// 9 <= M <= 16 on deep, narrow weights (K >= 8192; 2048 <= N < 8192, as
// auto_pairs): column singles with all 16 rows of x (GEMV variant 6, fp32
// partials added by the reduce launch), eight waves, one split fewer than
// fills the CUs.  down_proj (18944 x 3584) at M = 9 / 12 / 16 measured 16.6
// / 16.9 / 17.2 us against 17.2 / 17.7 / 18.2 for the 32-row tile below;
// 8 splits (224 workgroups) 0.3 - 0.5 us faster than 9 (252) at M = 12 - 16,
// as the partials the reduce launch reads shrink with the split.
int deep_small_m_gemv_plan(int64_t M, int64_t N, int64_t K, awq_w4a16_plan* p) {
    if (M < 9 || M > 16 || K < 8192 || N % 32 != 0 || !auto_pairs(1, N, K)) return AWQ_ERR_PATH;
    const int64_t split = cus() / gemv_strips_cw((int)N, 1) - 1;
    awq_w4a16_plan q;
    if (split < 2 || fill_gemv(M, N, K, 6, 128, 0, 8, split, 2, &q) != AWQ_OK) return AWQ_ERR_PATH;
    *p = q;
    return AWQ_OK;
}

int deep_small_m_tile_plan(int64_t M, int64_t N, int64_t K, awq_w4a16_plan* p) {
    if (M < 9 || M > 16 || K < 8192 || gemv_strips((int)N) >= 16) return AWQ_ERR_PATH;
    const int64_t groups = K / kGroup;
    const int64_t split = (groups + 4) / 5;
    awq_w4a16_plan q;
    if (fill_tile(M, N, K, 9, split, &q) != AWQ_OK || q.grid < cus() || q.grid > 2 * cus()) return AWQ_ERR_PATH;
    *p = q;
    return AWQ_OK;
}

// 5 <= M <= 16 on weights the stream path does not take (narrow and
// shallow: fewer than 16 strips of 512 columns, K < 8192): the 32-row
// register-dequant tile (variant 9) split 14 ways along K (in whole 128-row
// units) measured 1.0 - 3.3 us faster than the skinny kernel on 3584 x 4608
// and 3584 x 3584 (qkv and o of Qwen2-7B), and faster than 28 or 7 splits.
// Only where that grid covers at least half the CUs; else AWQ_ERR_PATH.
int small_m_tile_plan(int64_t M, int64_t N, int64_t K, awq_w4a16_plan* p) {
    if (M < 5 || M > 16) return AWQ_ERR_PATH;
    const int64_t units = K / kGroup;
    int64_t split = 14;
    if (split > units) split = units;
    const int64_t per = (units + split - 1) / split;
    split = (units + per - 1) / per;
    awq_w4a16_plan q;
    if (fill_tile(M, N, K, 9, split, &q) != AWQ_OK || q.grid * 2 < cus()) return AWQ_ERR_PATH;
    *p = q;
    return AWQ_OK;
}

// Predicted time (microseconds) of a tile plan, priced for the CU that
// holds the most workgroups: the grid runs in rounds of per_cu x CUs
// workgroup slots, every full round puts per_cu workgroups on each CU, the
// last one ceil(rest / CUs) on the busiest; a round costs steps x t1 x
// (1 + eta (c - 1)) for a CU holding c workgroups (a workgroup alone takes
// t1 per k-step: its waves expose their own latency); a fixed launch,
// prologue and epilogue cost; the reduce launch moves split x M x N x 8
// bytes (partials written, read, cleared).  Constants fitted so that the
// model's choice is fast, not its absolute times: over 3800 timings of
// variants 6 - 14 x 1 - 28 splits on the four Qwen2-7B GEMMs at M = 24 ..
// 4096 (MI355X, random operands) its picks are on average 1.3 % (at worst
// 10 %) slower than the best measured configuration.
double tile_cost_busiest(const TileModel& t, int64_t M, int64_t N, int64_t K, int64_t split) {
    const int64_t wg = tile_tiles((int)M, (int)N, t.variant) * split;
    const int64_t slots = (int64_t)t.per_cu * cus();
    const int64_t steps = 2 * ((K / kGroup + split - 1) / split);
    const int64_t full = wg / slots, rest = wg % slots;
    const int64_t c_last = (rest + cus() - 1) / cus();
    double time = 8.94 + (double)full * (double)steps * t.t1 * (1.0 + t.eta * (double)(t.per_cu - 1));
    if (rest > 0) time += (double)steps * t.t1 * (1.0 + t.eta * (double)(c_last - 1));
    if (split > 1) time += 0.14 + (double)split * (double)M * (double)N * 8.0 / 3.31e6;
    return time;
}

// Busiest-CU time of a hybrid plan (variants 13, 14 with the constants of
// variants 7, 8): `full` whole tiles on every CU, and on L x split CUs one
// piece of a leftover tile (ceil(groups / split) groups) beside them, whose
// partials (split x L x rows x 256 x 4 bytes) are added by the pieces' last
// arrivers while the whole tiles still run.
double tile_cost_hybrid(const TileModel& t, int64_t M, int64_t N, int64_t K, int64_t split) {
    const int64_t tiles = tile_tiles((int)M, (int)N, t.variant);
    const int64_t full = tiles / cus();
    const int64_t left = tiles - full * cus();
    const int64_t groups = K / kGroup;
    const int64_t steps = 2 * groups;
    const int64_t sk_steps = 2 * ((groups + split - 1) / split);
    return 7.54 + (double)sk_steps * t.t1 * (1.0 + t.eta * (double)full) +
           (double)(steps - sk_steps) * t.t1 * (1.0 + t.eta * (double)(full - 1)) +
           (double)split * (double)left * (double)t.rows * 256.0 * 4.0 / 4.56e6;
}

const TileModel* tile_model(int variant) {
    for (const TileModel& t : kTileModels)
        if (t.variant == variant) return &t;
    return nullptr;
}

// The tile plan of least busiest-CU time over variants 7, 8, 9 and 1 - 32
// splits (a split grid at most two workgroups per CU).  Where that choice is
// unsplit and M >= 512, the hybrid of least predicted time instead: an
// unsplit grid leaves CUs idle or some CUs a whole tile more than others.
int tile_plan(int64_t M, int64_t N, int64_t K, awq_w4a16_plan* p) {
    const int64_t groups = K / kGroup;
    // Deep weights (K >= 8192) at M >= 512: the eight-wave 512-column tile
    // (variant 15) at the largest split whose grid fits one workgroup per CU,
    // where one does.  down_proj 18944 x 3584, A/B in one process against the
    // 256-column tiles' AUTO plans (us): M = 512 80.7 (split 8) against 82.4;
    // M = 1024 137.6 (split 4) against 149.1 (139.8 at that tile's best
    // split); M = 1536 195.0 (split 3) against 195.2; M = 2048 255.6 (split 2)
    // against 266.6; M = 4096 470.7 (split 1) against 490.5.  Splits that
    // put a second workgroup on some CUs were slower (M = 2048 split 3 331.6,
    // M = 4096 split 2 521.3), and at K = 3584 the 512-column tile lost to the
    // 256-column one (o at M = 2048 66.7 against 59.1 us; gate||up even).
    // Every measured grid covered at least 7/8 of the CUs (224 - 252 of 256);
    // where that split leaves more CUs idle the cost model below decides.
    if (K >= 8192 && M >= 512) {
        for (int64_t sp = groups < 32 ? groups : 32; sp >= 1; --sp) {
            awq_w4a16_plan q;
            if (fill_tile(M, N, K, 15, sp, &q) == AWQ_OK && q.grid <= (int64_t)cus()) {
                if (q.grid * 8 >= (int64_t)cus() * 7) {
                    *p = q;
                    return AWQ_OK;
                }
                break;
            }
        }
    }
    // Deep weights (K >= 8192) up to M = 1024: a split grid with more than
    // one workgroup per CU measured slower than the model predicts (the second
    // workgroup of a CU competes for its load bandwidth through a short run
    // while the partials grow).  down_proj 18944 x 3584 at M = 24 .. 1024, tiles
    // of 128, 64 and 32 rows x splits 1 .. 30: the best plan fits one workgroup
    // per CU at every M (M = 64: 23.5 us at split 17 against 30.5 at split 25;
    // M = 512: 80.2 us at split 4 against 83.2 at split 9; M = 1024: 147.6 us
    // at split 2 against 150.2 at split 4).  At M = 2048 split 2 on 448
    // workgroups is best (256.1 us against 270.1 unsplit), hence the bound.
    const bool one_per_cu = K >= 8192 && M <= 1024;
    double best = 0.0;
    int64_t best_v = 0, best_s = 0;
    for (const TileModel& t : kTileModels) {
        // On deep weights the 32-row tile measured slower than the model
        // predicts above 32 rows (and was the best plan at 24 and 32).
        if (t.variant == 9 && M > 32 && K >= 8192) continue;
        for (int64_t sp = 1; sp <= groups && sp <= 32; ++sp) {
            awq_w4a16_plan q;
            if (fill_tile(M, N, K, t.variant, sp, &q) != AWQ_OK) continue;
            if (sp > 1 && q.grid > 2 * (int64_t)cus()) continue;
            if (one_per_cu && sp > 1 && q.grid > (int64_t)cus()) continue;
            const double time = tile_cost_busiest(t, M, N, K, sp);
            if (best_v == 0 || time < best) {
                best = time;
                best_v = t.variant;
                best_s = sp;
            }
        }
    }
    if (best_v != 0 && best_s == 1 && M >= 512) {
        double hbest = 0.0;
        int64_t hv = 0, hs = 0;
        // The 64-row hybrid only where the 128-row one has no whole tile per
        // CU: with its finish by helpers (the whole-tile workgroups add the
        // leftover tiles' partials after their own tiles) the 128-row hybrid
        // measured ahead wherever both apply (3584 x 4608 at M = 2048: 69.9 us
        // at split 3 against 72.6 - 80.3 for the 64-row one at splits 2 - 4).
        const bool v13_whole = tile_tiles((int)M, (int)N, 7) >= cus();
        for (int64_t v = 13; v <= 14; ++v) {
            if (v == 14 && v13_whole) continue;
            const TileModel* t = tile_model(v == 13 ? 7 : 8);
            for (int64_t sp = 2; sp <= 8; ++sp) {
                awq_w4a16_plan q;
                if (t == nullptr || fill_tile(M, N, K, v, sp, &q) != AWQ_OK) continue;
                const double time = tile_cost_hybrid(*t, M, N, K, sp);
                if (hv == 0 || time < hbest) {
                    hbest = time;
                    hv = v;
                    hs = sp;
                }
            }
        }
        if (hv != 0 && fill_tile(M, N, K, hv, hs, p) == AWQ_OK) return AWQ_OK;
    }
    if (best_v != 0 && fill_tile(M, N, K, best_v, best_s, p) == AWQ_OK) return AWQ_OK;
    return fill_tile(M, N, K, 7, 1, p);
}

// Checks a caller-supplied plan against the shape: it must be exactly what
// the planner derives from its tuning values.
int check_plan(int64_t M, int64_t N, int64_t K, const awq_w4a16_plan* p) {
    awq_w4a16_plan q;
    if (p->path == AWQ_PATH_SKINNY) {
        const int st = fill_skinny(M, N, K, p->rows_per_wave, p->k_waves, p->variant, p->factored_scale, &q);
        if (st != AWQ_OK) return st;
    } else if (p->path == AWQ_PATH_TILE) {
        const int st = fill_tile(M, N, K, p->variant, p->split_k, &q);
        if (st != AWQ_OK) return st;
    } else if (p->path == AWQ_PATH_STREAM) {
        const int st = fill_stream(M, N, K, p->rows_per_wave, p->variant, p->k_waves, p->split_k, p->depth, &q);
        if (st != AWQ_OK) return st;
    } else if (p->path == AWQ_PATH_GEMV) {
        const int st = fill_gemv(M, N, K, p->variant, p->tile_n, p->rows_per_wave, p->k_waves, p->split_k,
                                 p->depth, &q);
        if (st != AWQ_OK) return st;
    } else {
        return AWQ_ERR_PATH;
    }
    if (p->tile_m != q.tile_m || p->tile_n != q.tile_n || p->split_k != q.split_k || p->depth != q.depth ||
        p->block_threads != q.block_threads || p->grid != q.grid ||
        p->workspace_bytes != q.workspace_bytes || p->lds_bytes != q.lds_bytes)
        return AWQ_ERR_PATH;
    return AWQ_OK;
}

int check_pointers(const void* x, const void* qweight, const void* qzeros, const void* scales,
                   const void* out, int64_t M) {
    if (!qweight || !qzeros || !scales) return AWQ_ERR_NULL_POINTER;
    if (M > 0 && (!x || !out)) return AWQ_ERR_NULL_POINTER;
    if (!aligned(qweight, 4) || !aligned(qzeros, 4) || !aligned(scales, 16)) return AWQ_ERR_MISALIGNED;
    if (M > 0 && (!aligned(x, 16) || !aligned(out, 16))) return AWQ_ERR_MISALIGNED;
    return AWQ_OK;
}

int run_plan(const void* x, const int32_t* qweight, const int32_t* qzeros, const void* scales,
             void* out, int64_t M, int64_t N, int64_t K, void* workspace, const awq_w4a16_plan& p,
             void* stream, const void* bias = nullptr, const void* residual = nullptr) {
    if (M == 0) return AWQ_OK;
    GemmArgs a;
    a.bias = static_cast<const half_t*>(bias);
    a.residual = static_cast<const half_t*>(residual);
    a.x = static_cast<const half_t*>(x);
    a.qweight = reinterpret_cast<const uint32_t*>(qweight);
    a.qzeros = reinterpret_cast<const uint32_t*>(qzeros);
    a.scales = static_cast<const half_t*>(scales);
    a.out = static_cast<half_t*>(out);
    a.partials = nullptr;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e;
    if (p.path == AWQ_PATH_SKINNY) {
        SkinnyConfig cfg;
        cfg.m_blocks = p.tile_m / 16;
        cfg.rows_per_wave = p.rows_per_wave;
        cfg.kw_count = p.k_waves;
        cfg.split_k = p.split_k;
        cfg.variant = p.variant;
        cfg.factored = p.factored_scale != 0;
        uint32_t* counters = static_cast<uint32_t*>(workspace);
        a.partials = p.split_k > 1 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + kPartialsOffset)
                                   : nullptr;
        e = launch_skinny(a, cfg, counters, s);
    } else if (p.path == AWQ_PATH_STREAM) {
        a.partials = p.variant >= 2 && p.split_k > 1
                         ? reinterpret_cast<float*>(static_cast<char*>(workspace) + kPartialsOffset)
                         : nullptr;
        e = launch_stream(a, p.split_k, p.k_waves, p.depth, p.rows_per_wave, p.variant - 1,
                          static_cast<uint32_t*>(workspace), s);
    } else if (p.path == AWQ_PATH_GEMV) {
        GemvConfig cfg;
        cfg.variant = p.variant;
        cfg.rows_per_wave = p.rows_per_wave;
        cfg.kw_count = p.k_waves;
        cfg.split_k = p.split_k;
        const int64_t groups = K / kGroup;
        cfg.chunks_per_split = (int)((groups + p.split_k - 1) / p.split_k);
        cfg.depth = p.depth;
        cfg.cw = p.tile_n / 128;
        a.partials = p.split_k > 1 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + kPartialsOffset)
                                   : nullptr;
        e = launch_gemv(a, cfg, static_cast<uint32_t*>(workspace), s);
    } else {
        TileConfig cfg;
        cfg.variant = p.variant;
        cfg.tile_m = p.tile_m;
        cfg.tile_n = p.tile_n;
        cfg.split_k = p.split_k;
        cfg.k_per_split = p.rows_per_wave;
        cfg.grid = p.grid;
        a.partials = p.split_k > 1 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + kPartialsOffset)
                                   : nullptr;
        e = launch_tile(a, cfg, static_cast<uint32_t*>(workspace), s);
    }
    return e == hipSuccess ? AWQ_OK : AWQ_ERR_LAUNCH;
}

// ---- the allocation-free entry point (awq_w4a16_gemm_noalloc) ---------------
//
// Its split-K workspace is `scratch`, a file-scope device array of
// AWQ_NOALLOC_SCRATCH_BYTES: the code object loader gives every GPU the
// library runs on its own copy, at its own address, held until the process
// ends.  In host code the array's name is only a stand-in for the symbol:
// set-up asks the runtime for this device's address (hipGetSymbolAddress,
// with the device current) and the launches use that pointer.  The scratch
// follows the workspace contract of the other entry points (counters and
// fixed-point slots zero between calls and left zero by every call, the
// partials region rewritten by each call that reads it); set-up clears it
// once per device.  Every
// call on a device shares its scratch, so calls that overlap on one GPU race.
constexpr size_t kScratchBytes = (size_t)AWQ_NOALLOC_SCRATCH_BYTES;

__global__ void awq_zero_fill_kernel(u32x4* p, size_t n16) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) p[i] = u32x4{0u, 0u, 0u, 0u};
}

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device, once set up

// This device's scratch address; the first call on a device looks it up and
// clears the counter and slot regions with a fill kernel on the caller's
// stream (see the definition below).
int device_scratch(hipStream_t stream, void** ptr_out);

// The AUTO plan, with the tile path's split-K count lowered until its
// workspace fits the scratch (split 1 needs none); AWQ_ERR_SCRATCH if a
// plan of another path needs more.
int noalloc_plan(int64_t M, int64_t N, int64_t K, int32_t group_size, awq_w4a16_plan* p) {
    const int st = awq_w4a16_plan_for(M, N, K, group_size, AWQ_PATH_AUTO, p);
    if (st != AWQ_OK || p->workspace_bytes <= kScratchBytes) return st;
    if (p->path != AWQ_PATH_TILE) return AWQ_ERR_SCRATCH;
    // Fewer splits shrink the 512-column tile's grid below the CU count it
    // was chosen for; the 256-column tile (variant 7) at the same split needs
    // the same workspace and has twice the workgroups.
    const int64_t v = p->variant == 15 ? 7 : p->variant;
    for (int64_t sp = p->split_k - 1; sp >= 1; --sp) {
        awq_w4a16_plan q;
        if (fill_tile(M, N, K, v, sp, &q) == AWQ_OK && q.workspace_bytes <= kScratchBytes) {
            *p = q;
            return AWQ_OK;
        }
    }
    // A hybrid needs two splits at least; its unsplit tile needs no workspace.
    awq_w4a16_plan q;
    if (tile_hybrid(p->variant) && fill_tile(M, N, K, p->variant == 13 ? 7 : 8, 1, &q) == AWQ_OK) {
        *p = q;
        return AWQ_OK;
    }
    return AWQ_ERR_SCRATCH;
}

}  // namespace

// File scope, outside the anonymous namespace: the symbol the loader places.
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
// Set-up on the stream's device (the current device for the null stream):
// look up the device's copy of `scratch` with that device current, clear the
// regions that must start at zero -- the arrival counters and the
// fixed-point slots, the first kPartialsOffset bytes (every call writes the
// partials it reads before reading them, so the rest needs no clearing) --
// and wait for the clear, so that a later call on any stream finds them
// zero.  Refused while the stream is being captured (AWQ_ERR_CAPTURE): the
// fill kernel would become a node of the caller's graph and the wait is not
// allowed there; one eager call per device must come first.
int device_scratch(hipStream_t stream, void** ptr_out) {
    int dev = -1;
    if (stream != nullptr) {
        if (hipStreamGetDevice(stream, &dev) != hipSuccess) return AWQ_ERR_LAUNCH;
    } else if (hipGetDevice(&dev) != hipSuccess) {
        return AWQ_ERR_LAUNCH;
    }
    if (dev < 0 || dev >= kMaxDevices) return AWQ_ERR_LAUNCH;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cap) != hipSuccess) return AWQ_ERR_LAUNCH;
        if (cap != hipStreamCaptureStatusNone) return AWQ_ERR_CAPTURE;
        int prev = -1;
        if (hipGetDevice(&prev) != hipSuccess) return AWQ_ERR_LAUNCH;
        if (prev != dev && hipSetDevice(dev) != hipSuccess) return AWQ_ERR_LAUNCH;
        void* ptr = nullptr;
        const bool found = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) == hipSuccess && ptr != nullptr;
        int st = found ? AWQ_OK : AWQ_ERR_LAUNCH;
        if (found) {
            hipLaunchKernelGGL(awq_zero_fill_kernel, dim3(64), dim3(256), 0, stream, static_cast<u32x4*>(ptr),
                               kPartialsOffset / 16);
            if (hipGetLastError() != hipSuccess || hipStreamSynchronize(stream) != hipSuccess) st = AWQ_ERR_LAUNCH;
        }
        if (prev != dev && hipSetDevice(prev) != hipSuccess) st = AWQ_ERR_LAUNCH;
        if (st != AWQ_OK) return st;
        g_scratch_ptr[dev] = ptr;
    }
    *ptr_out = g_scratch_ptr[dev];
    return AWQ_OK;
}
}  // namespace

extern "C" {

int awq_w4a16_abi_version(void) { return AWQ_W4A16_ABI_VERSION; }

const char* awq_w4a16_error_string(int status) {
    switch (status) {
        case AWQ_OK: return "ok";
        case AWQ_ERR_NULL_POINTER: return "a required pointer is NULL";
        case AWQ_ERR_BAD_DIMS: return "bad dimensions: need M >= 0, N > 0, K > 0, N % 8 == 0, K % group_size == 0";
        case AWQ_ERR_GROUP_SIZE: return "unsupported group size (only 128 is served)";
        case AWQ_ERR_MISALIGNED: return "misaligned pointer: x, out, scales need 16-byte, qweight/qzeros 4-byte alignment";
        case AWQ_ERR_WORKSPACE: return "workspace missing or too small";
        case AWQ_ERR_LAUNCH: return "HIP kernel launch failed";
        case AWQ_ERR_PATH: return "kernel path or plan cannot serve this shape";
        case AWQ_ERR_TOO_LARGE: return "M exceeds 2^30, K exceeds 2^22, N exceeds 2^20, or an operand exceeds 2^31-1 bytes";
        case AWQ_ERR_SCRATCH:
            return "the shape's split-K workspace exceeds the allocation-free entry point's static scratch "
                   "(AWQ_NOALLOC_SCRATCH_BYTES); call awq_w4a16_gemm with a workspace instead";
        case AWQ_ERR_CAPTURE:
            return "the allocation-free entry point's first split-K call on a device was made under graph "
                   "capture; make one call outside capture on that device first (it clears the scratch)";
        default: return "unknown status";
    }
}

int awq_w4a16_plan_skinny(int64_t M, int64_t N, int64_t K, int32_t group_size, int32_t rows_per_wave,
                          int32_t k_waves, int32_t variant, int32_t factored_scale, awq_w4a16_plan* plan) {
    if (!plan) return AWQ_ERR_NULL_POINTER;
    const int d = check_dims(M, N, K, group_size);
    if (d != AWQ_OK) return d;
    return fill_skinny(M, N, K, rows_per_wave, k_waves, variant, factored_scale, plan);
}

size_t awq_w4a16_counter_bytes(void) { return skinny_counter_bytes(); }

int awq_w4a16_plan_tile(int64_t M, int64_t N, int64_t K, int32_t group_size, int32_t variant, int32_t split_k,
                        awq_w4a16_plan* plan) {
    if (!plan) return AWQ_ERR_NULL_POINTER;
    const int d = check_dims(M, N, K, group_size);
    if (d != AWQ_OK) return d;
    return fill_tile(M, N, K, variant, split_k, plan);
}

int awq_w4a16_plan_gemv(int64_t M, int64_t N, int64_t K, int32_t group_size, int32_t variant, int32_t tile_n,
                        int32_t rows_per_wave, int32_t k_waves, int32_t split_k, int32_t depth,
                        awq_w4a16_plan* plan) {
    if (!plan) return AWQ_ERR_NULL_POINTER;
    const int d = check_dims(M, N, K, group_size);
    if (d != AWQ_OK) return d;
    return fill_gemv(M, N, K, variant, tile_n, rows_per_wave, k_waves, split_k, depth, plan);
}

int awq_w4a16_plan_stream(int64_t M, int64_t N, int64_t K, int32_t group_size, int32_t rows_per_wave,
                          int32_t variant, int32_t k_waves, int32_t split_k, int32_t depth, awq_w4a16_plan* plan) {
    if (!plan) return AWQ_ERR_NULL_POINTER;
    const int d = check_dims(M, N, K, group_size);
    if (d != AWQ_OK) return d;
    return fill_stream(M, N, K, rows_per_wave, variant, k_waves, split_k, depth, plan);
}

int awq_w4a16_plan_for(int64_t M, int64_t N, int64_t K, int32_t group_size, int32_t path,
                       awq_w4a16_plan* plan) {
    if (!plan) return AWQ_ERR_NULL_POINTER;
    const int d = check_dims(M, N, K, group_size);
    if (d != AWQ_OK) return d;
    switch (path) {
        case AWQ_PATH_AUTO:
            if (auto_pairs(M, N, K) && pair_plan(M, N, K, plan) == AWQ_OK) return AWQ_OK;
            if (strip_class_plan(M, N, K, plan) == AWQ_OK) return AWQ_OK;
            if (M == 1 || (M <= kGemvMaxM && N % 32 != 0)) return gemv_plan(M, N, K, plan);
            if (deep_small_m_gemv_plan(M, N, K, plan) == AWQ_OK) return AWQ_OK;
            if (deep_small_m_tile_plan(M, N, K, plan) == AWQ_OK) return AWQ_OK;
            if (auto_stream(M, N, K) && stream_plan(M, N, K, plan) == AWQ_OK) return AWQ_OK;
            if (small_m_tile_plan(M, N, K, plan) == AWQ_OK) return AWQ_OK;
            return auto_skinny(M, N) ? skinny_plan(M, N, K, plan) : tile_plan(M, N, K, plan);
        case AWQ_PATH_SKINNY: return skinny_plan(M, N, K, plan);
        case AWQ_PATH_GEMV: return gemv_plan(M, N, K, plan);
        case AWQ_PATH_STREAM: return stream_plan(M, N, K, plan);
        case AWQ_PATH_TILE: return tile_plan(M, N, K, plan);
        default: return AWQ_ERR_PATH;
    }
}

size_t awq_w4a16_workspace_bytes_ex(int64_t M, int64_t N, int64_t K, int32_t group_size, int32_t path) {
    awq_w4a16_plan p;
    if (awq_w4a16_plan_for(M, N, K, group_size, path, &p) != AWQ_OK) return 0;
    return (size_t)p.workspace_bytes;
}

size_t awq_w4a16_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t group_size) {
    return awq_w4a16_workspace_bytes_ex(M, N, K, group_size, AWQ_PATH_AUTO);
}

int awq_w4a16_validate(const void* x, const void* qweight, const void* qzeros, const void* scales,
                       const void* out, int64_t M, int64_t N, int64_t K, int32_t group_size,
                       const void* workspace, size_t workspace_bytes, int32_t path) {
    awq_w4a16_plan p;
    int st = awq_w4a16_plan_for(M, N, K, group_size, path, &p);
    if (st != AWQ_OK) return st;
    st = check_pointers(x, qweight, qzeros, scales, out, M);
    if (st != AWQ_OK) return st;
    if (M > 0 && p.workspace_bytes > 0) {
        if (!workspace || workspace_bytes < p.workspace_bytes) return AWQ_ERR_WORKSPACE;
        if (!aligned(workspace, 16)) return AWQ_ERR_MISALIGNED;
    }
    return AWQ_OK;
}

int awq_w4a16_gemm_ex(const void* x, const int32_t* qweight, const int32_t* qzeros, const void* scales,
                      void* out, int64_t M, int64_t N, int64_t K, int32_t group_size, void* workspace,
                      size_t workspace_bytes, int32_t path, void* stream) {
    const int st = awq_w4a16_validate(x, qweight, qzeros, scales, out, M, N, K, group_size, workspace,
                                      workspace_bytes, path);
    if (st != AWQ_OK) return st;
    awq_w4a16_plan p;
    awq_w4a16_plan_for(M, N, K, group_size, path, &p);
    return run_plan(x, qweight, qzeros, scales, out, M, N, K, workspace, p, stream);
}

int awq_w4a16_gemm(const void* x, const int32_t* qweight, const int32_t* qzeros, const void* scales,
                   void* out, int64_t M, int64_t N, int64_t K, int32_t group_size, void* workspace,
                   size_t workspace_bytes, void* stream) {
    return awq_w4a16_gemm_ex(x, qweight, qzeros, scales, out, M, N, K, group_size, workspace,
                             workspace_bytes, AWQ_PATH_AUTO, stream);
}

int awq_w4a16_gemm_planned(const void* x, const int32_t* qweight, const int32_t* qzeros,
                           const void* scales, void* out, int64_t M, int64_t N, int64_t K,
                           int32_t group_size, void* workspace, size_t workspace_bytes,
                           const awq_w4a16_plan* plan, void* stream) {
    if (!plan) return AWQ_ERR_NULL_POINTER;
    int st = check_dims(M, N, K, group_size);
    if (st != AWQ_OK) return st;
    st = check_plan(M, N, K, plan);
    if (st != AWQ_OK) return st;
    st = check_pointers(x, qweight, qzeros, scales, out, M);
    if (st != AWQ_OK) return st;
    if (M > 0 && plan->workspace_bytes > 0) {
        if (!workspace || workspace_bytes < plan->workspace_bytes) return AWQ_ERR_WORKSPACE;
        if (!aligned(workspace, 16)) return AWQ_ERR_MISALIGNED;
    }
    return run_plan(x, qweight, qzeros, scales, out, M, N, K, workspace, *plan, stream);
}

int awq_w4a16_dequant(const int32_t* qweight, const int32_t* qzeros, const void* scales, void* w_out,
                      int64_t N, int64_t K, int32_t group_size, void* stream) {
    int st = check_dims(0, N, K, group_size);
    if (st != AWQ_OK) return st;
    if (!qweight || !qzeros || !scales || !w_out) return AWQ_ERR_NULL_POINTER;
    if (!aligned(qweight, 4) || !aligned(qzeros, 4) || !aligned(scales, 16) || !aligned(w_out, 16))
        return AWQ_ERR_MISALIGNED;
    const hipError_t e = launch_dequant(reinterpret_cast<const uint32_t*>(qweight),
                                        reinterpret_cast<const uint32_t*>(qzeros),
                                        static_cast<const half_t*>(scales), static_cast<half_t*>(w_out),
                                        (int)N, (int)K, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? AWQ_OK : AWQ_ERR_LAUNCH;
}

int awq_w4a16_gemm_epilogue(const void* x, const int32_t* qweight, const int32_t* qzeros, const void* scales,
                            const void* bias, const void* residual, void* out, int64_t M, int64_t N, int64_t K,
                            int32_t group_size, void* workspace, size_t workspace_bytes,
                            const awq_w4a16_plan* plan, void* stream) {
    if (M > 0 && ((bias && !aligned(bias, 2)) || (residual && !aligned(residual, 2)))) return AWQ_ERR_MISALIGNED;
    awq_w4a16_plan p;
    if (plan) {
        int st = check_dims(M, N, K, group_size);
        if (st != AWQ_OK) return st;
        st = check_plan(M, N, K, plan);
        if (st != AWQ_OK) return st;
        st = check_pointers(x, qweight, qzeros, scales, out, M);
        if (st != AWQ_OK) return st;
        if (M > 0 && plan->workspace_bytes > 0) {
            if (!workspace || workspace_bytes < plan->workspace_bytes) return AWQ_ERR_WORKSPACE;
            if (!aligned(workspace, 16)) return AWQ_ERR_MISALIGNED;
        }
        p = *plan;
    } else {
        const int st = awq_w4a16_validate(x, qweight, qzeros, scales, out, M, N, K, group_size, workspace,
                                          workspace_bytes, AWQ_PATH_AUTO);
        if (st != AWQ_OK) return st;
        awq_w4a16_plan_for(M, N, K, group_size, AWQ_PATH_AUTO, &p);
    }
    return run_plan(x, qweight, qzeros, scales, out, M, N, K, workspace, p, stream, bias, residual);
}

int awq_w4a16_gemm_noalloc(const void* x, const int32_t* qweight, const int32_t* qzeros, const void* scales,
                           void* out, int64_t M, int64_t N, int64_t K, int32_t group_size, void* stream) {
    awq_w4a16_plan p;
    int st = noalloc_plan(M, N, K, group_size, &p);
    if (st != AWQ_OK) return st;
    st = check_pointers(x, qweight, qzeros, scales, out, M);
    if (st != AWQ_OK || M == 0) return st;
    void* ws = nullptr;
    if (p.workspace_bytes > 0) {
        st = device_scratch(static_cast<hipStream_t>(stream), &ws);
        if (st != AWQ_OK) return st;
    }
    return run_plan(x, qweight, qzeros, scales, out, M, N, K, ws, p, stream);
}

int awq_silu_mul(const void* gate_up, void* out, int64_t M, int64_t I, void* stream) {
    if (M < 0 || I <= 0 || I % 8 != 0) return AWQ_ERR_BAD_DIMS;
    if (M * 2 * I > kBytesLimit / 2) return AWQ_ERR_TOO_LARGE;
    if (M == 0) return AWQ_OK;
    if (!gate_up || !out) return AWQ_ERR_NULL_POINTER;
    if (!aligned(gate_up, 16) || !aligned(out, 16)) return AWQ_ERR_MISALIGNED;
    const hipError_t e = launch_silu_mul(static_cast<const half_t*>(gate_up), static_cast<half_t*>(out), (int)M,
                                         (int)I, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? AWQ_OK : AWQ_ERR_LAUNCH;
}

int awq_fp16_linear(const void* x, const void* weight, void* out, int64_t M, int64_t N, int64_t K, void* stream) {
    if (M < 0 || N <= 0 || K <= 0 || K % 8 != 0) return AWQ_ERR_BAD_DIMS;
    if (M > kFp16LinearMaxM) return AWQ_ERR_PATH;
    if (K > fp16_gemv_max_k() || N > (int64_t)1 << 30 ||
        (uint64_t)N * (uint64_t)K * 2u >= ((uint64_t)1 << 31))
        return AWQ_ERR_TOO_LARGE;
    if (M == 0) return AWQ_OK;
    if (!x || !weight || !out) return AWQ_ERR_NULL_POINTER;
    if (!aligned(x, 16) || !aligned(weight, 16) || !aligned(out, 2)) return AWQ_ERR_MISALIGNED;
    const hipError_t e = launch_fp16_gemv(static_cast<const half_t*>(x), static_cast<const half_t*>(weight),
                                          static_cast<half_t*>(out), (int)M, (int)N, (int)K, (int)cus(),
                                          static_cast<hipStream_t>(stream));
    return e == hipSuccess ? AWQ_OK : AWQ_ERR_LAUNCH;
}

}  // extern "C"
