// Streaming W4A16 AWQ GEMM for small M (M <= 16) on the MFMA units of gfx950.
//
// A workgroup owns a 512-column strip (64 packed columns, a 256-byte segment
// of every weight row) and a range of whole 128-row groups, split among its
// waves group by group (wave w takes every nw-th group); each wave streams
// its groups chunk by chunk through a ring of R chunk buffers (R - 1 chunks'
// loads in flight while one is computed; loads past the end use an
// out-of-range offset and read zeros, so the compiler's wait counts stay
// static).  Zeros and scales of the workgroup's groups are staged in LDS once
// as fp32 pairs (s, s(b + z)) per column, where b is the offset the
// magic-number unpack gives that column's codes (1024, or 64 for the columns
// kpairs_magic_inplace cuts in place).
//
// Arithmetic (both layouts): v_mfma_f32_16x16x32_f16 with the magic-number
// k-pairs (b + q) of a lane's 8 rows of one column as its B fragment and
// rows of x as A.  Over a group one MFMA per column accumulates
//     C[m][n] = sum_k x[m][k] * (b + q[k][n])
// and one MFMA against ones S[m] = sum_k x[m][k]; at the end of the group
//     acc[m][n] += s[n] * C[m][n] - s(b + z)[n] * S[m]
// in fp32 (one fold per column and row per group).
//
// Row layout (awq_stream_row_kernel, M <= 8): every load instruction covers
// whole 256-byte row segments: lane l (n = l % 16, kb = l / 16) reads packed
// columns 2 (n + 16 (kb & 1)) and +1 (8 bytes) of rows 8 (kb >> 1) + u of a
// 16-row chunk (u = 0 .. 7, one load each).  The MFMA's k-block kb is lane
// kb's 8 rows, and the two column halves (kb & 1) are kept apart in the rows
// of A: A row m holds x row m % 8 in the k-blocks of half m / 8 and zeros in
// the others, so D rows 0..7 are the outputs of half 0 and rows 8..15 those
// of half 1 -- 16 columns x 8 rows per lane and MFMA, no wasted columns.
// Lane (n, kb) holds x rows 4 (kb & 1) + r of half kb >> 1.  The waves of
// a workgroup share every group (wave w reads its own 16-row chunks of it)
// and x comes from LDS.
//
// Half-strip layout (awq_stream_kernel, M <= 16): waves come in pairs, wave
// 2*kw + h reads packed columns 32*h + 2*c4 and +1 (c4 = l % 16) of rows
// 4*rq .. 4*rq+3 (rq = l / 16) of each 16-row half of a 32-row chunk; the
// MFMA's n is c4 and its k-block rq, A is x row c4 (rows >= M read zeros);
// lane (c4, rq) holds rows 4*rq + r of its 16 columns.  Each wave reads only
// half of a row segment, which costs bandwidth, but all 16 rows of x share
// one MFMA.
//
// Split-K finish (FIN): 0 -- fixed-point slots, one 64-bit atomic per output
// element per workgroup (fixed_point_word / finish_batch: deterministic, one
// round trip; direct fp16 store when split_k == 1); 1 -- fp32 partials
// [split, M, N] with device-scope stores and an arrival counter per strip,
// the last workgroup of a strip adds the partials in split order; 2 -- fp32
// partials, also with device-scope (write-through) stores, added by
// awq_splitk_reduce_kernel in a second launch (spreads the additions over
// the whole device when a strip has many splits).
#include "awq_kernels.h"

namespace awq {

namespace {
constexpr int kStreamItemsPerThread = 4;  // prologue constant loads per thread

// Zeros and scales of groups g0 .. g0 + n_g - 1 of a strip: issued first (so
// that they are in flight with the first chunk loads), stored to LDS after.
// LDS layout float4 [n_g][2 halves][8][16]: piece i of lane n of a half holds
// (s, s(b + z)) of the half's columns 16 n + 2 i and + 1 (one
// wave-wide read of a half is 256 consecutive bytes).
struct StagedConsts {
    u32x4 sv[kStreamItemsPerThread];
    uint32_t zv[kStreamItemsPerThread];

    __device__ __forceinline__ void issue(const GemmArgs& a, int strip, int g0, int n_g) {
        const int pn = a.N >> 3;
        const int groups = a.K / kGroup;
        const __amdgpu_buffer_rsrc_t rz = make_rsrc(a.qzeros, (uint32_t)((size_t)groups * pn * 4));
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.scales, (uint32_t)((size_t)groups * a.N * 2));
#pragma unroll
        for (int i = 0; i < kStreamItemsPerThread; ++i) {
            const int item = min((int)threadIdx.x + i * (int)blockDim.x, max(n_g * 64 - 1, 0));
            const int g = min(g0 + item / 64, groups - 1);
            const int j = min(strip * 64 + item % 64, pn - 1);
            zv[i] = buf_load_b32(rz, (uint32_t)(g * pn + j) * 4u, 0u);
            sv[i] = buf_load_u4(rs, (uint32_t)(((size_t)g * a.N + 8 * j) * 2), 0u);
        }
    }
    __device__ __forceinline__ void store(floatx4* lc, int n_g) const {
#pragma unroll
        for (int i = 0; i < kStreamItemsPerThread; ++i) {
            const int item = (int)threadIdx.x + i * (int)blockDim.x;
            if (item < n_g * 64) {
                const int g = item / 64;
                const int j = item % 64;  // packed column of the strip: half j / 32, lane (j % 32) / 2, word j % 2
                const half8_t s8 = __builtin_bit_cast(half8_t, sv[i]);
#pragma unroll
                for (int c = 0; c < 8; c += 2) {
                    floatx4 v;
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const int cc = c + e;
                        const uint32_t z = (zv[i] >> col_shift(cc)) & 0xFu;
                        const float sc = (float)s8[cc];
                        const float zz = magic_base(cc) + (float)z;
                        v[2 * e] = sc;
                        v[2 * e + 1] = sc * zz;
                    }
                    const int col = 8 * (j % 2) + c;  // lane-local column 0..15
                    lc[((g * 2 + j / 32) * 8 + col / 2) * 16 + (j % 32) / 2] = v;
                }
            }
        }
    }
};

// The 16 column MFMAs of one chunk for each of MH blocks of x rows: k-pairs
// of the lane's 8 rows (w[0..7], two packed words each) against A; first:
// start the group's sums.
template <int MH>
__device__ __forceinline__ void chunk_mfma(const u32x2 (&w)[8], const half8_t (&xa)[MH], bool first,
                                           floatx4 (&S)[MH], floatx4 (&Cc)[MH][16]) {
    const uint32_t one2 = 0x3C003C00u;  // fp16 (1, 1)
    const half8_t ones8 = __builtin_bit_cast(half8_t, u32x4{one2, one2, one2, one2});
    const floatx4 zero4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int h = 0; h < MH; ++h) S[h] = mfma16x16x32(xa[h], ones8, first ? zero4 : S[h]);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        uint32_t kp[4][8];
#pragma unroll
        for (int t = 0; t < 4; ++t) kpairs_magic_inplace(w[2 * t][p], w[2 * t + 1][p], kp[t]);
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) {
            const half8_t b = __builtin_bit_cast(half8_t, u32x4{kp[0][cc], kp[1][cc], kp[2][cc], kp[3][cc]});
#pragma unroll
            for (int h = 0; h < MH; ++h) Cc[h][8 * p + cc] = mfma16x16x32(xa[h], b, first ? zero4 : Cc[h][8 * p + cc]);
        }
    }
}

// acc[r][j] += s[j] * C[j][r] - s(b + z)[j] * S[r] with the constants
// of lane n of half `half` of group gi (relative to the workgroup's first).
__device__ __forceinline__ void fold_group(const floatx4* lc, int gi, int half, int n, const floatx4& S,
                                           const floatx4 (&Cc)[16], float (&acc)[4][16]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const floatx4 v = lc[((gi * 2 + half) * 8 + i) * 16 + n];
#pragma unroll
        for (int e = 0; e < 2; ++e)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                acc[r][2 * i + e] =
                    __builtin_fmaf(-v[2 * e + 1], S[r], __builtin_fmaf(v[2 * e], Cc[2 * i + e][r], acc[r][2 * i + e]));
    }
}

// Finish of a strip: red[w][row < MP][512 columns] in LDS holds the sums of
// the workgroup's nred waves (or wave pairs); output = their sum over this
// workgroup's split.  Called by the whole workgroup.
template <int MP, int FIN>
__device__ __forceinline__ void stream_finish(const GemmArgs& a, int split_k, uint32_t* counters, float* red,
                                              int nred, int strip, int split) {
    const int nt = blockDim.x;
    const int mrows = min(a.M, MP);
    const int ncols = min(512, a.N - strip * 512);
    if (FIN != 0 && split_k > 1) {
        // This workgroup's partial: rows < M, columns of the strip, as float4.
        const uint32_t part_bytes = (uint32_t)((size_t)split_k * a.M * a.N * 4);
        const __amdgpu_buffer_rsrc_t rp = make_rsrc(a.partials, part_bytes);
        for (int it = threadIdx.x; it < mrows * 128; it += nt) {
            const int m = it / 128;
            const int q = it % 128;  // column quad of the strip
            if (4 * q >= ncols) continue;
            floatx4 v = {0.f, 0.f, 0.f, 0.f};
            for (int w = 0; w < nred; ++w) v += *reinterpret_cast<const floatx4*>(&red[(w * MP + m) * 512 + 4 * q]);
            const uint32_t off = (uint32_t)((((size_t)split * a.M + m) * a.N + strip * 512 + 4 * q) * 4);
            buf_store_f4_device(v, rp, off);
        }
        if (FIN == 2) return;
        __shared__ int last_flag;
        wait_vm_stores();
        __syncthreads();
        if (threadIdx.x == 0)
            last_flag = __hip_atomic_fetch_add(&counters[strip], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                        (uint32_t)(split_k - 1);
        __syncthreads();
        if (!last_flag) return;
        splitk_finish<2>(rp, a.out, a.bias, a.residual, a.M, a.N, 0, a.M, strip * 512, ncols, split_k, reinterpret_cast<floatx4*>(red));
        if (threadIdx.x == 0) __hip_atomic_store(&counters[strip], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }

    // Fixed-point finish (or the direct store when split_k == 1): every
    // output of the thread in one batch (512 threads: MP outputs each), all
    // atomics in flight together.
    unsigned long long* fix = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(counters) + kCounterBytes);
    const int items = mrows * 512;
    constexpr int BATCH = MP;
    for (int base = threadIdx.x; base < items; base += BATCH * nt) {
        float sum[BATCH];
        int col[BATCH], m[BATCH];
        bool ok[BATCH];
#pragma unroll
        for (int b = 0; b < BATCH; ++b) {
            const int it = base + b * nt;
            m[b] = it / 512;
            col[b] = strip * 512 + it % 512;
            ok[b] = it < items && col[b] < a.N;
            sum[b] = 0.f;
            if (ok[b])
                for (int w = 0; w < nred; ++w) sum[b] += red[(w * MP + m[b]) * 512 + it % 512];
        }
        finish_batch<BATCH>(fix, a.out, a.bias, a.residual, a.M, a.N, split_k, sum, m, col, ok);
    }
}
}  // namespace

// Row layout, M <= 8.  CPG: 16-row chunks of every group per wave (8 /
// waves); R: chunk buffers per wave (1 or 2).  The waves read each group
// together -- wave w its chunks w*CPG .. w*CPG+CPG-1 -- so they all have the
// same work and stream adjacent rows; each folds its part of a group once.
// x rows of the workgroup's K range are staged in LDS with the constants.
template <int FIN, int CPG, int R, bool NT>
__global__ __launch_bounds__(512) void awq_stream_row_kernel(GemmArgs a, int split_k, uint32_t* counters) {
    constexpr int MH = 1;  // blocks of 8 x rows
    constexpr int XI = 4;  // x prologue loads per thread
    extern __shared__ __align__(16) uint32_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nw = blockDim.x >> 6;  // 8 / CPG
    const int nt = blockDim.x;
    const int n = lane & 15;
    const int kb = lane >> 4;
    const int pn = a.N >> 3;
    const int n_strips = (pn + 63) / 64;
    const int strip = blockIdx.x % n_strips;
    const int split = blockIdx.x / n_strips;
    const int groups = a.K / kGroup;
    const int g0 = (int)((int64_t)groups * split / split_k);
    const int g1 = (int)((int64_t)groups * (split + 1) / split_k);
    const int n_g = g1 - g0;

    // Lane's loads: half kb & 1, row slot kb >> 1 (rows 8 (kb >> 1) + u).
    const int jl = min(strip * 64 + 2 * (n + 16 * (kb & 1)), pn - 2);  // in range; lanes past pn drop results
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.qweight, (uint32_t)((size_t)a.K * pn * 4));
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (uint32_t)((size_t)a.M * a.K * 2));
    const uint32_t row_bytes = (uint32_t)pn * 4u;
    const uint32_t voff_w = (uint32_t)(8 * (kb >> 1)) * row_bytes + (uint32_t)jl * 4u;

    // LDS: constants (n_g * 4 KiB), then x [M][n_g * 128] fp16.
    floatx4* lc = reinterpret_cast<floatx4*>(lds);
    half_t* lx = reinterpret_cast<half_t*>(lds + n_g * 1024);
    const int xrow_len = n_g * kGroup;
    StagedConsts consts;
    consts.issue(a, strip, g0, n_g);
    const int x_items = a.M * n_g * 16;  // 16-byte pieces
    u32x4 xv[XI];
#pragma unroll
    for (int i = 0; i < XI; ++i) {
        const int item = (int)threadIdx.x + i * nt;
        const int m = item / max(n_g * 16, 1);
        const int piece = item - m * n_g * 16;
        xv[i] = buf_load_u4(rx, item < x_items ? (uint32_t)((m * a.K + g0 * kGroup + 8 * piece) * 2) : 0x80000000u, 0u);
    }
    auto fence = [] { __builtin_amdgcn_sched_barrier(0); };

    // The wave's chunk k: group t = k / CPG of the range, chunk w*CPG + k%CPG of it.
    const int nk = n_g * CPG;
    auto chunk_row = [&](int k) { return (k / CPG) * kGroup + 16 * (wave * CPG + k % CPG); };  // in the range
    auto load_chunk = [&](int k, u32x2 (&w)[8]) {
        const bool live = k < nk;
        const uint32_t oob = live ? 0u : 0x80000000u;
        const uint32_t r0 = live ? (uint32_t)(g0 * kGroup + chunk_row(k)) : 0u;
#pragma unroll
        for (int u = 0; u < 8; ++u)
            w[u] = __builtin_bit_cast(u32x2,
                                      __builtin_amdgcn_raw_buffer_load_b64(rw, voff_w + oob, (r0 + u) * row_bytes, NT ? kCpolNT : 0));
    };
    u32x2 ring[R][8];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        fence();
        load_chunk(i, ring[i]);
    }
    fence();
    consts.store(lc, n_g);
#pragma unroll
    for (int i = 0; i < XI; ++i) {
        const int item = (int)threadIdx.x + i * nt;
        if (item < x_items) *reinterpret_cast<u32x4*>(lx + 8 * item) = xv[i];
    }
    __syncthreads();

    float acc[MH][4][16];
#pragma unroll
    for (int h = 0; h < MH; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[h][r][i] = 0.f;
    floatx4 S[MH];
    floatx4 Cc[MH][16];
    // A: lane (n, kb) supplies A row n = x row n % 8 (+ 8 h) when n / 8 is its half.
    bool x_live[MH];
    const half_t* lxl[MH];
#pragma unroll
    for (int h = 0; h < MH; ++h) {
        x_live[h] = (n >> 3) == (kb & 1) && (n & 7) + 8 * h < a.M;
        lxl[h] = lx + ((n & 7) + 8 * h) * xrow_len + 8 * (kb >> 1);
    }

    // ring[i % R] holds chunk k + i at the top of each iteration of U chunks
    // (whole parts and ring turns).  With R = 1 a wave computes a chunk only
    // after its loads complete and issues the next chunk's loads after it
    // (the other wave of the SIMD computes meanwhile).
    constexpr int U = CPG > R ? CPG : R;
    for (int k = 0; k < nk; k += U) {
#pragma unroll
        for (int i = 0; i < U; ++i) {
            fence();
            half8_t xa[MH];
#pragma unroll
            for (int h = 0; h < MH; ++h) {
                u32x4 v = {0u, 0u, 0u, 0u};
                if (x_live[h] && k + i < nk) v = *reinterpret_cast<const u32x4*>(lxl[h] + chunk_row(k + i));
                xa[h] = __builtin_bit_cast(half8_t, v);
            }
            chunk_mfma<MH>(ring[i % R], xa, i % CPG == 0, S, Cc);
            fence();
            load_chunk(k + i + R, ring[i % R]);
            fence();
            if (i % CPG == CPG - 1 && k + i < nk) {
#pragma unroll
                for (int h = 0; h < MH; ++h) fold_group(lc, (k + i) / CPG, kb >> 1, n, S[h], Cc[h], acc[h]);
            }
        }
    }

    // Cross-wave sum through LDS: red[w][row < 8 MH][512 columns]; lane
    // (n, kb) holds x rows 8 h + 4 (kb & 1) + r of columns 256 (kb >> 1) +
    // 16 n + j.
    __syncthreads();  // every wave is done with the staged constants and x
    float* red = reinterpret_cast<float*>(lds);
#pragma unroll
    for (int h = 0; h < MH; ++h) {
        if (8 * h + 4 * (kb & 1) < a.M) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int i = 0; i < 16; i += 4)
                    *reinterpret_cast<floatx4*>(
                        &red[(wave * 8 * MH + 8 * h + 4 * (kb & 1) + r) * 512 + 256 * (kb >> 1) + 16 * n + i]) =
                        floatx4{acc[h][r][i], acc[h][r][i + 1], acc[h][r][i + 2], acc[h][r][i + 3]};
        }
    }
    __syncthreads();
    stream_finish<8 * MH, FIN>(a, split_k, counters, red, nw, strip, split);
}

// Half-strip layout, M <= 16.  MP: rows of x covered by the finish (4 or 16,
// >= M); R: chunk buffers per wave (2: two waves per SIMD, up to 512
// threads; 4 or 6: one wave per SIMD, up to 256 threads).
template <int MP, int FIN, int R, bool NT>
__global__ __launch_bounds__(R == 2 ? 512 : 256) void awq_stream_kernel(GemmArgs a, int split_k, uint32_t* counters) {
    extern __shared__ __align__(16) uint32_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = wave & 1;    // half of the strip
    const int kw = wave >> 1;  // K-interleave index of the wave pair
    const int nkw = blockDim.x >> 7;
    const int c4 = lane & 15;
    const int rq = lane >> 4;
    const int pn = a.N >> 3;
    const int n_strips = (pn + 63) / 64;
    const int strip = blockIdx.x % n_strips;
    const int split = blockIdx.x / n_strips;
    const int jl = min(strip * 64 + 32 * h + 2 * c4, pn - 2);  // in-range pair; lanes past pn drop their results
    const int groups = a.K / kGroup;
    const int g0 = (int)((int64_t)groups * split / split_k);
    const int g1 = (int)((int64_t)groups * (split + 1) / split_k);
    const int n_g = g1 - g0;

    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.qweight, (uint32_t)((size_t)a.K * pn * 4));
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (uint32_t)((size_t)a.M * a.K * 2));
    const uint32_t row_bytes = (uint32_t)pn * 4u;
    const uint32_t voff_w = (uint32_t)(4 * rq) * row_bytes + (uint32_t)jl * 4u;
    const uint32_t voff_x = (uint32_t)((c4 * a.K + 4 * rq) * 2);  // row c4 of x; rows >= M read 0

    floatx4* lc = reinterpret_cast<floatx4*>(lds);
    StagedConsts consts;
    consts.issue(a, strip, g0, n_g);
    auto fence = [] { __builtin_amdgcn_sched_barrier(0); };

    struct Chunk {
        u32x2 w[8];
        u32x2 xa[2];
    };
    // The pair's chunk k: group g0 + kw + (k / 4) * nkw, rows 32 * (k % 4) of it.
    const int nk = kw < n_g ? 4 * ((n_g - kw + nkw - 1) / nkw) : 0;
    auto load_chunk = [&](int k, Chunk& ck) {
        const bool live = k < nk;
        const uint32_t oob = live ? 0u : 0x80000000u;
        const uint32_t r0 = live ? (uint32_t)((g0 + kw + (k >> 2) * nkw) * kGroup + (k & 3) * 32) : 0u;
#pragma unroll
        for (int u = 0; u < 8; ++u)
            ck.w[u] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(
                                                    rw, voff_w + oob, (r0 + (u & 3) + 16 * (u >> 2)) * row_bytes, NT ? kCpolNT : 0));
#pragma unroll
        for (int t = 0; t < 2; ++t)
            ck.xa[t] = __builtin_bit_cast(u32x2,
                                          __builtin_amdgcn_raw_buffer_load_b64(rx, voff_x + oob, (r0 + 16 * t) * 2u, 0));
    };
    Chunk ring[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        fence();
        load_chunk(i, ring[i]);
    }
    fence();
    consts.store(lc, n_g);
    __syncthreads();

    float acc[4][16];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[r][i] = 0.f;
    floatx4 S[1];
    floatx4 Cc[1][16];

    // ring[i % R] holds chunk k + i at the top of each iteration of U chunks
    // (a whole number of groups and of ring turns).  A lane's 8 rows of a
    // chunk, in k order: 4 rq + 0..3 and 16 + 4 rq + 0..3.
    constexpr int U = R == 2 ? 4 : (R == 6 ? 12 : R);
    for (int k = 0; k < nk; k += U) {
#pragma unroll
        for (int i = 0; i < U; ++i) {
            fence();
            const Chunk& ck = ring[i % R];
            const half8_t xa[1] = {
                __builtin_bit_cast(half8_t, u32x4{ck.xa[0][0], ck.xa[0][1], ck.xa[1][0], ck.xa[1][1]})};
            chunk_mfma<1>(ck.w, xa, i % 4 == 0, S, Cc);
            fence();
            load_chunk(k + i + R, ring[i % R]);
            fence();
            if (i % 4 == 3 && k + i < nk) fold_group(lc, kw + ((k + i) >> 2) * nkw, h, c4, S[0], Cc[0], acc);
        }
    }

    // Cross-pair sum through LDS: red[kw][row < MP][512 columns]; lane
    // (c4, rq) of half h holds rows 4*rq + r of columns 256*h + 16*c4 + i.
    __syncthreads();  // every wave is done with the staged constants
    float* red = reinterpret_cast<float*>(lds);
    if (4 * rq < MP) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int i = 0; i < 16; i += 4)
                *reinterpret_cast<floatx4*>(&red[(kw * MP + 4 * rq + r) * 512 + 256 * h + 16 * c4 + i]) =
                    floatx4{acc[r][i], acc[r][i + 1], acc[r][i + 2], acc[r][i + 3]};
    }
    __syncthreads();
    stream_finish<MP, FIN>(a, split_k, counters, red, nkw, strip, split);
}

// Second launch of FIN 2: out[m, n] = fp16(sum over split of partials[split,
// m, n]), each element summed in split order (deterministic).  P threads
// share an output quad (splits part, part + P, ...; at most eight loads each,
// all in flight together) and combine through LDS in part order.  The
// partials are read once and left as they are (the workspace's partials
// region is not kept zero).
__global__ __launch_bounds__(256) void awq_splitk_reduce_kernel(float* __restrict__ partials, half_t* __restrict__ out,
                                                               const half_t* bias, const half_t* residual, int M,
                                                               int N, int split_k, int P) {
    __shared__ floatx4 fin[256];
    const int qpb = 256 / P;  // output quads per workgroup
    const int t = threadIdx.x;
    const int part = t / qpb;
    const int quads = M * N / 4;
    const int q = blockIdx.x * qpb + t % qpb;
    const bool valid = q < quads;
    const size_t stride = (size_t)M * N;
    floatx4 s = {0.f, 0.f, 0.f, 0.f};
    if (valid) {
        floatx4* p = reinterpret_cast<floatx4*>(partials) + q;
        const size_t step = stride / 4;  // one split, in float4
#pragma unroll 8
        for (int sp = part; sp < split_k; sp += P) s += __builtin_nontemporal_load(p + (size_t)sp * step);
    }
    fin[t] = s;
    __syncthreads();
    if (valid && part == 0) {
        for (int i = 1; i < P; ++i) s += fin[i * qpb + t];
        const float y[4] = {s[0], s[1], s[2], s[3]};
        const int m = (int)(((size_t)q * 4) / N);
        store_out<4>(out, bias, residual, N, m, q * 4 - m * N, y);
    }
}

int64_t stream_threads(int layout, int k_waves) { return (layout == kStreamRowLayout ? 64 : 128) * (int64_t)k_waves; }

size_t stream_lds_bytes(int M, int K, int split_k, int k_waves, int layout) {
    const int64_t groups = K / kGroup;
    const int64_t n_g = (groups + split_k - 1) / split_k;
    const bool row = layout == kStreamRowLayout;
    const size_t staged = (size_t)n_g * 4096 + (row ? (size_t)M * n_g * kGroup * 2 : 0);
    const size_t red = (size_t)k_waves * (row ? 8 : (M <= 4 ? 4 : 16)) * 512 * 4;
    return staged > red ? staged : red;
}

bool stream_fits(int M, int K, int split_k, int k_waves, int layout) {
    const int64_t groups = K / kGroup;
    const int64_t n_g = (groups + split_k - 1) / split_k;
    const int64_t items = (int64_t)kStreamItemsPerThread * stream_threads(layout, k_waves);
    return split_k <= groups && n_g * 64 <= items && (layout != kStreamRowLayout || (int64_t)M * n_g * 16 <= items);
}

// Threads per output quad of the reduce launch: enough that each adds at
// most eight splits, and eight from 12 splits up -- measured behind the
// 32-row tile at M = 8 and 16 (14 and 28 splits) 0.5 - 1.25 us faster than
// two or four, with no change at 36 splits (already eight) or at 3 (one).
int stream_reduce_parts(int split_k) {
    int P = 1;
    while (P < 16 && P * 8 < split_k) P *= 2;
    if (split_k >= 12 && P < 8) P = 8;
    return P;
}

int64_t stream_reduce_blocks(int M, int N, int split_k) {
    const int64_t qpb = 256 / stream_reduce_parts(split_k);
    return ((int64_t)M * N / 4 + qpb - 1) / qpb;
}

hipError_t splitk_reduce_launch(const GemmArgs& a, int split_k, hipStream_t stream) {
    const int P = stream_reduce_parts(split_k);
    hipLaunchKernelGGL(awq_splitk_reduce_kernel, dim3((unsigned)stream_reduce_blocks(a.M, a.N, split_k)), dim3(256), 0,
                       stream, a.partials, a.out, a.bias, a.residual, a.M, a.N, split_k, P);
    return hipGetLastError();
}

namespace {
hipError_t reduce_launch(const GemmArgs& a, int split_k, hipStream_t stream) { return splitk_reduce_launch(a, split_k, stream); }

template <int MP, int FIN, int R>
hipError_t half_launch(const GemmArgs& a, int split_k, int k_waves, uint32_t* counters, hipStream_t stream) {
    const size_t lds = stream_lds_bytes(a.M, a.K, split_k, k_waves, kStreamHalfLayout);
    const dim3 grid((unsigned)(gemv_strips(a.N) * split_k)), block((unsigned)stream_threads(kStreamHalfLayout, k_waves));
    if (split_k <= kNonTemporalMaxSplit)
        hipLaunchKernelGGL((awq_stream_kernel<MP, FIN, R, true>), grid, block, lds, stream, a, split_k, counters);
    else
        hipLaunchKernelGGL((awq_stream_kernel<MP, FIN, R, false>), grid, block, lds, stream, a, split_k, counters);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || FIN != 2 || split_k <= 1) return e;
    return reduce_launch(a, split_k, stream);
}

template <int FIN, int CPG, int R>
hipError_t row_launch(const GemmArgs& a, int split_k, uint32_t* counters, hipStream_t stream) {
    const size_t lds = stream_lds_bytes(a.M, a.K, split_k, 8 / CPG, kStreamRowLayout);
    const dim3 grid((unsigned)(gemv_strips(a.N) * split_k)), block((unsigned)stream_threads(kStreamRowLayout, 8 / CPG));
    if (split_k <= kNonTemporalMaxSplit)
        hipLaunchKernelGGL((awq_stream_row_kernel<FIN, CPG, R, true>), grid, block, lds, stream, a, split_k, counters);
    else
        hipLaunchKernelGGL((awq_stream_row_kernel<FIN, CPG, R, false>), grid, block, lds, stream, a, split_k, counters);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || FIN != 2 || split_k <= 1) return e;
    return reduce_launch(a, split_k, stream);
}

template <int FIN>
hipError_t launch_fin(const GemmArgs& a, int split_k, int k_waves, int depth, int layout, uint32_t* counters,
                      hipStream_t stream) {
    if (layout == kStreamRowLayout) {
        switch (k_waves * 4 + depth) {
            case 33: return row_launch<FIN, 1, 1>(a, split_k, counters, stream);
            case 34: return row_launch<FIN, 1, 2>(a, split_k, counters, stream);
            case 17: return row_launch<FIN, 2, 1>(a, split_k, counters, stream);
            case 18: return row_launch<FIN, 2, 2>(a, split_k, counters, stream);
            case 10: return row_launch<FIN, 4, 2>(a, split_k, counters, stream);
            case 6: return row_launch<FIN, 8, 2>(a, split_k, counters, stream);
            default: return hipErrorInvalidValue;
        }
    }
    const bool small = a.M <= 4;
    switch (depth) {
        case 2: return small ? half_launch<4, FIN, 2>(a, split_k, k_waves, counters, stream)
                             : half_launch<16, FIN, 2>(a, split_k, k_waves, counters, stream);
        case 4: return small ? half_launch<4, FIN, 4>(a, split_k, k_waves, counters, stream)
                             : half_launch<16, FIN, 4>(a, split_k, k_waves, counters, stream);
        case 6: return small ? half_launch<4, FIN, 6>(a, split_k, k_waves, counters, stream)
                             : half_launch<16, FIN, 6>(a, split_k, k_waves, counters, stream);
        default: return hipErrorInvalidValue;
    }
}
}  // namespace

hipError_t launch_stream(const GemmArgs& a, int split_k, int k_waves, int depth, int layout, int finish,
                         uint32_t* counters, hipStream_t stream) {
    switch (finish) {
        case 0: return launch_fin<0>(a, split_k, k_waves, depth, layout, counters, stream);
        case 1: return launch_fin<1>(a, split_k, k_waves, depth, layout, counters, stream);
        case 2: return launch_fin<2>(a, split_k, k_waves, depth, layout, counters, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace awq
