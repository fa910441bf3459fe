// Decode GEMV (M <= 2) of the W4A16 AWQ GEMM for gfx950.
//
// At batch 1 the kernel is a pure stream of the int4 weights, and the time
// is set by how many bytes are in flight against the HBM latency and by the
// split-K finish at the end.  Two kernels:
//  * variant 2 (awq_gemv_stream_kernel): one 128-row group per step, lane =
//    packed column, v_dot2_f32_f16 sums; serves N % 32 != 0;
//  * variant 5 (awq_gemv_quad_kernel): column quads, 16-byte loads,
//    interleaved 32-row chunks, MFMA column sums, fixed-point split-K
//    finish; the default.
// Both handle the zero outside the dot products: the codes are read as
// fp16 (b + q) by the magic-number unpack (b = 1024, or 64 for the nibbles
// cut in place, see awq_device.h), the lanes accumulate
// sum_r x[r] * (b + q[r]) and sum_r x[r], and each group folds
// s * (that - (b + z) * sum_r x[r]) in fp32 once.
#include <type_traits>

#include "awq_kernels.h"

namespace awq {

// ---------------------------------------------------------------------------
// Variant 2: K-streaming GEMV.
//
// A workgroup walks its K range
// one 128-row group ("chunk") at a time, top to bottom, with the next chunk's
// loads in flight while the current one is computed; every workgroup runs
// the same schedule, so at any moment the machine reads a few bands of
// whole rows -- the access order of a contiguous stream.
//
// Workgroup = KW = 128 / R waves on one 64-packed-column strip; in chunk c,
// wave w reads rows 128c + R*w .. +R-1 (all inside the chunk's group), one
// 256-byte row segment per load instruction.  The zero is handled outside
// the dot products: the lanes accumulate sum_r x[r] * (b + q[r]) (the
// magic-number code) with v_dot2_f32_f16, and the chunk's result is
// (that - (b + z) * sum_r x[r]) * s, so a weight costs its unpack and one
// dot2 per row of x.  The products are exact and the fp32 sums carry the
// offset b (about 10 bits of headroom lost), far inside the tolerance; the
// weight is not rounded to fp16 before the product.
template <int MR, int R, int D>
__global__ __launch_bounds__(512) void awq_gemv_stream_kernel(GemmArgs a, int chunks_per_split, int split_k,
                                                              uint32_t* counters) {
    constexpr int KW = kGroup / R;
    __shared__ float red[(KW - 1) * MR * 8 * 64];
    __shared__ int last_flag;
    __shared__ floatx4 fin[512];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int pn = a.N >> 3;
    const int n_strips = (pn + 63) / 64;
    const int strip = blockIdx.x % n_strips;
    const int split = blockIdx.x / n_strips;
    const int j = strip * 64 + lane;
    const bool col_ok = j < pn;
    const int jc = col_ok ? j : pn - 1;
    const int groups = a.K / kGroup;
    const int c_begin = split * chunks_per_split;
    const int c_end = min(groups, c_begin + chunks_per_split);

    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.qweight, (uint32_t)((size_t)a.K * pn * 4));
    const __amdgpu_buffer_rsrc_t rz = make_rsrc(a.qzeros, (uint32_t)((size_t)groups * pn * 4));
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.scales, (uint32_t)((size_t)groups * a.N * 2));
    const uint32_t row_bytes = (uint32_t)pn * 4u;
    const uint32_t voff = (uint32_t)jc * 4u;
    const uint32_t* x32 = reinterpret_cast<const uint32_t*>(a.x);
    const uint32_t ones = 0x3C003C00u;  // fp16 (1, 1)

    float acc[MR][8];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[m][c] = 0.f;

    struct Chunk {
        uint32_t w[R];
        uint32_t zw;
        half8_t s8;
        uint32_t xp[MR][R / 2];
    };
    auto load = [&](int c, Chunk& ck) {
        const int r0 = c * kGroup + wave * R;
#pragma unroll
        for (int i = 0; i < R; ++i) ck.w[i] = buf_load_b32(rw, voff, (uint32_t)(r0 + i) * row_bytes);
        ck.zw = buf_load_b32(rz, voff, (uint32_t)c * row_bytes);
        ck.s8 = buf_load_h8(rs, (uint32_t)jc * 16u, (uint32_t)c * (uint32_t)a.N * 2u);
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int p = 0; p < R / 2; ++p)
                ck.xp[m][p] = __builtin_amdgcn_readfirstlane(x32[((size_t)m * a.K + r0) / 2 + p]);
    };
    auto compute = [&](const Chunk& ck) {
        float in[MR][8], sx[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            sx[m] = 0.f;
#pragma unroll
            for (int c = 0; c < 8; ++c) in[m][c] = 0.f;
        }
#pragma unroll
        for (int p = 0; p < R / 2; ++p) {
            uint32_t kp[8];
            kpairs_magic_inplace(ck.w[2 * p], ck.w[2 * p + 1], kp);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                sx[m] = __builtin_amdgcn_fdot2(as_h2(ck.xp[m][p]), as_h2(ones), sx[m], false);
#pragma unroll
                for (int c = 0; c < 8; ++c)
                    in[m][c] = __builtin_amdgcn_fdot2(as_h2(kp[c]), as_h2(ck.xp[m][p]), in[m][c], false);
            }
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint32_t z = (ck.zw >> col_shift(c)) & 0xFu;
            const float zz = magic_base(c) + (float)z;
            const float sc = (float)ck.s8[c];
#pragma unroll
            for (int m = 0; m < MR; ++m) acc[m][c] += sc * (in[m][c] - zz * sx[m]);
        }
    };

    // Ring of D chunk buffers: chunk c + D - 1 is loaded before chunk c is
    // computed (static buffer indices: the inner loop is unrolled).  Loads
    // past the last chunk re-read it instead of being skipped, so that every
    // compute step has the same number of loads issued after its own and the
    // compiler's wait counts stay partial (a conditional load makes it wait
    // for all outstanding loads).
    // Full rounds of D chunks have no early exit (an exit to the loop latch
    // would merge unequal load states there, with the same effect); at the
    // start of a round ck[0 .. D-2] hold its first D-1 chunks, so the last
    // (fewer than D) chunks are already loaded when the rounds end.
    if (c_begin < c_end) {
        const int c_last = c_end - 1;
        Chunk ck[D];
#pragma unroll
        for (int d = 0; d < D - 1; ++d) load(min(c_begin + d, c_last), ck[d]);
        int c = c_begin;
        for (; c + D <= c_end; c += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                load(min(c + d + D - 1, c_last), ck[(d + D - 1) % D]);
                compute(ck[d]);
            }
        }
        const int rest = c_end - c;
#pragma unroll
        for (int d = 0; d < D - 1; ++d)
            if (d < rest) compute(ck[d]);
    }

    // K reduction inside the workgroup through LDS ([wave][m][c][lane]).
    if (wave > 0) {
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int c = 0; c < 8; ++c) red[(((wave - 1) * MR + m) * 8 + c) * 64 + lane] = acc[m][c];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int q = 1; q < KW; ++q)
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int c = 0; c < 8; ++c) acc[m][c] += red[(((q - 1) * MR + m) * 8 + c) * 64 + lane];
    }

    if (split_k == 1) {
        if (wave != 0 || !col_ok) return;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            if (m >= a.M) break;
            store_out<8>(a.out, a.bias, a.residual, a.N, m, 8 * j, acc[m]);
        }
        return;
    }

    const uint32_t part_bytes = (uint32_t)((size_t)split_k * a.M * a.N * 4);
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(a.partials, part_bytes);
    if (wave == 0 && col_ok) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            if (m >= a.M) break;
            const uint32_t off = (uint32_t)((((size_t)split * a.M + m) * a.N + 8 * j) * 4);
            buf_store_f4_device(floatx4{acc[m][0], acc[m][1], acc[m][2], acc[m][3]}, rp, off);
            buf_store_f4_device(floatx4{acc[m][4], acc[m][5], acc[m][6], acc[m][7]}, rp, off + 16);
        }
    }
    wait_vm_stores();
    __syncthreads();
    if (threadIdx.x == 0)
        last_flag = __hip_atomic_fetch_add(&counters[strip], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                    (uint32_t)(split_k - 1);
    __syncthreads();
    if (!last_flag) return;
    splitk_finish<2>(rp, a.out, a.bias, a.residual, a.M, a.N, 0, a.M, strip * 512, min(512, a.N - strip * 512), split_k, fin);
    if (threadIdx.x == 0) __hip_atomic_store(&counters[strip], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Variant 5: column-quad GEMV, interleaved 32-row chunks, fixed-point split-K.
//
// Lane l: c4 = l % 16 owns packed columns CW*c4 .. CW*c4+CW-1 of the
// workgroup's 16 CW-column strip (8 CW outputs) and reads them with one
// 4 CW-byte load per row, so the 16 lanes of a row cover one 64 CW-byte row
// segment; rq = l / 16 picks rows 4*rq .. 4*rq+3 of each 16-row half of a
// 32-row chunk (one load instruction = four row segments, eight per chunk).
// CW = 4 (column quads): 512-column strips, 256-byte segments, M <= 2.
// CW = 2 (column pairs): 256-column strips, 128-byte segments, M <= 4 (the
// accumulators are 8 CW per row of x): twice the strips of the quads, so the
// same grid needs half the K splits, and the fixed-point finish half the
// atomics.
//
// Work split: the K/32 chunks of a strip are divided evenly among split_k
// workgroups (the planner keeps split_k * strips within one workgroup per
// CU: a CU holding two workgroups of this kernel finishes last); inside a
// workgroup the waves take every nw-th chunk, so at any time they read
// adjacent rows (measured faster than giving each wave a contiguous range).
// A chunk lies inside one 128-row group.
//
// Prologue: the workgroup turns the zeros and scales of the groups it
// touches into fp32 pairs (s, s * (b + z)) per column -- b the offset of the
// column's magic-number codes -- and stages them and its rows of x
// in LDS.  The main loop's only vector memory operations are then the weight
// loads: a ring of D chunk buffers keeps D - 1 chunks' loads in flight while
// one chunk is computed, every load is issued (chunks past the wave's range get an
// out-of-range offset, so the compiler's wait counts stay static), and
// scheduling barriers keep a chunk's arithmetic after the loads issued
// before it.
//
// Arithmetic: per chunk, sum_r x[r] * (b + q) per column on
// v_mfma_f32_16x16x32_f16: the magic-number k-pairs of a lane's 8 rows of
// one column are its B fragment as they are (lane n = c4, k-block = rq: the
// MFMA operand layout), x rows m = c4 < M supply A in the same k order, and
// an MFMA against ones gives sum_r x[r]; the MFMA sums the 32 rows inside the
// chunk, so lane (c4, rq = 0) holds row m of its 8 CW columns in register m
// and no cross-lane reduction is needed.  After each chunk acc += s * sum -
// s(b + z) * sum_x for the M live rows.  At the end the waves are added
// through LDS and each output's partial is stored (split_k == 1) or goes
// through the fixed-point finish.  Needs N % 32 == 0 (whole quads).
constexpr int kQuadItemsPerThread = 4;  // prologue loads per thread (consts and x each)

template <int MR, int D, bool NT, int CW, bool RED = false>
__global__ __launch_bounds__(512) void awq_gemv_quad_kernel(GemmArgs a, int split_k, unsigned long long* fix) {
    extern __shared__ __align__(16) uint32_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nw = blockDim.x >> 6;
    const int c4 = lane & 15;
    const int rq = lane >> 4;
    constexpr int SP = 16 * CW;  // packed columns of a strip
    constexpr int SC = 8 * SP;   // output columns of a strip
    // D rows live per lane: MR <= 4, rows 0 .. MR - 1 in the lanes of k-block
    // 0; MR = 8 / 16, rows 4 rq .. 4 rq + 3 in the lanes of k-blocks 0 .. 1 / 0 .. 3.
    constexpr int NR = MR > 4 ? 4 : MR;
    constexpr int XI = MR > 8 ? 16 : (MR > 4 ? 8 : kQuadItemsPerThread);  // x prologue loads per thread
    static_assert(MR <= 8 || RED, "16 rows of x take the reduce-launch finish");
    const int pn = a.N >> 3;
    const int n_strips = (pn + SP - 1) / SP;
    // Work item w = (split, strip), strip fastest, numbered in XCD order:
    // workgroups are dispatched round-robin over the 8 XCDs (workgroup b on
    // XCD b % 8), and the workgroups one XCD runs get consecutive items, so
    // neighbouring strips run on one XCD -- with 128-column strips (64-byte
    // row segments) two strips share each 128-byte line, which one L2 then
    // fetches once.  Any numbering is correct; this one is about traffic.
    const int total = (int)gridDim.x;
    const int xb = (int)blockIdx.x & 7, xi = (int)blockIdx.x >> 3, per_x = (total + 7) >> 3, rem_x = total & 7;
    const int w_item = (rem_x == 0 || xb < rem_x) ? xb * per_x + xi : rem_x * per_x + (xb - rem_x) * (per_x - 1) + xi;
    const int strip = w_item % n_strips;
    const int split = w_item / n_strips;
    const int jl = min(strip * SP + CW * c4, pn - CW);  // in-range columns; lanes past pn drop their results
    const int C = a.K / 32;
    const int c0 = (int)((int64_t)C * split / split_k);
    const int c1 = (int)((int64_t)C * (split + 1) / split_k);
    const int nc = c1 - c0;
    const int g_lo = c0 / 4;
    const int n_g = nc > 0 ? (c1 - 1) / 4 - g_lo + 1 : 0;
    const int groups = a.K / kGroup;

    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.qweight, (uint32_t)((size_t)a.K * pn * 4));
    const __amdgpu_buffer_rsrc_t rz = make_rsrc(a.qzeros, (uint32_t)((size_t)groups * pn * 4));
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.scales, (uint32_t)((size_t)groups * a.N * 2));
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (uint32_t)((size_t)a.M * a.K * 2));
    const uint32_t row_bytes = (uint32_t)pn * 4u;
    const uint32_t voff_w = (uint32_t)(4 * rq) * row_bytes + (uint32_t)jl * 4u;

    // LDS: consts float4 [n_g][4 CW][16] ((s', s'(1024+z')) of two columns,
    // indexed [group][column pair i of the lane][lane c4]: one wave-wide read
    // is 256 consecutive bytes), then x [MR][nc * 32] fp16.
    floatx4* lc = reinterpret_cast<floatx4*>(lds);
    half_t* lx = reinterpret_cast<half_t*>(lds + n_g * (4 * CW) * 16 * 4);

    // Prologue loads: item (g, j) = zero word and 8 scales of packed column j
    // of group g_lo + g; x in 16-byte pieces.  Issued before the weights.
    const int nt = blockDim.x;
    u32x4 sv[kQuadItemsPerThread];
    uint32_t zv[kQuadItemsPerThread];
    u32x4 xv[XI];
    auto fence = [] { __builtin_amdgcn_sched_barrier(0); };
#pragma unroll
    for (int i = 0; i < kQuadItemsPerThread; ++i) {
        const int item = min((int)threadIdx.x + i * nt, max(n_g * SP - 1, 0));
        const int g = g_lo + item / SP;
        const int j = min(strip * SP + item % SP, pn - 1);
        zv[i] = buf_load_b32(rz, (uint32_t)(g * pn + j) * 4u, 0u);
        sv[i] = buf_load_u4(rs, (uint32_t)(((size_t)g * a.N + 8 * j) * 2), 0u);
    }
#pragma unroll
    for (int i = 0; i < XI; ++i) {
        const int xi = (int)threadIdx.x + i * nt;  // x piece: row m, 8 rows at c0*32 + 8 * (xi % (nc * 4))
        const int m = xi / max(nc * 4, 1);
        const uint32_t xoff = (uint32_t)(((size_t)m * a.K + (size_t)c0 * 32 + 8 * (xi % max(nc * 4, 1))) * 2);
        xv[i] = buf_load_u4(rx, m < MR ? xoff : 0x80000000u, 0u);
    }

    typedef uint32_t cwv_t __attribute__((ext_vector_type(CW < 2 ? 2 : CW)));
    using cw_t = std::conditional_t<CW == 1, uint32_t, cwv_t>;
    struct Chunk {
        cw_t w[8];
    };
    // Packed column p of the lane's words.
    auto word = [](const cw_t& v, int p) -> uint32_t {
        if constexpr (CW == 1)
            return v;
        else
            return v[p];
    };
    // Chunk c (rows 32c .. 32c+31); chunks past the wave's range read zeros.
    auto load_chunk = [&](int c, Chunk& ck) {
        const bool live = c < c1;
        const uint32_t oob = live ? 0u : 0x80000000u;
        const uint32_t r0 = live ? (uint32_t)c * 32u : 0u;
#pragma unroll
        for (int u = 0; u < 8; ++u)
        {
            const uint32_t so = (r0 + (u & 3) + 16 * (u >> 2)) * row_bytes;
            if constexpr (CW == 4)
                ck.w[u] = __builtin_bit_cast(cw_t, __builtin_amdgcn_raw_buffer_load_b128(rw, voff_w + oob, so, NT ? kCpolNT : 0));
            else if constexpr (CW == 2)
                ck.w[u] = __builtin_bit_cast(cw_t, __builtin_amdgcn_raw_buffer_load_b64(rw, voff_w + oob, so, NT ? kCpolNT : 0));
            else
                ck.w[u] = __builtin_amdgcn_raw_buffer_load_b32(rw, voff_w + oob, so, NT ? kCpolNT : 0);
        }
    };
    // Ring of D chunk buffers: the wave's chunks i = 0, 1, ... (chunk c0 + wave
    // + i * nw) go to buffer i % D; chunk i + D is loaded right after chunk i
    // is computed, so D - 1 chunks are in flight during each computation.
    Chunk ring[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        fence();
        load_chunk(c0 + wave + d * nw, ring[d]);
    }
    fence();

#pragma unroll
    for (int i = 0; i < kQuadItemsPerThread; ++i) {
        const int item = (int)threadIdx.x + i * nt;
        if (item < n_g * SP) {
            const int g = item / SP;
            const int j = item % SP;  // packed column of the strip: lane j / CW, its columns 8 (j % CW) + c
            const half8_t s8 = __builtin_bit_cast(half8_t, sv[i]);
#pragma unroll
            for (int c = 0; c < 8; c += 2) {
                floatx4 v;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int cc = c + h;
                    const uint32_t z = (zv[i] >> col_shift(cc)) & 0xFu;
                    const float sc = (float)s8[cc];
                    const float zz = magic_base(cc) + (float)z;
                    v[2 * h] = sc;
                    v[2 * h + 1] = sc * zz;
                }
                const int col = 8 * (j % CW) + c;  // column of the lane: pair index col / 2
                lc[(g * (4 * CW) + col / 2) * 16 + j / CW] = v;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < XI; ++i) {
        const int item = (int)threadIdx.x + i * nt;
        if (item < MR * nc * 4) *reinterpret_cast<u32x4*>(lx + 8 * item) = xv[i];
    }
    __syncthreads();

    float acc[NR][8 * CW];
#pragma unroll
    for (int m = 0; m < NR; ++m)
#pragma unroll
        for (int i = 0; i < 8 * CW; ++i) acc[m][i] = 0.f;
    const uint32_t ones = 0x3C003C00u;  // fp16 (1, 1)

    // A = x rows (zero for lanes c4 >= M), S = row sums of x.
    auto compute = [&](const Chunk& ck, int c) {
        const int cl = c - c0;
        u32x4 av = {0u, 0u, 0u, 0u};
        if (c4 < MR) {
            const u32x2 lo = *reinterpret_cast<const u32x2*>(lx + (size_t)c4 * nc * 32 + cl * 32 + 4 * rq);
            const u32x2 hi = *reinterpret_cast<const u32x2*>(lx + (size_t)c4 * nc * 32 + cl * 32 + 16 + 4 * rq);
            av = u32x4{lo[0], lo[1], hi[0], hi[1]};
        }
        const half8_t xa = __builtin_bit_cast(half8_t, av);
        const floatx4 zero4 = {0.f, 0.f, 0.f, 0.f};
        const floatx4 S = mfma16x16x32(xa, __builtin_bit_cast(half8_t, u32x4{ones, ones, ones, ones}), zero4);
        const int gi = c / 4 - g_lo;
#pragma unroll
        for (int p = 0; p < CW; ++p) {
            uint32_t kp[4][8];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 2; ++i)
                    kpairs_magic_inplace(word(ck.w[4 * h + 2 * i], p), word(ck.w[4 * h + 2 * i + 1], p), kp[2 * h + i]);
#pragma unroll
            for (int cc = 0; cc < 8; cc += 2) {
                const floatx4 v = lc[(gi * (4 * CW) + (8 * p + cc) / 2) * 16 + c4];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int col = 8 * p + cc + e;
                    const floatx4 Cv = mfma16x16x32(
                        xa, __builtin_bit_cast(half8_t, u32x4{kp[0][cc + e], kp[1][cc + e], kp[2][cc + e], kp[3][cc + e]}),
                        zero4);
#pragma unroll
                    for (int m = 0; m < NR; ++m)
                        acc[m][col] = __builtin_fmaf(-v[2 * e + 1], S[m], __builtin_fmaf(v[2 * e], Cv[m], acc[m][col]));
                }
            }
        }
    };

    for (int c = c0 + wave; c < c1; c += D * nw) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            fence();
            if (c + d * nw < c1) compute(ring[d], c + d * nw);
            fence();
            load_chunk(c + (d + D) * nw, ring[d]);
        }
        fence();
    }

    __syncthreads();  // every wave is done with the staged consts: the LDS becomes the reduction buffer
    float* red = reinterpret_cast<float*>(lds);
    if (rq < (MR + 3) / 4) {
        const int row0 = 4 * rq;
#pragma unroll
        for (int m = 0; m < NR; ++m)
#pragma unroll
            for (int i = 0; i < 8 * CW; i += 4)
                *reinterpret_cast<floatx4*>(&red[(wave * MR + row0 + m) * SC + 8 * CW * c4 + i]) =
                    floatx4{acc[m][i], acc[m][i + 1], acc[m][i + 2], acc[m][i + 3]};
    }
    __syncthreads();
    if constexpr (RED) {
        if (split_k > 1) {
            // fp32 partials [split_k, M, N] (write-through), added by a second
            // launch of awq_splitk_reduce_kernel.  A thread takes four
            // consecutive columns (N % 32 == 0: all or none of them exist),
            // so a wave's store covers 1 KB of a row.
            const __amdgpu_buffer_rsrc_t rp = make_rsrc(a.partials, (uint32_t)((size_t)split_k * a.M * a.N * 4));
            for (int idx = threadIdx.x; idx < MR * SC / 4; idx += nt) {
                const int m = idx / (SC / 4), t = 4 * (idx - m * (SC / 4)), n = strip * SC + t;
                if (m >= a.M || n >= a.N) continue;
                floatx4 v = {0.f, 0.f, 0.f, 0.f};
                for (int w = 0; w < nw; ++w) v += *reinterpret_cast<const floatx4*>(&red[(w * MR + m) * SC + t]);
                buf_store_f4_device(v, rp, (uint32_t)((((size_t)split * a.M + m) * a.N + n) * 4));
            }
            return;
        }
    }
    // Thread t finishes outputs t, t + nt, ... of the strip (at most SC / 64
    // per row of x) in one batch: one memory round trip per thread.
    constexpr int kOwn = SC / 64;
    constexpr int FB = MR > 8 ? 8 : MR;  // rows per finish batch (16 rows: two, at split_k 1 only)
#pragma unroll
    for (int mb = 0; mb < MR; mb += FB) {
        float fs[kOwn * FB];
        int fm[kOwn * FB], fn[kOwn * FB];
        bool fok[kOwn * FB];
#pragma unroll
        for (int i = 0; i < kOwn; ++i)
#pragma unroll
            for (int mm = 0; mm < FB; ++mm) {
                const int m = mb + mm;
                const int t = threadIdx.x + i * nt;
                float s = 0.f;
                if (t < SC)
                    for (int w = 0; w < nw; ++w) s += red[(w * MR + m) * SC + t];
                fs[i * FB + mm] = s;
                fm[i * FB + mm] = m;
                fn[i * FB + mm] = strip * SC + t;
                fok[i * FB + mm] = t < SC && strip * SC + t < a.N && m < a.M;
            }
        finish_batch<kOwn * FB>(fix, a.out, a.bias, a.residual, a.M, a.N, split_k, fs, fm, fn, fok);
    }
}

// Groups a workgroup's chunk range can touch: at most ceil(per / 4) + 1.
int64_t gemv_quad_max_groups(int K, int split_k) {
    const int64_t C = K / 32;
    const int64_t per = (C + split_k - 1) / split_k;
    return (per + 2) / 4 + 1;
}

// Rows of x a column-quad / column-pair GEMV instance carries for M rows.
static int gemv_quad_mr(int M) { return M <= 1 ? 1 : (M <= 2 ? 2 : (M <= 4 ? 4 : (M <= 8 ? 8 : 16))); }

// LDS of the column-quad (cw 4) or column-pair (cw 2) GEMV: staged consts
// (1 KiB x cw per group) and x rows, or the cross-wave reduction buffer,
// whichever is larger.
size_t gemv_quad_lds_bytes(int M, int K, int split_k, int k_waves, int cw) {
    const int64_t C = K / 32;
    const int64_t per = (C + split_k - 1) / split_k;
    const int mr = gemv_quad_mr(M);
    const size_t staged = (size_t)gemv_quad_max_groups(K, split_k) * 1024 * cw + (size_t)mr * per * 64;
    const size_t red = (size_t)k_waves * mr * 128 * cw * 4;
    return staged > red ? staged : red;
}

// Whether the prologue's fixed number of loads per thread covers the shape.
bool gemv_quad_fits(int M, int K, int split_k, int k_waves, int cw) {
    const int64_t C = K / 32;
    const int64_t per = (C + split_k - 1) / split_k;
    const int64_t threads = 64 * (int64_t)k_waves;
    const int mr = gemv_quad_mr(M);
    return gemv_quad_max_groups(K, split_k) * 16 * cw <= kQuadItemsPerThread * threads &&
           mr * per * 4 <= (mr > 8 ? 16 : (mr > 4 ? 8 : kQuadItemsPerThread)) * threads;
}

int64_t gemv_strips(int N) { return ((N >> 3) + 63) / 64; }
int64_t gemv_strips_cw(int N, int cw) { return ((N >> 3) + 16 * cw - 1) / (16 * cw); }

template <int MR, int R, int D>
static hipError_t gemv_stream_launch(const GemmArgs& a, const GemvConfig& cfg, uint32_t* counters,
                                     hipStream_t stream) {
    const dim3 grid((unsigned)(gemv_strips(a.N) * cfg.split_k)), block(64 * (kGroup / R));
    hipLaunchKernelGGL((awq_gemv_stream_kernel<MR, R, D>), grid, block, 0, stream, a, cfg.chunks_per_split,
                       cfg.split_k, counters);
    return hipGetLastError();
}

template <int MR, int D, int CW, bool RED = false>
static hipError_t gemv_quad_launch(const GemmArgs& a, const GemvConfig& cfg, uint32_t* counters,
                                   hipStream_t stream) {
    unsigned long long* fix = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(counters) + kCounterBytes);
    const size_t lds = gemv_quad_lds_bytes(a.M, a.K, cfg.split_k, cfg.kw_count, CW);
    const dim3 grid((unsigned)(gemv_strips_cw(a.N, CW) * cfg.split_k)), block(64 * cfg.kw_count);
    // Weight loads marked non-temporal where each workgroup streams a long
    // K range (few splits): 3584 x 37888 at split 3 measured 2.7 - 4.7 %
    // faster with them at M = 1 - 16, the 100 - 500-row ranges of 18 - 36
    // splits up to 3 % slower.
    if (cfg.split_k <= kNonTemporalMaxSplit)
        hipLaunchKernelGGL((awq_gemv_quad_kernel<MR, D, true, CW, RED>), grid, block, lds, stream, a, cfg.split_k, fix);
    else
        hipLaunchKernelGGL((awq_gemv_quad_kernel<MR, D, false, CW, RED>), grid, block, lds, stream, a, cfg.split_k, fix);
    const hipError_t e = hipGetLastError();
    if (!RED || e != hipSuccess || cfg.split_k <= 1) return e;
    return splitk_reduce_launch(a, cfg.split_k, stream);
}

static hipError_t gemv_quad_dispatch(const GemmArgs& a, const GemvConfig& cfg, uint32_t* counters,
                                     hipStream_t stream) {
    if (cfg.cw == 1) {
        switch (gemv_quad_mr(a.M) * 10 + cfg.depth) {
            case 12: return gemv_quad_launch<1, 2, 1>(a, cfg, counters, stream);
            case 13: return gemv_quad_launch<1, 3, 1>(a, cfg, counters, stream);
            case 22: return gemv_quad_launch<2, 2, 1>(a, cfg, counters, stream);
            case 23: return gemv_quad_launch<2, 3, 1>(a, cfg, counters, stream);
            case 42: return gemv_quad_launch<4, 2, 1>(a, cfg, counters, stream);
            case 43: return gemv_quad_launch<4, 3, 1>(a, cfg, counters, stream);
            case 82: return gemv_quad_launch<8, 2, 1>(a, cfg, counters, stream);
            case 83: return gemv_quad_launch<8, 3, 1>(a, cfg, counters, stream);
            default: return hipErrorInvalidValue;
        }
    }
    if (cfg.cw == 2) {
        switch (gemv_quad_mr(a.M) * 10 + cfg.depth) {
            case 12: return gemv_quad_launch<1, 2, 2>(a, cfg, counters, stream);
            case 13: return gemv_quad_launch<1, 3, 2>(a, cfg, counters, stream);
            case 22: return gemv_quad_launch<2, 2, 2>(a, cfg, counters, stream);
            case 23: return gemv_quad_launch<2, 3, 2>(a, cfg, counters, stream);
            case 42: return gemv_quad_launch<4, 2, 2>(a, cfg, counters, stream);
            case 43: return gemv_quad_launch<4, 3, 2>(a, cfg, counters, stream);
            default: return hipErrorInvalidValue;
        }
    }
    if (cfg.cw != 4 || a.M > 2) return hipErrorInvalidValue;
    switch ((a.M <= 1 ? 10 : 20) + cfg.depth) {
        case 12: return gemv_quad_launch<1, 2, 4>(a, cfg, counters, stream);
        case 13: return gemv_quad_launch<1, 3, 4>(a, cfg, counters, stream);
        case 14: return gemv_quad_launch<1, 4, 4>(a, cfg, counters, stream);
        case 22: return gemv_quad_launch<2, 2, 4>(a, cfg, counters, stream);
        case 23: return gemv_quad_launch<2, 3, 4>(a, cfg, counters, stream);
        case 24: return gemv_quad_launch<2, 4, 4>(a, cfg, counters, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv(const GemmArgs& a, const GemvConfig& cfg, uint32_t* counters, hipStream_t stream) {
    if (cfg.variant == 5) return gemv_quad_dispatch(a, cfg, counters, stream);
    if (cfg.variant == 6) {
        // Column singles with 16 rows of x, fp32 partials and the reduce launch.
        if (cfg.cw != 1 || gemv_quad_mr(a.M) != 16 || cfg.depth != 2) return hipErrorInvalidValue;
        return gemv_quad_launch<16, 2, 1, true>(a, cfg, counters, stream);
    }
    if (cfg.variant == 2) {
        const int key2 = (a.M <= 1 ? 1 : 2) * 10000 + cfg.rows_per_wave * 10 + cfg.depth;
        switch (key2) {
            case 10162: return gemv_stream_launch<1, 16, 2>(a, cfg, counters, stream);
            case 10163: return gemv_stream_launch<1, 16, 3>(a, cfg, counters, stream);
            case 10164: return gemv_stream_launch<1, 16, 4>(a, cfg, counters, stream);
            case 10322: return gemv_stream_launch<1, 32, 2>(a, cfg, counters, stream);
            case 10323: return gemv_stream_launch<1, 32, 3>(a, cfg, counters, stream);
            case 20162: return gemv_stream_launch<2, 16, 2>(a, cfg, counters, stream);
            case 20163: return gemv_stream_launch<2, 16, 3>(a, cfg, counters, stream);
            case 20164: return gemv_stream_launch<2, 16, 4>(a, cfg, counters, stream);
            case 20322: return gemv_stream_launch<2, 32, 2>(a, cfg, counters, stream);
            case 20323: return gemv_stream_launch<2, 32, 3>(a, cfg, counters, stream);
            default: return hipErrorInvalidValue;
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace awq
