// Streaming W4A16 AWQ GEMM for small M (M <= 16) on the MFMA units of gfx950.
//
// The weight stream is the whole cost, so the memory side is the column-quad
// GEMV's (awq_gemv.hip, variant 4): lane l, c4 = l % 16, reads packed
// columns 4*c4 .. 4*c4+3 of a 64-column strip with one 16-byte load per row
// (16 lanes = one 256-byte row segment); rq = l / 16 picks rows 4*rq ..
// 4*rq+3 of each 16-row half of a 32-row chunk; the waves of a workgroup
// take every nw-th chunk of the workgroup's share of K; one 128-row group's
// zeros and scales are staged in LDS; the next chunk's loads are in flight
// while one is computed; fixed-point split-K finish.
//
// That lane layout is also the operand layout of v_mfma_f32_16x16x32_f16
// with n = c4 and k-block = rq: a lane's 8 rows of one logical column form
// its B fragment (k slots 0..3 = rows 4rq..4rq+3 of the first half, 4..7 =
// the same rows of the second half), and x supplies A with the same k order
// (lane m = c4 reads its row of x; rows >= M read as zeros).  Each of the 32
// logical columns of a lane is one MFMA per chunk; the accumulators hold
// out[4*rq + r][column] for r = 0..3 -- all 16 rows of x at once.
//
// The weight is formed exactly as the reference does, fp16((q - z) * s)
// (kernels/awq_gemm.py:59): from the magic-number k-pairs (1024 + q', x16
// for columns 2, 3, 6, 7) one packed fp16 op gives q - z exactly
// ((1024 + q') * f - (1024 + z') * f with f = 1 or 1/16, both exact) and one
// packed multiply by the scale rounds once.  The staged constants are the
// fp16 splats -(1024 + z') * f and s of every column.
//
// Split-K: see PART below.
#include "awq_kernels.h"

namespace awq {

namespace {
constexpr int kStreamItemsPerThread = 4;  // prologue loads per thread
constexpr uint32_t kSixteenth2 = 0x2C002C00u;  // fp16 pair (1/16, 1/16)
}  // namespace

// PART selects the split-K finish: false -- 64-bit fixed-point slots, one
// atomic per output element per workgroup (one memory round trip; best when
// M * N * split_k is small); true -- fp32 partials [split, M, N] stored with
// device-scope stores, an arrival counter per strip, and the last workgroup
// adds the partials in split order (three round trips, but no per-element
// atomics, whose device-wide rate falls short at M >= 4).
template <int MP, bool PART>  // MP: rows of x covered by the finish: 4, 8 or 16 (>= M)
__global__ __launch_bounds__(256) void awq_stream_kernel(GemmArgs a, int split_k, uint32_t* counters) {
    extern __shared__ __align__(16) uint32_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nw = blockDim.x >> 6;
    const int c4 = lane & 15;
    const int rq = lane >> 4;
    const int pn = a.N >> 3;
    const int n_strips = (pn + 63) / 64;
    const int strip = blockIdx.x % n_strips;
    const int split = blockIdx.x / n_strips;
    const int jl = min(strip * 64 + 4 * c4, pn - 4);  // in-range quad; lanes past pn drop their results
    const int C = a.K / 32;
    const int c0 = (int)((int64_t)C * split / split_k);
    const int c1 = (int)((int64_t)C * (split + 1) / split_k);
    const int g_lo = c0 / 4;
    const int n_g = c1 > c0 ? (c1 - 1) / 4 - g_lo + 1 : 0;
    const int groups = a.K / kGroup;

    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.qweight, (uint32_t)((size_t)a.K * pn * 4));
    const __amdgpu_buffer_rsrc_t rz = make_rsrc(a.qzeros, (uint32_t)((size_t)groups * pn * 4));
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.scales, (uint32_t)((size_t)groups * a.N * 2));
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (uint32_t)((size_t)a.M * a.K * 2));
    const uint32_t row_bytes = (uint32_t)pn * 4u;
    const uint32_t voff_w = (uint32_t)(4 * rq) * row_bytes + (uint32_t)jl * 4u;
    const uint32_t voff_x = (uint32_t)((c4 * a.K + 4 * rq) * 2);  // row c4 of x; rows >= M read 0
    unsigned long long* fix = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(counters) + kCounterBytes);

    // Staged constants: u32x4 [n_g][16][16], piece i of lane quad c4 holds the
    // splats (nz, s) of its columns 2i and 2i+1 (one wave-wide read = 256
    // consecutive bytes).
    u32x4* lc = reinterpret_cast<u32x4*>(lds);
    const int nt = blockDim.x;
    u32x4 sv[kStreamItemsPerThread];
    uint32_t zv[kStreamItemsPerThread];
    auto fence = [] { __builtin_amdgcn_sched_barrier(0); };
#pragma unroll
    for (int i = 0; i < kStreamItemsPerThread; ++i) {
        const int item = min((int)threadIdx.x + i * nt, max(n_g * 64 - 1, 0));
        const int g = g_lo + item / 64;
        const int j = min(strip * 64 + item % 64, pn - 1);
        zv[i] = buf_load_b32(rz, (uint32_t)(g * pn + j) * 4u, 0u);
        sv[i] = buf_load_u4(rs, (uint32_t)(((size_t)g * a.N + 8 * j) * 2), 0u);
    }

    struct Chunk {
        u32x4 w[8];
        u32x2 xa[2];
    };
    // Chunk c (rows 32c .. 32c+31); chunks past the wave's range read zeros
    // (out-of-range VGPR offset: no memory access, static wait counts).
    auto load_chunk = [&](int c, Chunk& ck) {
        const bool live = c < c1;
        const uint32_t oob = live ? 0u : 0x80000000u;
        const uint32_t r0 = live ? (uint32_t)c * 32u : 0u;
#pragma unroll
        for (int u = 0; u < 8; ++u)
            ck.w[u] = buf_load_u4(rw, voff_w + oob, (r0 + (u & 3) + 16 * (u >> 2)) * row_bytes);
#pragma unroll
        for (int h = 0; h < 2; ++h)
            ck.xa[h] = __builtin_bit_cast(u32x2,
                                          __builtin_amdgcn_raw_buffer_load_b64(rx, voff_x + oob, (r0 + 16 * h) * 2u, 0));
    };
    Chunk A, B;
    fence();
    load_chunk(c0 + wave, A);
    fence();
    load_chunk(c0 + wave + nw, B);
    fence();

#pragma unroll
    for (int i = 0; i < kStreamItemsPerThread; ++i) {
        const int item = (int)threadIdx.x + i * nt;
        if (item < n_g * 64) {
            const int g = item / 64;
            const int j = item % 64;  // packed column of the strip: lane quad j / 4, columns 8 (j % 4) + c
            const half8_t s8 = __builtin_bit_cast(half8_t, sv[i]);
#pragma unroll
            for (int c = 0; c < 8; c += 2) {
                u32x4 v;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int cc = c + h;
                    const uint32_t z = (zv[i] >> col_shift(cc)) & 0xFu;
                    // -(1024 + z') * f: -(1024 + z) or -(64 + z), exact in fp16.
                    const half_t nz = x16_column(cc) ? (half_t)(-(float)(64u + z)) : (half_t)(-(float)(1024u + z));
                    v[2 * h] = as_u32(half2_t{nz, nz});
                    v[2 * h + 1] = as_u32(half2_t{s8[cc], s8[cc]});
                }
                const int col = 8 * (j % 4) + c;
                lc[(g * 16 + col / 2) * 16 + j / 4] = v;
            }
        }
    }
    __syncthreads();

    floatx4 tot[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) tot[i] = floatx4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](const Chunk& ck, int c) {
        const int gi = c / 4 - g_lo;
        const half8_t xa = __builtin_bit_cast(half8_t, u32x4{ck.xa[0][0], ck.xa[0][1], ck.xa[1][0], ck.xa[1][1]});
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            uint32_t kp[4][8];
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < 2; ++i) kpairs_magic_x16(ck.w[4 * h + 2 * i][p], ck.w[4 * h + 2 * i + 1][p], kp[2 * h + i]);
#pragma unroll
            for (int cc = 0; cc < 8; cc += 2) {
                const u32x4 cv = lc[(gi * 16 + (8 * p + cc) / 2) * 16 + c4];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int col = cc + e;
                    const half2_t nz = as_h2(cv[2 * e]);
                    const half2_t s2 = as_h2(cv[2 * e + 1]);
                    u32x4 b;
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const half2_t d = x16_column(col)
                                              ? __builtin_elementwise_fma(as_h2(kp[t][col]), as_h2(kSixteenth2), nz)
                                              : as_h2(kp[t][col]) + nz;
                        b[t] = as_u32(d * s2);
                    }
                    tot[8 * p + col] = mfma16x16x32(xa, __builtin_bit_cast(half8_t, b), tot[8 * p + col]);
                }
            }
        }
    };

    // A holds chunk c, B chunk c + nw at the top of each iteration.
    for (int c = c0 + wave; c < c1; c += 2 * nw) {
        fence();
        compute(A, c);
        fence();
        load_chunk(c + 2 * nw, A);
        fence();
        if (c + nw < c1) compute(B, c + nw);
        fence();
        load_chunk(c + 3 * nw, B);
        fence();
    }

    // Cross-wave sum through LDS, rows < MP: red[w][m][512 columns]; lane
    // (c4, rq) holds rows 4*rq + r of its 32 columns 32*c4 + 8*p + cc.
    __syncthreads();  // every wave is done with the staged constants
    float* red = reinterpret_cast<float*>(lds);
    if (4 * rq < MP) {
#pragma unroll
        for (int p = 0; p < 4; ++p)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int cc = 0; cc < 8; cc += 4)
                    *reinterpret_cast<floatx4*>(&red[(wave * MP + 4 * rq + r) * 512 + 32 * c4 + 8 * p + cc]) =
                        floatx4{tot[8 * p + cc][r], tot[8 * p + cc + 1][r], tot[8 * p + cc + 2][r],
                                tot[8 * p + cc + 3][r]};
    }
    __syncthreads();

    if constexpr (PART) {
        // This workgroup's partial of rows < M, columns of the strip.
        __shared__ int last_flag;
        const int ncols = min(512, a.N - strip * 512);
        const uint32_t part_bytes = (uint32_t)((size_t)split_k * a.M * a.N * 4);
        const __amdgpu_buffer_rsrc_t rp = make_rsrc(a.partials, part_bytes);
        if (split_k > 1) {
            for (int it = threadIdx.x; it < a.M * 128; it += nt) {
                const int m = it / 128;
                const int q = it % 128;  // column quad of the strip
                if (4 * q >= ncols) continue;
                floatx4 v = {0.f, 0.f, 0.f, 0.f};
                for (int w = 0; w < nw; ++w) v += *reinterpret_cast<const floatx4*>(&red[(w * MP + m) * 512 + 4 * q]);
                buf_store_f4_device(v, rp, (uint32_t)((((size_t)split * a.M + m) * a.N + strip * 512 + 4 * q) * 4));
            }
            wait_vm_stores();
            __syncthreads();
            if (threadIdx.x == 0)
                last_flag = __hip_atomic_fetch_add(&counters[strip], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                            (uint32_t)(split_k - 1);
            __syncthreads();
            if (!last_flag) return;
            splitk_finish<4>(rp, a.out, a.M, a.N, 0, a.M, strip * 512, ncols, split_k, reinterpret_cast<floatx4*>(red));
            if (threadIdx.x == 0) __hip_atomic_store(&counters[strip], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            for (int it = threadIdx.x; it < a.M * 512; it += nt) {
                const int m = it / 512;
                const int col = strip * 512 + it % 512;
                if (col >= a.N) continue;
                float sum = 0.f;
                for (int w = 0; w < nw; ++w) sum += red[(w * MP + m) * 512 + it % 512];
                a.out[(size_t)m * a.N + col] = (half_t)sum;
            }
        }
        return;
    }

    // Output items (m, column): all atomics of a batch are issued before
    // their returns are examined.
    const int items = min(a.M, MP) * 512;
    constexpr int BATCH = 8;
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
                for (int w = 0; w < nw; ++w) sum[b] += red[(w * MP + m[b]) * 512 + it % 512];
        }
        if (split_k == 1) {
#pragma unroll
            for (int b = 0; b < BATCH; ++b)
                if (ok[b]) a.out[(size_t)m[b] * a.N + col[b]] = (half_t)sum[b];
            continue;
        }
        unsigned long long v[BATCH], now[BATCH];
#pragma unroll
        for (int b = 0; b < BATCH; ++b) {
            v[b] = fixed_point_word(sum[b]);
            now[b] = ok[b] ? __hip_atomic_fetch_add(fix + (size_t)m[b] * a.N + col[b], v[b], __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT) + v[b]
                           : 0ull;
        }
#pragma unroll
        for (int b = 0; b < BATCH; ++b)
            if (ok[b]) fixed_point_complete(now[b], fix + (size_t)m[b] * a.N + col[b], a.out + (size_t)m[b] * a.N + col[b],
                                            split_k);
    }
}

// Groups a workgroup's chunk range can touch, and the LDS the kernel needs:
// staged constants (4 KiB per group) or the cross-wave sums, the larger.
int64_t stream_max_groups(int K, int split_k) {
    const int64_t C = K / 32;
    const int64_t per = (C + split_k - 1) / split_k;
    return (per + 2) / 4 + 1;
}

int stream_rows(int M) { return M <= 4 ? 4 : (M <= 8 ? 8 : 16); }

size_t stream_lds_bytes(int M, int K, int split_k, int k_waves) {
    const size_t staged = (size_t)stream_max_groups(K, split_k) * 4096;
    const size_t red = (size_t)k_waves * stream_rows(M) * 512 * 4;
    return staged > red ? staged : red;
}

bool stream_fits(int K, int split_k, int k_waves) {
    return stream_max_groups(K, split_k) * 64 <= kStreamItemsPerThread * 64 * (int64_t)k_waves;
}

template <int MP, bool PART>
static hipError_t stream_launch(const GemmArgs& a, int split_k, int k_waves, uint32_t* counters, hipStream_t stream) {
    const size_t lds = stream_lds_bytes(a.M, a.K, split_k, k_waves);
    hipLaunchKernelGGL((awq_stream_kernel<MP, PART>), dim3((unsigned)(gemv_strips(a.N) * split_k)), dim3(64 * k_waves),
                       lds, stream, a, split_k, counters);
    return hipGetLastError();
}

hipError_t launch_stream(const GemmArgs& a, int split_k, int k_waves, bool partials, uint32_t* counters,
                         hipStream_t stream) {
    switch (stream_rows(a.M) * 2 + (partials ? 1 : 0)) {
        case 8: return stream_launch<4, false>(a, split_k, k_waves, counters, stream);
        case 9: return stream_launch<4, true>(a, split_k, k_waves, counters, stream);
        case 16: return stream_launch<8, false>(a, split_k, k_waves, counters, stream);
        case 17: return stream_launch<8, true>(a, split_k, k_waves, counters, stream);
        case 32: return stream_launch<16, false>(a, split_k, k_waves, counters, stream);
        default: return stream_launch<16, true>(a, split_k, k_waves, counters, stream);
    }
}

}  // namespace awq
