// Narrow-M W4A16 AWQ GEMM (M <= 16) for gfx950: the K-streaming GEMV's
// memory schedule with MFMA arithmetic.
//
// v_mfma_f32_4x4x4_16b_f16 computes 16 independent 4x4x4 products per wave.
// Lane l supplies, for block b = l / 4: A_b[i][k] (i = l % 4, k = 0..3) and
// B_b[k][j] (j = l % 4), and receives D_b[i][j] for i = 0..3.  So if every
// block takes the same 4 rows of x as A and lane l supplies 4 consecutive
// rows of one logical column c of its own packed column as B, the wave
// computes out[4mb + i][8l + c] for the 64 packed columns of the wave at
// once: exactly the GEMV lane layout (lane = packed column, one 256-byte row
// segment per load), which a 16x16 MFMA cannot use (its B fragment needs 8
// consecutive rows of one column spread over 4 lanes).
//
// Per 4 rows a lane turns its 4 words into the k-pairs of kpairs_magic
// (v_perm_b32 + magic-number decode) and issues 8 MFMAs per block of 4 rows
// of x (MB blocks: M <= 4 * MB).  Two ways to handle zero and scale:
//  * FACT (group-factored): B = 1024 + q (x16 for columns 2, 3, 6, 7), and
//    an extra MFMA with B = 1 gives sum_k x; at the end of each 128-row
//    group  tot += s * (acc - (1024 + z) * sum_k x),  so a weight costs only
//    its unpack (0.75 VALU op).  The fp32 sums carry the 1024 offset
//    (~10 bits of headroom); the weight is not rounded to fp16 first.
//  * per weight: B = fp16((q - z) * s) formed exactly as the reference
//    does (kernels/awq_gemm.py:59), accumulated straight into the totals.
//
// Schedule (as awq_gemv_stream_kernel): workgroup = KW = 128 / R waves on a
// 64-packed-column strip; chunk c = one 128-row group, wave w reads rows
// 128c + R*w .. +R-1; a ring of D chunks in flight with unconditional loads;
// the KW waves' totals are added through LDS in a fixed tree order; split-K
// across workgroups finishes in-kernel (device-scope partials, arrival
// counter, deterministic split-order sum).
#include "awq_kernels.h"

namespace awq {

namespace {
typedef _Float16 half4n_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma4x4x4(u32x2 a, u32x2 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(half4n_t, a), __builtin_bit_cast(half4n_t, b), c, 0,
                                              0, 0);
}
}  // namespace

template <int MB, int R, int D, bool FACT>
__global__ __launch_bounds__(512) void awq_narrow_kernel(GemmArgs a, int chunks_per_split, int split_k,
                                                         uint32_t* counters) {
    constexpr int KW = kGroup / R;
    constexpr int S4 = R / 4;        // 4-row MFMA steps per chunk
    constexpr int XQ = R / 8;        // 16-byte x loads per 4-row block per chunk
    constexpr int SLOTS = KW / 2;    // LDS slots of the first reduction round
    __shared__ floatx4 red[SLOTS * MB * 8 * 64];
    __shared__ int last_flag;
    floatx4* fin = red;              // split-K finish, after the reduction

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
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (uint32_t)((size_t)a.M * a.K * 2));
    const uint32_t row_bytes = (uint32_t)pn * 4u;
    const uint32_t voff = (uint32_t)jc * 4u;
    // x rows of this lane: 4mb + (lane & 3); rows >= M read as zeros (offset past the buffer).
    uint32_t xoff[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) xoff[mb] = (uint32_t)((4 * mb + (lane & 3)) * a.K * 2);

    floatx4 tot[MB][8];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int c = 0; c < 8; ++c) tot[mb][c] = floatx4{0.f, 0.f, 0.f, 0.f};

    struct Chunk {
        uint32_t w[R];
        u32x4 xq[MB][XQ];
        uint32_t zw;
        half8_t s8;
    };
    auto load = [&](int c, Chunk& ck) {
        const int r0 = c * kGroup + wave * R;
#pragma unroll
        for (int i = 0; i < R; ++i) ck.w[i] = buf_load_b32(rw, voff, (uint32_t)(r0 + i) * row_bytes);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int q = 0; q < XQ; ++q)
                ck.xq[mb][q] = __builtin_bit_cast(u32x4, buf_load_h8(rx, xoff[mb], (uint32_t)(r0 + 8 * q) * 2u));
        ck.zw = buf_load_b32(rz, voff, (uint32_t)c * row_bytes);
        ck.s8 = buf_load_h8(rs, (uint32_t)jc * 16u, (uint32_t)c * (uint32_t)a.N * 2u);
    };
    auto compute = [&](const Chunk& ck) {
        if constexpr (FACT) {
            const u32x2 ones = {0x3C003C00u, 0x3C003C00u};
            floatx4 acc[MB][8], sx[MB];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                sx[mb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int c = 0; c < 8; ++c) acc[mb][c] = floatx4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int s = 0; s < S4; ++s) {
                uint32_t k01[8], k23[8];
                kpairs_magic_x16(ck.w[4 * s], ck.w[4 * s + 1], k01);
                kpairs_magic_x16(ck.w[4 * s + 2], ck.w[4 * s + 3], k23);
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    const u32x4 xv = ck.xq[mb][s >> 1];
                    const u32x2 av = (s & 1) ? u32x2{xv[2], xv[3]} : u32x2{xv[0], xv[1]};
                    sx[mb] = mfma4x4x4(av, ones, sx[mb]);
#pragma unroll
                    for (int c = 0; c < 8; ++c) acc[mb][c] = mfma4x4x4(av, u32x2{k01[c], k23[c]}, acc[mb][c]);
                }
            }
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const uint32_t z = (ck.zw >> col_shift(c)) & 0xFu;
                const float zz = 1024.f + (float)(x16_column(c) ? 16u * z : z);
                const float sc = (float)ck.s8[c] * (x16_column(c) ? 0.0625f : 1.0f);
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) tot[mb][c] += sc * (acc[mb][c] - zz * sx[mb]);
            }
        } else {
            uint32_t zs[8], ss[8];
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                zs[c] = zero_splat(ck.zw, c);
                ss[c] = as_u32(half2_t{ck.s8[c], ck.s8[c]});
            }
#pragma unroll
            for (int s = 0; s < S4; ++s) {
                uint32_t k01[8], k23[8];
                kpairs_magic(ck.w[4 * s], ck.w[4 * s + 1], k01);
                kpairs_magic(ck.w[4 * s + 2], ck.w[4 * s + 3], k23);
                u32x2 bw[8];
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    // fp16((1024 + q) - (1024 + z)) = q - z exactly; one RNE rounding by the scale.
                    bw[c][0] = as_u32((as_h2(k01[c]) - as_h2(zs[c])) * as_h2(ss[c]));
                    bw[c][1] = as_u32((as_h2(k23[c]) - as_h2(zs[c])) * as_h2(ss[c]));
                }
#pragma unroll
                for (int mb = 0; mb < MB; ++mb) {
                    const u32x4 xv = ck.xq[mb][s >> 1];
                    const u32x2 av = (s & 1) ? u32x2{xv[2], xv[3]} : u32x2{xv[0], xv[1]};
#pragma unroll
                    for (int c = 0; c < 8; ++c) tot[mb][c] = mfma4x4x4(av, bw[c], tot[mb][c]);
                }
            }
        }
    };

    // Ring of D chunks; unconditional (clamped) loads keep the wait counts partial.
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

    // Tree reduction over the KW waves in a fixed order: in each round the
    // upper half of the remaining waves stores, the lower half adds.
#pragma unroll
    for (int half_w = KW / 2; half_w >= 1; half_w >>= 1) {
        if (wave >= half_w && wave < 2 * half_w) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int c = 0; c < 8; ++c) red[(((wave - half_w) * MB + mb) * 8 + c) * 64 + lane] = tot[mb][c];
        }
        __syncthreads();
        if (wave < half_w) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int c = 0; c < 8; ++c) tot[mb][c] += red[((wave * MB + mb) * 8 + c) * 64 + lane];
        }
        __syncthreads();
    }

    // tot[mb][c][i] = out[4mb + i][8j + c] (wave 0 holds the workgroup's sum).
    if (split_k == 1) {
        if (wave != 0 || !col_ok) return;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 4 * mb + i;
                if (m >= a.M) continue;
                float y[8];
#pragma unroll
                for (int c = 0; c < 8; ++c) y[c] = tot[mb][c][i];
                store_out<8>(a.out, a.bias, a.residual, a.N, m, 8 * j, y);
            }
        return;
    }

    const uint32_t part_bytes = (uint32_t)((size_t)split_k * a.M * a.N * 4);
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(a.partials, part_bytes);
    if (wave == 0 && col_ok) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = 4 * mb + i;
                if (m >= a.M) continue;
                const uint32_t off = (uint32_t)((((size_t)split * a.M + m) * a.N + 8 * j) * 4);
                buf_store_f4_device(floatx4{tot[mb][0][i], tot[mb][1][i], tot[mb][2][i], tot[mb][3][i]}, rp, off);
                buf_store_f4_device(floatx4{tot[mb][4][i], tot[mb][5][i], tot[mb][6][i], tot[mb][7][i]}, rp,
                                    off + 16);
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

template <int MB, int R, int D, bool FACT>
static hipError_t narrow_launch(const GemmArgs& a, const NarrowConfig& cfg, uint32_t* counters, hipStream_t stream) {
    const dim3 grid((unsigned)(gemv_strips(a.N) * cfg.split_k)), block(64 * (kGroup / R));
    hipLaunchKernelGGL((awq_narrow_kernel<MB, R, D, FACT>), grid, block, 0, stream, a, cfg.chunks_per_split,
                       cfg.split_k, counters);
    return hipGetLastError();
}

int narrow_blocks_for(int M) { return M <= 4 ? 1 : (M <= 8 ? 2 : 4); }

hipError_t launch_narrow(const GemmArgs& a, const NarrowConfig& cfg, uint32_t* counters, hipStream_t stream) {
    const int mb = narrow_blocks_for(a.M);
    const int key = mb * 1000 + cfg.rows_per_wave * 10 + cfg.depth + (cfg.factored ? 0 : 5);
    switch (key) {
        case 1162: return narrow_launch<1, 16, 2, true>(a, cfg, counters, stream);
        case 1163: return narrow_launch<1, 16, 3, true>(a, cfg, counters, stream);
        case 1322: return narrow_launch<1, 32, 2, true>(a, cfg, counters, stream);
        case 1167: return narrow_launch<1, 16, 2, false>(a, cfg, counters, stream);
        case 1168: return narrow_launch<1, 16, 3, false>(a, cfg, counters, stream);
        case 1327: return narrow_launch<1, 32, 2, false>(a, cfg, counters, stream);
        case 2162: return narrow_launch<2, 16, 2, true>(a, cfg, counters, stream);
        case 2163: return narrow_launch<2, 16, 3, true>(a, cfg, counters, stream);
        case 2322: return narrow_launch<2, 32, 2, true>(a, cfg, counters, stream);
        case 2167: return narrow_launch<2, 16, 2, false>(a, cfg, counters, stream);
        case 2168: return narrow_launch<2, 16, 3, false>(a, cfg, counters, stream);
        case 2327: return narrow_launch<2, 32, 2, false>(a, cfg, counters, stream);
        case 4167: return narrow_launch<4, 16, 2, false>(a, cfg, counters, stream);
        case 4168: return narrow_launch<4, 16, 3, false>(a, cfg, counters, stream);
        case 4327: return narrow_launch<4, 32, 2, false>(a, cfg, counters, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace awq
