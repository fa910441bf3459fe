// Decode / skinny-M W4A16 AWQ GEMM (M <= 64) for gfx950.
//
// The weight stream is the whole cost at small M, so each qweight word is
// read from HBM exactly once, straight into registers, never staged in LDS.
//
// Wave = 128 output columns (16 packed columns) x `rows_per_wave` K rows:
//   lane l: c16 = l % 16 picks packed column j = 16*tile + c16,
//           kq  = l / 16 picks rows 8*kq .. 8*kq+7 of each 32-row k-step.
// That is the B-operand layout of v_mfma_f32_16x16x32_f16 (a lane holds 8
// consecutive k of one column), so the 8 words a lane loads per k-step turn
// into 8 B fragments -- one per logical column of the packed word -- after
// the in-register unpack (v_perm_b32 row pairing, fp16 magic-number decode,
// exact fp16 zero subtraction).  Rows of x are the A operand, 16 per MFMA
// block; rows >= M read as zeros (buffer out-of-range).
//
// Two ways to apply the scale (template flag FACTORED):
//  * factored: the column scale multiplies the fp32 group sum
//    sum_k x*(q - z) once per group; the unpack is 20 VALU ops per 16
//    weights but needs a second accumulator set for the group sum.
//  * per weight: w = (q - z)*s is formed in fp16 as in the reference and the
//    MFMAs accumulate straight into the totals (28 VALU ops per 16 weights,
//    fewer registers).
// Both read the codes with kpairs_magic_inplace, whose columns 2, 3, 6, 7
// carry the offset 64 instead of 1024; the matching zero splat makes q - z
// exact either way.
//
// Main loop variants:
//  1  chunked software pipeline: the loads of the next group (4 k-steps) are
//     issued before the MFMAs of the current one (two register buffers);
//  2  plain loop over k-steps; latency is hidden by occupancy (more waves
//     per SIMD thanks to the smaller register footprint).
//
// Workgroup = 2 adjacent column tiles x KW consecutive K ranges (2*KW
// waves).  The two tiles of a pair read the two 64-byte halves of the same
// 128-byte qweight lines at the same time on the same CU.  The KW partial
// sums of each tile are added through LDS.  With several workgroups along K
// (split_k > 1) each writes its fp32 partial [split, M, 256 columns] to the
// workspace and bumps the pair's arrival counter; the last workgroup to
// arrive adds the partials in split order (deterministic), writes the fp16
// output and resets the counter to zero, so one launch does the whole GEMM.
#include "awq_kernels.h"

namespace awq {

template <int MB, bool FACTORED, int VARIANT>
__global__ __launch_bounds__(512) void awq_skinny_kernel(GemmArgs a, int rows_per_wave, int kw_count,
                                                         int split_k, uint32_t* counters) {
    extern __shared__ float red[];
    __shared__ int last_flag;
    __shared__ floatx4 fin[512];
    const int lane = threadIdx.x & 63;
    // Wave-uniform by construction; readfirstlane lets the compiler keep the
    // K offsets derived from it in SGPRs (buffer-load soffset).
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ctl = wave & 1;
    const int kw = wave >> 1;
    const int c16 = lane & 15;
    const int kq = lane >> 4;

    const int n_ct = (a.N + kSkinnyCols - 1) / kSkinnyCols;
    const int n_pairs = (n_ct + 1) >> 1;
    const int pair = blockIdx.x % n_pairs;
    const int split = blockIdx.x / n_pairs;
    const int ct = 2 * pair + ctl;
    const int pn = a.N >> 3;
    const int j = ct * 16 + c16;
    const bool col_ok = j < pn;
    const int jc = col_ok ? j : pn - 1;  // in-bounds address; results of such lanes are dropped

    const int k_begin = (split * kw_count + kw) * rows_per_wave;
    const int k_len = max(0, min(a.K, k_begin + rows_per_wave) - k_begin);

    floatx4 tot[MB][8];
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int c = 0; c < 8; ++c) tot[b][c] = floatx4{0.f, 0.f, 0.f, 0.f};

    if (k_len > 0 && ct < n_ct) {
        const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.qweight, (uint32_t)((size_t)a.K * pn * 4));
        const __amdgpu_buffer_rsrc_t rz = make_rsrc(a.qzeros, (uint32_t)((size_t)(a.K / kGroup) * pn * 4));
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.scales, (uint32_t)((size_t)(a.K / kGroup) * a.N * 2));
        const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (uint32_t)((size_t)a.M * a.K * 2));
        const uint32_t voff_w = (uint32_t)((8 * kq * pn + jc) * 4);
        uint32_t voff_x[MB];
#pragma unroll
        for (int b = 0; b < MB; ++b) voff_x[b] = (uint32_t)(((16 * b + c16) * a.K + 8 * kq) * 2);
        const uint32_t row_bytes = (uint32_t)pn * 4u;

        // Splats of one group's zero and scale for this lane's 8 columns.
        auto group_consts = [&](uint32_t zw, half8_t s8, uint32_t (&zs)[8], uint32_t (&ss)[8], float (&sf)[8]) {
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                zs[c] = zero_splat_inplace(zw, c);
                if (FACTORED) sf[c] = (float)s8[c];
                else ss[c] = as_u32(half2_t{s8[c], s8[c]});
            }
        };
        // One 32-row k-step: unpack 8 words into 8 B fragments, MFMA with x.
        auto kstep = [&](const uint32_t (&w)[8], const half8_t (&xf)[MB], const uint32_t (&zs)[8],
                         const uint32_t (&ss)[8], floatx4 (&dst)[MB][8], bool first) {
            u32x4 bf[8];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                uint32_t kp[8];
                kpairs_magic_inplace(w[2 * p], w[2 * p + 1], kp);
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    const half2_t d = as_h2(kp[c]) - as_h2(zs[c]);
                    bf[c][p] = FACTORED ? as_u32(d) : as_u32(d * as_h2(ss[c]));
                }
            }
#pragma unroll
            for (int b = 0; b < MB; ++b)
#pragma unroll
                for (int c = 0; c < 8; ++c)
                    dst[b][c] = mfma16x16x32(xf[b], __builtin_bit_cast(half8_t, bf[c]),
                                             first ? floatx4{0.f, 0.f, 0.f, 0.f} : dst[b][c]);
        };
        auto load_step = [&](int kb, uint32_t (&w)[8], half8_t (&xf)[MB]) {
#pragma unroll
            for (int i = 0; i < 8; ++i) w[i] = buf_load_b32(rw, voff_w, (uint32_t)(kb + i) * row_bytes);
#pragma unroll
            for (int b = 0; b < MB; ++b) xf[b] = buf_load_h8(rx, voff_x[b], (uint32_t)kb * 2u);
        };

        if (VARIANT == 2) {
            // Group by group; inside a group, one k-step at a time.
            for (int g0 = k_begin; g0 < k_begin + k_len;) {
                const int g = g0 / kGroup;
                const int g_end = min(k_begin + k_len, (g + 1) * kGroup);
                uint32_t zs[8], ss[8];
                float sf[8];
                const uint32_t zw = buf_load_b32(rz, (uint32_t)jc * 4u, (uint32_t)g * row_bytes);
                const half8_t s8 = buf_load_h8(rs, (uint32_t)jc * 16u, (uint32_t)g * (uint32_t)a.N * 2u);
                group_consts(zw, s8, zs, ss, sf);
                floatx4 acc[MB][8];  // group sums (factored mode only)
#pragma unroll 1
                for (int kb = g0; kb < g_end; kb += 32) {
                    uint32_t w[8];
                    half8_t xf[MB];
                    load_step(kb, w, xf);
                    if constexpr (FACTORED) kstep(w, xf, zs, ss, acc, kb == g0);
                    else kstep(w, xf, zs, ss, tot, false);
                }
                if (FACTORED) {
#pragma unroll
                    for (int b = 0; b < MB; ++b)
#pragma unroll
                        for (int c = 0; c < 8; ++c) tot[b][c] += acc[b][c] * sf[c];
                }
                g0 = g_end;
            }
        } else {
            // Chunks of up to 4 k-steps inside one group, one chunk ahead.
            constexpr int CH = 4;
            const int nchunks = (k_len + 32 * CH - 1) / (32 * CH);
            const int last = nchunks - 1;
            uint32_t wA[CH][8], wB[CH][8];
            half8_t xA[CH][MB], xB[CH][MB];
            uint32_t zA, zB;
            half8_t sA, sB;
            auto steps_in = [&](int chunk) { return min(CH, (k_len - chunk * 32 * CH) / 32); };
            auto load_chunk = [&](int chunk, uint32_t (&wv)[CH][8], half8_t (&xv)[CH][MB], uint32_t& z,
                                  half8_t& s) {
                const int kb = k_begin + chunk * 32 * CH;
                const int ns = steps_in(chunk);
#pragma unroll
                for (int st = 0; st < CH; ++st) load_step(kb + 32 * min(st, ns - 1), wv[st], xv[st]);
                const int g = kb / kGroup;
                z = buf_load_b32(rz, (uint32_t)jc * 4u, (uint32_t)g * row_bytes);
                s = buf_load_h8(rs, (uint32_t)jc * 16u, (uint32_t)g * (uint32_t)a.N * 2u);
            };
            auto compute_chunk = [&](int chunk, const uint32_t (&wv)[CH][8], const half8_t (&xv)[CH][MB],
                                     uint32_t z, half8_t s) {
                uint32_t zs[8], ss[8];
                float sf[8];
                group_consts(z, s, zs, ss, sf);
                const int ns = steps_in(chunk);
                floatx4 acc[MB][8];  // group sums (factored mode only)
#pragma unroll
                for (int st = 0; st < CH; ++st) {
                    if (st < ns) {
                        if constexpr (FACTORED) kstep(wv[st], xv[st], zs, ss, acc, st == 0);
                        else kstep(wv[st], xv[st], zs, ss, tot, false);
                    }
                }
                if (FACTORED) {
#pragma unroll
                    for (int b = 0; b < MB; ++b)
#pragma unroll
                        for (int c = 0; c < 8; ++c) tot[b][c] += acc[b][c] * sf[c];
                }
            };
            // Each load is issued unconditionally (past the end it re-reads
            // the last chunk), so the wait before a chunk's MFMAs covers that
            // chunk's loads only; sched_barrier keeps the scheduler from
            // sinking the prefetch below the MFMAs.
            load_chunk(0, wA, xA, zA, sA);
            for (int chunk = 0; chunk < nchunks; chunk += 2) {
                load_chunk(min(chunk + 1, last), wB, xB, zB, sB);
                __builtin_amdgcn_sched_barrier(0);
                compute_chunk(chunk, wA, xA, zA, sA);
                load_chunk(min(chunk + 2, last), wA, xA, zA, sA);
                __builtin_amdgcn_sched_barrier(0);
                if (chunk + 1 < nchunks) compute_chunk(chunk + 1, wB, xB, zB, sB);
            }
        }
    }

    // Lane holds rows m = 16b + 4kq + ii of columns 8j .. 8j+7 (contiguous).
    // K reduction inside the workgroup: waves kw > 0 park their totals in LDS
    // as [slot][b][c][lane] float4 (each store covers 64 consecutive float4:
    // no bank conflicts), wave kw == 0 adds them.  Rows >= M hold exact zeros
    // (their x rows read as zeros), so every lane takes part, branch-free.
    if (kw_count > 1) {
        if (kw > 0) {
            floatx4* slot = reinterpret_cast<floatx4*>(red) + (size_t)((kw - 1) * 2 + ctl) * MB * 8 * 64;
#pragma unroll
            for (int b = 0; b < MB; ++b)
#pragma unroll
                for (int c = 0; c < 8; ++c) slot[(b * 8 + c) * 64 + lane] = tot[b][c];
        }
        __syncthreads();
        if (kw == 0) {
            for (int q = 1; q < kw_count; ++q) {
                const floatx4* slot = reinterpret_cast<const floatx4*>(red) + (size_t)((q - 1) * 2 + ctl) * MB * 8 * 64;
#pragma unroll
                for (int b = 0; b < MB; ++b)
#pragma unroll
                    for (int c = 0; c < 8; ++c) tot[b][c] += slot[(b * 8 + c) * 64 + lane];
            }
        }
    }

    if (split_k == 1) {
        if (kw != 0 || !col_ok) return;
#pragma unroll
        for (int b = 0; b < MB; ++b)
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                const int m = 16 * b + 4 * kq + ii;
                if (m >= a.M) continue;
                float y[8];
#pragma unroll
                for (int c = 0; c < 8; ++c) y[c] = tot[b][c][ii];
                store_out<8>(a.out, a.bias, a.residual, a.N, m, 8 * j, y);
            }
        return;
    }

    // Split-K: partial [split][M][N] fp32, then the last workgroup of the pair
    // reduces.  The partials are written and read with device-scope (sc1)
    // buffer operations, which go through to the coherence point shared by
    // all XCDs; waiting for the stores' completion before the arrival atomic
    // then orders them for the last workgroup without the L2-wide writeback
    // and invalidate that a __threadfence() costs on a multi-XCD device.
    const uint32_t part_bytes = (uint32_t)((size_t)split_k * a.M * a.N * 4);
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(a.partials, part_bytes);
    if (kw == 0 && col_ok) {
#pragma unroll
        for (int b = 0; b < MB; ++b)
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                const int m = 16 * b + 4 * kq + ii;
                if (m >= a.M) continue;
                const uint32_t off = (uint32_t)((((size_t)split * a.M + m) * a.N + 8 * j) * 4);
                buf_store_f4_device(floatx4{tot[b][0][ii], tot[b][1][ii], tot[b][2][ii], tot[b][3][ii]}, rp, off);
                buf_store_f4_device(floatx4{tot[b][4][ii], tot[b][5][ii], tot[b][6][ii], tot[b][7][ii]}, rp,
                                    off + 16);
            }
    }
    wait_vm_stores();
    __syncthreads();
    if (threadIdx.x == 0)
        last_flag = __hip_atomic_fetch_add(&counters[pair], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                    (uint32_t)(split_k - 1);
    __syncthreads();
    if (!last_flag) return;
    splitk_finish<4>(rp, a.out, a.bias, a.residual, a.M, a.N, 0, a.M, pair * 2 * kSkinnyCols, min(2 * kSkinnyCols, a.N - pair * 2 * kSkinnyCols),
                  split_k, fin);
    if (threadIdx.x == 0) __hip_atomic_store(&counters[pair], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

size_t skinny_lds_bytes(int /*M*/, int m_blocks, int kw_count) {
    // (kw_count - 1) parked waves per column tile, 2 tiles, MB*8 float4 per lane.
    return kw_count > 1 ? (size_t)(kw_count - 1) * 2 * m_blocks * 8 * 64 * 16 : 0;
}

int64_t skinny_pairs(int N) {
    const int64_t n_ct = (N + kSkinnyCols - 1) / kSkinnyCols;
    return (n_ct + 1) / 2;
}

int64_t skinny_blocks(int N, int K, int rows_per_wave, int kw_count) {
    const int64_t rows_per_block = (int64_t)rows_per_wave * kw_count;
    return skinny_pairs(N) * ((K + rows_per_block - 1) / rows_per_block);
}

size_t skinny_counter_bytes() { return kCounterBytes; }

template <int MB, bool F, int V>
static hipError_t launch_one(const GemmArgs& a, const SkinnyConfig& cfg, dim3 grid, dim3 block, size_t lds,
                             uint32_t* counters, hipStream_t stream) {
    hipLaunchKernelGGL((awq_skinny_kernel<MB, F, V>), grid, block, lds, stream, a, cfg.rows_per_wave, cfg.kw_count,
                       cfg.split_k, counters);
    return hipGetLastError();
}

hipError_t launch_skinny(const GemmArgs& a, const SkinnyConfig& cfg, uint32_t* counters, hipStream_t stream) {
    const int64_t blocks = skinny_blocks(a.N, a.K, cfg.rows_per_wave, cfg.kw_count);
    const dim3 grid((unsigned)blocks), block(128 * cfg.kw_count);
    const size_t lds = skinny_lds_bytes(a.M, cfg.m_blocks, cfg.kw_count);
    const int key = cfg.m_blocks * 100 + (cfg.factored ? 10 : 0) + cfg.variant;
    switch (key) {
        case 111: return launch_one<1, true, 1>(a, cfg, grid, block, lds, counters, stream);
        case 112: return launch_one<1, true, 2>(a, cfg, grid, block, lds, counters, stream);
        case 101: return launch_one<1, false, 1>(a, cfg, grid, block, lds, counters, stream);
        case 102: return launch_one<1, false, 2>(a, cfg, grid, block, lds, counters, stream);
        case 212: return launch_one<2, true, 2>(a, cfg, grid, block, lds, counters, stream);
        case 202: return launch_one<2, false, 2>(a, cfg, grid, block, lds, counters, stream);
        case 402: return launch_one<4, false, 2>(a, cfg, grid, block, lds, counters, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace awq
