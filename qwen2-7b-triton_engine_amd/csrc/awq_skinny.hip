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
// block, rows >= M read as zeros (buffer out-of-range).
//
// Two ways to apply the scale (template flag FACTORED):
//  * factored (M <= 32): the column scale multiplies the fp32 group sum
//    sum_k x*(q - z) once per chunk; the unpack is 20 VALU ops per 16
//    weights.  Needs a second set of accumulators for the group sum.
//  * per weight (M <= 64): w = (q - z)*s is formed in fp16 as in the
//    reference and the MFMAs accumulate straight into the totals, which
//    leaves room in the register file for 4 row blocks.
// Both fold the 16x of kpairs_magic_x16's columns 2, 3, 6, 7 back into the
// fp32 result (an exact power-of-two scaling).
//
// Workgroup = 2 adjacent column tiles x KW consecutive K ranges (2*KW
// waves).  The two tiles of a pair read the two 64-byte halves of the same
// 128-byte qweight lines at the same time on the same CU.  The KW partial
// sums of each tile are added through LDS, so only one partial per
// workgroup leaves the CU.  With more than one workgroup along K (split_k >
// 1) the partials go to an fp32 workspace [split, M, N] and
// awq_splitk_reduce_kernel adds them in split order (deterministic).
//
// Loads run one chunk (up to 4 k-steps = one group) ahead of the MFMAs.
// Every load is unconditional -- the last prefetch re-reads the last chunk --
// so the compiler's wait counts never have to drain the prefetch early.
#include "awq_kernels.h"

namespace awq {

template <int MB, int CH, bool FACTORED>
__global__ __launch_bounds__(512) void awq_skinny_kernel(GemmArgs a, int rows_per_wave, int kw_count,
                                                         int split_k) {
    extern __shared__ float red[];
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
    const int nchunks = k_len / (32 * CH);

    floatx4 tot[MB][8];
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int c = 0; c < 8; ++c) tot[b][c] = floatx4{0.f, 0.f, 0.f, 0.f};

    if (nchunks > 0 && ct < n_ct) {
        const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.qweight, (uint32_t)((size_t)a.K * pn * 4));
        const __amdgpu_buffer_rsrc_t rz = make_rsrc(a.qzeros, (uint32_t)((size_t)(a.K / kGroup) * pn * 4));
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.scales, (uint32_t)((size_t)(a.K / kGroup) * a.N * 2));
        const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, (uint32_t)((size_t)a.M * a.K * 2));
        const uint32_t voff_w = (uint32_t)((8 * kq * pn + jc) * 4);
        uint32_t voff_x[MB];
#pragma unroll
        for (int b = 0; b < MB; ++b) voff_x[b] = (uint32_t)(((16 * b + c16) * a.K + 8 * kq) * 2);
        const uint32_t row_bytes = (uint32_t)pn * 4u;

        // Two chunk buffers used in turn (no register copies between them).
        uint32_t wA[CH][8], wB[CH][8];
        half8_t xA[CH][MB], xB[CH][MB];
        uint32_t zA, zB;
        half8_t sA, sB;

        auto load_chunk = [&](int chunk, uint32_t (&wv)[CH][8], half8_t (&xv)[CH][MB], uint32_t& z,
                              half8_t& s) {
            const int kb = k_begin + chunk * 32 * CH;
#pragma unroll
            for (int st = 0; st < CH; ++st)
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    wv[st][i] = buf_load_b32(rw, voff_w, (uint32_t)(kb + 32 * st + i) * row_bytes);
#pragma unroll
            for (int st = 0; st < CH; ++st)
#pragma unroll
                for (int b = 0; b < MB; ++b) xv[st][b] = buf_load_h8(rx, voff_x[b], (uint32_t)(kb + 32 * st) * 2u);
            const int g = kb / kGroup;
            z = buf_load_b32(rz, (uint32_t)jc * 4u, (uint32_t)g * row_bytes);
            s = buf_load_h8(rs, (uint32_t)jc * 16u, (uint32_t)g * (uint32_t)a.N * 2u);
        };

        auto compute_chunk = [&](const uint32_t (&w)[CH][8], const half8_t (&xf)[CH][MB], uint32_t zw,
                                 half8_t s8) {
            uint32_t zs[8];
            uint32_t ss[8];
            float sf[8];
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                zs[c] = zero_splat_x16(zw, c);
                if (FACTORED) sf[c] = (float)s8[c] * (x16_column(c) ? 0.0625f : 1.0f);
                else ss[c] = as_u32(half2_t{s8[c], s8[c]});
            }
            floatx4 acc[FACTORED ? MB : 1][8];
#pragma unroll
            for (int st = 0; st < CH; ++st) {
                u32x4 bf[8];
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    uint32_t kp[8];
                    kpairs_magic_x16(w[st][2 * p], w[st][2 * p + 1], kp);
#pragma unroll
                    for (int c = 0; c < 8; ++c) {
                        const half2_t d = as_h2(kp[c]) - as_h2(zs[c]);
                        bf[c][p] = FACTORED ? as_u32(d) : as_u32(d * as_h2(ss[c]));
                    }
                }
#pragma unroll
                for (int b = 0; b < MB; ++b)
#pragma unroll
                    for (int c = 0; c < 8; ++c) {
                        const half8_t bc = __builtin_bit_cast(half8_t, bf[c]);
                        if (FACTORED)
                            acc[b][c] = mfma16x16x32(xf[st][b], bc,
                                                     st == 0 ? floatx4{0.f, 0.f, 0.f, 0.f} : acc[b][c]);
                        else
                            tot[b][c] = mfma16x16x32(xf[st][b], bc, tot[b][c]);
                    }
            }
            if (FACTORED) {
#pragma unroll
                for (int b = 0; b < MB; ++b)
#pragma unroll
                    for (int c = 0; c < 8; ++c) tot[b][c] += acc[b][c] * sf[c];
            }
        };

        // Software pipeline, one chunk ahead.  Each load is issued
        // unconditionally (past the end it re-reads the last chunk), so the
        // wait before a chunk's MFMAs covers that chunk's loads only.
        // sched_barrier keeps the scheduler from sinking the prefetch below
        // the MFMAs (it would, to shorten register live ranges).
        const int last = nchunks - 1;
        load_chunk(0, wA, xA, zA, sA);
        for (int chunk = 0; chunk < nchunks; chunk += 2) {
            load_chunk(min(chunk + 1, last), wB, xB, zB, sB);
            __builtin_amdgcn_sched_barrier(0);
            compute_chunk(wA, xA, zA, sA);
            load_chunk(min(chunk + 2, last), wA, xA, zA, sA);
            __builtin_amdgcn_sched_barrier(0);
            if (chunk + 1 < nchunks) compute_chunk(wB, xB, zB, sB);
        }
    }

    if (!FACTORED) {
#pragma unroll
        for (int b = 0; b < MB; ++b)
#pragma unroll
            for (int c = 0; c < 8; ++c)
                if (x16_column(c)) tot[b][c] *= 0.0625f;
    }

    // Lane holds rows m = 16b + 4kq + ii of columns 8j .. 8j+7 (contiguous).
    const int mv = min(a.M, 16 * MB);
    if (kw_count > 1) {
        if (kw > 0) {
            float* slot = red + (size_t)((kw - 1) * 2 + ctl) * mv * kSkinnyCols;
#pragma unroll
            for (int b = 0; b < MB; ++b)
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
                    const int m = 16 * b + 4 * kq + ii;
                    if (m >= mv) continue;
                    floatx4* d = reinterpret_cast<floatx4*>(slot + m * kSkinnyCols + 8 * c16);
                    d[0] = floatx4{tot[b][0][ii], tot[b][1][ii], tot[b][2][ii], tot[b][3][ii]};
                    d[1] = floatx4{tot[b][4][ii], tot[b][5][ii], tot[b][6][ii], tot[b][7][ii]};
                }
        }
        __syncthreads();
        if (kw == 0) {
            for (int q = 1; q < kw_count; ++q) {
                const float* slot = red + (size_t)((q - 1) * 2 + ctl) * mv * kSkinnyCols;
#pragma unroll
                for (int b = 0; b < MB; ++b)
#pragma unroll
                    for (int ii = 0; ii < 4; ++ii) {
                        const int m = 16 * b + 4 * kq + ii;
                        if (m >= mv) continue;
                        const floatx4* s = reinterpret_cast<const floatx4*>(slot + m * kSkinnyCols + 8 * c16);
                        const floatx4 v0 = s[0], v1 = s[1];
                        tot[b][0][ii] += v0[0];
                        tot[b][1][ii] += v0[1];
                        tot[b][2][ii] += v0[2];
                        tot[b][3][ii] += v0[3];
                        tot[b][4][ii] += v1[0];
                        tot[b][5][ii] += v1[1];
                        tot[b][6][ii] += v1[2];
                        tot[b][7][ii] += v1[3];
                    }
            }
        }
    }
    if (kw != 0 || !col_ok) return;
#pragma unroll
    for (int b = 0; b < MB; ++b) {
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            const int m = 16 * b + 4 * kq + ii;
            if (m >= a.M) continue;
            if (split_k == 1) {
                half8_t h;
#pragma unroll
                for (int c = 0; c < 8; ++c) h[c] = (half_t)tot[b][c][ii];
                *reinterpret_cast<half8_t*>(a.out + (size_t)m * a.N + 8 * j) = h;
            } else {
                float* dst = a.partials + ((size_t)split * a.M + m) * a.N + 8 * j;
                reinterpret_cast<floatx4*>(dst)[0] =
                    floatx4{tot[b][0][ii], tot[b][1][ii], tot[b][2][ii], tot[b][3][ii]};
                reinterpret_cast<floatx4*>(dst)[1] =
                    floatx4{tot[b][4][ii], tot[b][5][ii], tot[b][6][ii], tot[b][7][ii]};
            }
        }
    }
}

__global__ __launch_bounds__(256) void awq_splitk_reduce_kernel(const float* __restrict__ partials,
                                                                half_t* __restrict__ out,
                                                                int64_t mn, int split_k) {
    const int64_t i4 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (i4 >= mn) return;
    floatx4 s = *reinterpret_cast<const floatx4*>(partials + i4);
    for (int k = 1; k < split_k; ++k) s += *reinterpret_cast<const floatx4*>(partials + (int64_t)k * mn + i4);
    const half4_t h = {(half_t)s[0], (half_t)s[1], (half_t)s[2], (half_t)s[3]};
    *reinterpret_cast<half4_t*>(out + i4) = h;
}

size_t skinny_lds_bytes(int M, int m_blocks, int kw_count) {
    const int mv = M < 16 * m_blocks ? M : 16 * m_blocks;
    return kw_count > 1 ? (size_t)(kw_count - 1) * 2 * mv * kSkinnyCols * sizeof(float) : 0;
}

int64_t skinny_blocks(int N, int K, int rows_per_wave, int kw_count) {
    const int64_t n_ct = (N + kSkinnyCols - 1) / kSkinnyCols;
    const int64_t n_pairs = (n_ct + 1) / 2;
    const int64_t rows_per_block = (int64_t)rows_per_wave * kw_count;
    return n_pairs * ((K + rows_per_block - 1) / rows_per_block);
}

// Chunk length (k-steps per prefetch) for MB row blocks: as long as the
// register file allows (two chunks of weights and x are live at once).
int skinny_chunk_steps(int m_blocks, int rows_per_wave) {
    const int max_ch = m_blocks == 1 ? 4 : (m_blocks == 2 ? 2 : 1);
    const int ch = rows_per_wave >= 128 ? 4 : rows_per_wave / 32;
    return ch < max_ch ? ch : max_ch;
}

template <int MB, int CH, bool F>
static hipError_t launch_one(const GemmArgs& a, const SkinnyConfig& cfg, dim3 grid, dim3 block, size_t lds,
                             hipStream_t stream) {
    hipLaunchKernelGGL((awq_skinny_kernel<MB, CH, F>), grid, block, lds, stream, a, cfg.rows_per_wave,
                       cfg.kw_count, cfg.split_k);
    return hipGetLastError();
}

hipError_t launch_skinny(const GemmArgs& a, const SkinnyConfig& cfg, hipStream_t stream) {
    const int64_t blocks = skinny_blocks(a.N, a.K, cfg.rows_per_wave, cfg.kw_count);
    const dim3 grid((unsigned)blocks), block(128 * cfg.kw_count);
    const size_t lds = skinny_lds_bytes(a.M, cfg.m_blocks, cfg.kw_count);
    const int ch = skinny_chunk_steps(cfg.m_blocks, cfg.rows_per_wave);
    if (cfg.m_blocks == 1) {
        if (ch == 1) return launch_one<1, 1, true>(a, cfg, grid, block, lds, stream);
        if (ch == 2) return launch_one<1, 2, true>(a, cfg, grid, block, lds, stream);
        if (ch == 4) return launch_one<1, 4, true>(a, cfg, grid, block, lds, stream);
    } else if (cfg.m_blocks == 2) {
        if (ch == 1) return launch_one<2, 1, true>(a, cfg, grid, block, lds, stream);
        if (ch == 2) return launch_one<2, 2, true>(a, cfg, grid, block, lds, stream);
    } else if (cfg.m_blocks == 4) {
        if (ch == 1) return launch_one<4, 1, false>(a, cfg, grid, block, lds, stream);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_splitk_reduce(const float* partials, half_t* out, int64_t mn, int split_k,
                                hipStream_t stream) {
    if (mn == 0) return hipSuccess;
    const int64_t threads = (mn + 3) / 4;
    const unsigned blocks = (unsigned)((threads + 255) / 256);
    hipLaunchKernelGGL(awq_splitk_reduce_kernel, dim3(blocks), dim3(256), 0, stream, partials, out, mn, split_k);
    return hipGetLastError();
}

}  // namespace awq
