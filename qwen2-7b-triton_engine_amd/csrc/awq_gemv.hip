// Decode GEMV (M <= 2) of the W4A16 AWQ GEMM for gfx950.
//
// At batch 1 the kernel is a pure stream of the int4 weights, and the time
// is set by how many bytes are in flight against the HBM latency.  So:
//
// * lane l of a wave owns one packed column j = 64*strip + l (8 output
//   columns), and the wave reads whole 256-byte row segments (64 lanes x one
//   dword of the same row), rows r0 .. r0+R-1 of its K range;
// * all R loads of a wave are issued at once, before any arithmetic, and a
//   wave is small (about 70 VGPRs), so many waves per SIMD keep the HBM queue
//   full;
// * no MFMA: with one or two rows of x the 16x16 MFMA tile would be mostly
//   padding.  Each pair of rows (r, r+1) of a packed column is turned into
//   fp16 k-pairs (v_perm_b32 + magic-number decode, see awq_device.h), the
//   zero is subtracted exactly in fp16 and v_dot2_f32_f16 accumulates
//   x[r]*(q[r]-z) + x[r+1]*(q[r+1]-z) in fp32;
// * x is uniform across the wave: its row pairs are read with scalar loads
//   into SGPRs, the second dot2 operand;
// * a wave covers R rows of one 128-row group, so the scale multiplies its
//   fp32 sum once at the end.
//
// Workgroup = KW waves on the same strip and consecutive K ranges; their
// sums are added through LDS.  Several workgroups along K (split_k > 1)
// finish in one launch exactly as the skinny kernel does: device-scope
// partials [split, M, N], an arrival counter per strip, the last workgroup
// adds the partials in split order and resets the counter.
#include "awq_kernels.h"

namespace awq {

template <int MR, int R>
__global__ __launch_bounds__(512) void awq_gemv_kernel(GemmArgs a, int kw_count, int split_k,
                                                       uint32_t* counters) {
    __shared__ float red[7 * MR * 8 * 64];
    __shared__ int last_flag;
    __shared__ floatx4 fin[512];
    const int lane = threadIdx.x & 63;
    const int kw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int pn = a.N >> 3;
    const int n_strips = (pn + 63) / 64;
    const int strip = blockIdx.x % n_strips;
    const int split = blockIdx.x / n_strips;
    const int j = strip * 64 + lane;
    const bool col_ok = j < pn;
    const int jc = col_ok ? j : pn - 1;
    const int r0 = (split * kw_count + kw) * R;
    const bool active = r0 < a.K;  // wave-uniform

    float acc[MR][8];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[m][c] = 0.f;

    if (active) {
        const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.qweight, (uint32_t)((size_t)a.K * pn * 4));
        const uint32_t row_bytes = (uint32_t)pn * 4u;
        const uint32_t voff = (uint32_t)jc * 4u;
        uint32_t w[R];
#pragma unroll
        for (int i = 0; i < R; ++i) w[i] = buf_load_b32(rw, voff, (uint32_t)(r0 + i) * row_bytes);
        const int g = r0 / kGroup;
        const uint32_t zw = a.qzeros[(size_t)g * pn + jc];
        const half8_t s8 = *reinterpret_cast<const half8_t*>(a.scales + (size_t)g * a.N + 8 * jc);
        // x row pairs (x[r], x[r+1]) as fp16 pairs; the index is wave-uniform.
        const uint32_t* x32 = reinterpret_cast<const uint32_t*>(a.x);
        uint32_t xp[MR][R / 2];
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int p = 0; p < R / 2; ++p)
                xp[m][p] = __builtin_amdgcn_readfirstlane(x32[((size_t)m * a.K + r0) / 2 + p]);
        uint32_t zs[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) zs[c] = zero_splat_x16(zw, c);
#pragma unroll
        for (int p = 0; p < R / 2; ++p) {
            uint32_t kp[8];
            kpairs_magic_x16(w[2 * p], w[2 * p + 1], kp);
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const half2_t d = as_h2(kp[c]) - as_h2(zs[c]);
#pragma unroll
                for (int m = 0; m < MR; ++m)
                    acc[m][c] = __builtin_amdgcn_fdot2(d, as_h2(xp[m][p]), acc[m][c], false);
            }
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const float sc = (float)s8[c] * (x16_column(c) ? 0.0625f : 1.0f);
#pragma unroll
            for (int m = 0; m < MR; ++m) acc[m][c] *= sc;
        }
    }

    // K reduction inside the workgroup through LDS ([wave][m][c][lane]).
    if (kw_count > 1) {
        if (kw > 0) {
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int c = 0; c < 8; ++c) red[(((kw - 1) * MR + m) * 8 + c) * 64 + lane] = acc[m][c];
        }
        __syncthreads();
        if (kw == 0) {
            for (int q = 1; q < kw_count; ++q)
#pragma unroll
                for (int m = 0; m < MR; ++m)
#pragma unroll
                    for (int c = 0; c < 8; ++c) acc[m][c] += red[(((q - 1) * MR + m) * 8 + c) * 64 + lane];
        }
    }

    if (split_k == 1) {
        if (kw != 0 || !col_ok) return;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            if (m >= a.M) break;
            half8_t h;
#pragma unroll
            for (int c = 0; c < 8; ++c) h[c] = (half_t)acc[m][c];
            *reinterpret_cast<half8_t*>(a.out + (size_t)m * a.N + 8 * j) = h;
        }
        return;
    }

    const uint32_t part_bytes = (uint32_t)((size_t)split_k * a.M * a.N * 4);
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(a.partials, part_bytes);
    if (kw == 0 && col_ok) {
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
    splitk_finish<2>(rp, a.out, a.M, a.N, 0, a.M, strip * 512, min(512, a.N - strip * 512), split_k, fin);
    if (threadIdx.x == 0) __hip_atomic_store(&counters[strip], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

int64_t gemv_strips(int N) { return ((N >> 3) + 63) / 64; }

int64_t gemv_blocks(int N, int K, int rows_per_wave, int kw_count) {
    const int64_t rows_per_block = (int64_t)rows_per_wave * kw_count;
    return gemv_strips(N) * ((K + rows_per_block - 1) / rows_per_block);
}

template <int MR, int R>
static hipError_t gemv_launch(const GemmArgs& a, const GemvConfig& cfg, uint32_t* counters, hipStream_t stream) {
    const dim3 grid((unsigned)gemv_blocks(a.N, a.K, R, cfg.kw_count)), block(64 * cfg.kw_count);
    hipLaunchKernelGGL((awq_gemv_kernel<MR, R>), grid, block, 0, stream, a, cfg.kw_count, cfg.split_k, counters);
    return hipGetLastError();
}

hipError_t launch_gemv(const GemmArgs& a, const GemvConfig& cfg, uint32_t* counters, hipStream_t stream) {
    const int key = (a.M <= 1 ? 1 : 2) * 1000 + cfg.rows_per_wave;
    switch (key) {
        case 1016: return gemv_launch<1, 16>(a, cfg, counters, stream);
        case 1032: return gemv_launch<1, 32>(a, cfg, counters, stream);
        case 1064: return gemv_launch<1, 64>(a, cfg, counters, stream);
        case 2016: return gemv_launch<2, 16>(a, cfg, counters, stream);
        case 2032: return gemv_launch<2, 32>(a, cfg, counters, stream);
        case 2064: return gemv_launch<2, 64>(a, cfg, counters, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace awq
