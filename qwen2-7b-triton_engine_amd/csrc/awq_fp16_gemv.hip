// fp16 GEMV for the output projection: out[M, N] = x[M, K] @ weight[N, K]^T
// with fp32 accumulation and fp16 results -- the lm_head of
// model/qwen2.py:253,280 (nn.Linear(hidden, vocab, bias=False)) at decode
// sizes (M <= 8; greedy decoding needs the last position's logits only).
// HBM-bound: 152064 x 3584 fp16 = 1.09 GB per token for Qwen2-7B.
#include "awq_kernels.h"

namespace awq {
namespace {

constexpr int kF16Threads = 256;
constexpr int kF16MaxK = 4096;

// v_mfma_f32_16x16x32_f16 takes its A operand as 8 consecutive
// k of row l % 16 in k-block l / 16 of each lane l: for a row-major [N, K]
// weight that is one 16-byte load per lane, 16 rows x 64 bytes per
// instruction, used as it arrives.  A wave owns 16-row blocks of the weight
// (grid-stride), 32 k per step: one load, one x fragment from LDS (B: x row
// l % 16, zero for rows past M) and one MFMA into D[16 weight rows][16 x
// rows]; after the row block's last step lane l holds out[l % 16][n + 4 (l /
// 16) + r], r = 0..3 -- no cross-lane reduction, no per-row VALU work beyond
// the store.  Loads run in batches of B steps, double-buffered: a batch is
// issued while the previous one is computed.  Weight chunks past K and rows
// past N read zeros (range check); x is zero-padded to whole steps in LDS,
// each row padded by 16 bytes so the rows' reads fall on different banks.
template <int B>
__global__ __launch_bounds__(kF16Threads) void awq_fp16_mfma_kernel(const half_t* __restrict__ x,
                                                                     const half_t* __restrict__ w,
                                                                     half_t* __restrict__ out, int M, int N, int K) {
    extern __shared__ __align__(16) uint32_t lds[];
    half_t* lx = reinterpret_cast<half_t*>(lds);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row = lane & 15;  // weight row within the block (A) and x row (B)
    const int kb = lane >> 4;   // k-block of 8
    const int steps = (K + 31) / 32;
    const int xs = 32 * steps + 8;  // halfs per LDS row of x

    for (int i = threadIdx.x; i < M * (xs / 8); i += kF16Threads) {
        const int m = i / (xs / 8);
        const int ch = i - m * (xs / 8);
        reinterpret_cast<u32x4*>(lx)[i] =
            8 * ch < K ? reinterpret_cast<const u32x4*>(x)[((size_t)m * K) / 8 + ch] : u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();

    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (uint32_t)((size_t)N * K * 2));
    const int nblocks = (N + 15) / 16;
    const int tw = (int)gridDim.x * (kF16Threads / 64);
    const int gw = (int)blockIdx.x * (kF16Threads / 64) + wave;
    const int my_blocks = gw < nblocks ? (nblocks - 1 - gw) / tw + 1 : 0;
    const bool xrow = row < M;
    const half_t* xl = lx + (size_t)row * xs + 8 * kb;

    int iss_b = 0, iss_s = 0;  // next step to issue: local block, step
    auto issue = [&](u32x4 (&dst)[B]) {
#pragma unroll
        for (int j = 0; j < B; ++j) {
            const int n = (gw + iss_b * tw) * 16 + row;
            const int k = 32 * iss_s + 8 * kb;
            const bool ok = iss_b < my_blocks && n < N && k < K;
            dst[j] = buf_load_u4(rw, ok ? ((uint32_t)n * (uint32_t)K + (uint32_t)k) * 2u : 0x80000000u, 0u);
            if (++iss_s == steps) {
                iss_s = 0;
                ++iss_b;
            }
        }
    };
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    int cmp_b = 0, cmp_s = 0;  // next step to compute
    auto compute = [&](const u32x4 (&src)[B]) {
#pragma unroll
        for (int j = 0; j < B; ++j) {
            if (cmp_b >= my_blocks) break;
            half8_t xb = {};
            if (xrow) xb = *reinterpret_cast<const half8_t*>(xl + 32 * cmp_s);
            acc = mfma16x16x32(__builtin_bit_cast(half8_t, src[j]), xb, acc);
            if (++cmp_s == steps) {
                const int n0 = (gw + cmp_b * tw) * 16 + 4 * kb;
                if (xrow) {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (n0 + r < N) out[(size_t)row * N + n0 + r] = (half_t)acc[r];
                }
                acc = floatx4{0.f, 0.f, 0.f, 0.f};
                cmp_s = 0;
                ++cmp_b;
            }
        }
    };
    const int units = my_blocks * steps;
    u32x4 b0[B], b1[B];
    issue(b0);
    for (int t = 0; t < units; t += 2 * B) {
        issue(b1);
        compute(b0);
        issue(b0);
        compute(b1);
    }
}

}  // namespace

int fp16_gemv_max_k() { return kF16MaxK; }

// Workgroups: one wave per SIMD's worth of waves (4 per CU), the row blocks
// divided so that every wave holds the same number of them (9504 blocks of
// the Qwen2-7B lm_head: 951 waves of 10 in 238 workgroups).  Measured on that
// shape at M = 1 / 8, graphs over three weight copies: 178 / 197 us; with
// two, three or four times the waves 182 - 211 us; with one workgroup on
// every CU but 9 or 10 blocks per wave 190 / 206 us; with half the waves
// 303 us (half the CUs idle).
int fp16_mfma_blocks(int N, int cus) {
    const int nblocks = (N + 15) / 16;
    const int slots = 4 * cus;
    const int per = (nblocks + slots - 1) / slots;
    const int waves = (nblocks + per - 1) / per;
    return (waves + kF16Threads / 64 - 1) / (kF16Threads / 64);
}

hipError_t launch_fp16_gemv(const half_t* x, const half_t* w, half_t* out, int M, int N, int K, int cus,
                            hipStream_t stream) {
    if (M == 0) return hipSuccess;
    const int steps = (K + 31) / 32;
    const size_t lds = (size_t)M * (32 * steps + 8) * 2;
    hipLaunchKernelGGL((awq_fp16_mfma_kernel<8>), dim3((unsigned)fp16_mfma_blocks(N, cus)), dim3(kF16Threads), lds,
                       stream, x, w, out, M, N, K);
    return hipGetLastError();
}

}  // namespace awq
