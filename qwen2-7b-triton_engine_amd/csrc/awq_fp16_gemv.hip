// fp16 GEMV for the output projection: out[M, N] = x[M, K] @ weight[N, K]^T
// with fp32 accumulation and fp16 results -- the lm_head of
// model/qwen2.py:253,280 (nn.Linear(hidden, vocab, bias=False)) at decode
// sizes (M <= 8; greedy decoding needs the last position's logits only).
// HBM-bound: 152064 x 3584 fp16 = 1.09 GB per token for Qwen2-7B.
//
// Layout: weight rows are contiguous K-vectors (nn.Linear's [out, in]).  A
// wave takes four rows at a time: lane l reads 16-byte chunk c = l % 16 +
// 16 j (j = 0, 1, ...) of row 4 q + l / 16, so one load instruction covers
// four 256-byte row segments.  All of a row quad's loads are issued before
// any is used (28 per lane at K = 3584); the workgroups, up to four per CU
// with four waves each, keep enough of them in flight to cover HBM latency.  x
// (M x K fp16) is staged in LDS once per workgroup; each chunk's products go
// through v_dot2_f32_f16 into one fp32 sum per (lane, row of x), and the 16
// lanes of a row segment are added with cross-lane shuffles (a DPP row is 16
// lanes).  Rows past N read zeros (buffer range check) and are not stored.
#include "awq_kernels.h"

namespace awq {
namespace {

constexpr int kF16Threads = 256;
constexpr int kF16MaxChunks = 32;  // 16-byte chunks per lane and row: K <= 16 * 32 * 8 = 4096

template <int MR, int NJ>
__global__ __launch_bounds__(kF16Threads) void awq_fp16_gemv_kernel(const half_t* __restrict__ x,
                                                                     const half_t* __restrict__ w,
                                                                     half_t* __restrict__ out, int M, int N,
                                                                     int K) {
    extern __shared__ __align__(16) uint32_t lds[];
    half_t* lx = reinterpret_cast<half_t*>(lds);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15;
    const int r = lane >> 4;
    const int chunks = K / 8;                // 16-byte chunks per row
    constexpr int kp = 16 * NJ;              // chunks per LDS row of x, zero-padded to the unrolled loop

    // x -> LDS (M rows of kp chunks, the padding zero), 16 bytes per thread
    // per step.  With the padding and the weight chunks past K reading zero
    // (range check), every lane runs the same straight-line loop.
    for (int i = threadIdx.x; i < M * kp; i += kF16Threads) {
        const int m = i / kp;
        const int ch = i - m * kp;
        reinterpret_cast<u32x4*>(lx)[i] =
            ch < chunks ? reinterpret_cast<const u32x4*>(x)[(size_t)m * chunks + ch] : u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();

    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (uint32_t)((size_t)N * K * 2));
    const int quads = (N + 3) / 4;
    const int waves_total = (int)gridDim.x * (kF16Threads / 64);
    for (int q = (int)blockIdx.x * (kF16Threads / 64) + wave; q < quads; q += waves_total) {
        const int row = 4 * q + r;
        const uint32_t rbase = row < N ? (uint32_t)((size_t)row * K * 2) + 16u * (uint32_t)c : 0x80000000u;
        u32x4 wv[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j)
            wv[j] = buf_load_u4(rw, c + 16 * j < chunks ? rbase + 256u * (uint32_t)j : 0x80000000u, 0u);
        float acc[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) acc[m] = 0.f;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                if (m >= M) break;
                const u32x4 xv = *reinterpret_cast<const u32x4*>(lx + 8 * ((size_t)m * kp + c + 16 * j));
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc[m] = __builtin_amdgcn_fdot2(as_h2(wv[j][e]), as_h2(xv[e]), acc[m], false);
            }
        }
        // The 16 lanes of a row segment hold the row's partial sums.
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int off = 8; off >= 1; off >>= 1) acc[m] += __shfl_xor(acc[m], off);
        if (c == 0 && row < N) {
#pragma unroll
            for (int m = 0; m < MR; ++m)
                if (m < M) out[(size_t)m * N + row] = (half_t)acc[m];
        }
    }
}

template <int MR>
hipError_t launch_mr(const half_t* x, const half_t* w, half_t* out, int M, int N, int K, int blocks,
                     hipStream_t stream) {
    const int nj = (K / 8 + 15) / 16;
    // LDS: M rows of 16 * NJ chunks of 16 bytes (at most 8 x 32 x 256 B = 64 KiB).
    if (nj <= 8)
        hipLaunchKernelGGL((awq_fp16_gemv_kernel<MR, 8>), dim3(blocks), dim3(kF16Threads), (size_t)M * 8 * 256,
                           stream, x, w, out, M, N, K);
    else if (nj <= 16)
        hipLaunchKernelGGL((awq_fp16_gemv_kernel<MR, 16>), dim3(blocks), dim3(kF16Threads), (size_t)M * 16 * 256,
                           stream, x, w, out, M, N, K);
    else if (nj <= 28)
        hipLaunchKernelGGL((awq_fp16_gemv_kernel<MR, 28>), dim3(blocks), dim3(kF16Threads), (size_t)M * 28 * 256,
                           stream, x, w, out, M, N, K);
    else
        hipLaunchKernelGGL((awq_fp16_gemv_kernel<MR, kF16MaxChunks>), dim3(blocks), dim3(kF16Threads),
                           (size_t)M * kF16MaxChunks * 256, stream, x, w, out, M, N, K);
    return hipGetLastError();
}

}  // namespace

int fp16_gemv_max_k() { return 16 * kF16MaxChunks * 8; }

int fp16_gemv_blocks(int N) {
    const int quads = (N + 3) / 4;
    const int per_block = kF16Threads / 64;
    const int need = (quads + per_block - 1) / per_block;
    const int cap = 4 * 256;  // four workgroups per CU (<= 128 VGPRs at K <= 3584), grid-stride beyond
    return need < cap ? need : cap;
}

hipError_t launch_fp16_gemv(const half_t* x, const half_t* w, half_t* out, int M, int N, int K,
                            hipStream_t stream) {
    if (M == 0) return hipSuccess;
    const int blocks = fp16_gemv_blocks(N);
    if (M == 1) return launch_mr<1>(x, w, out, M, N, K, blocks, stream);
    if (M == 2) return launch_mr<2>(x, w, out, M, N, K, blocks, stream);
    if (M <= 4) return launch_mr<4>(x, w, out, M, N, K, blocks, stream);
    return launch_mr<8>(x, w, out, M, N, K, blocks, stream);
}

}  // namespace awq
