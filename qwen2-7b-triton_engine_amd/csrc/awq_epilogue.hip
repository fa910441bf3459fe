// SiLU * up over the fused gate||up projection: out[m, i] = fp16(silu(g) *
// u) with g = gate_up[m, i], u = gate_up[m, I + i], computed in fp32 --
// the reference's kernels/silu_mul.py:17-39 (x * sigmoid(x) * y in fp32,
// one rounding), reading the fused output in place instead of its two
// .contiguous() copies (model/qwen2.py:187-194): one pass, 6 bytes read and
// 2 written per output.  Each thread handles 8 consecutive outputs with
// 16-byte loads and stores (I % 8 == 0).
#include "awq_kernels.h"

namespace awq {
namespace {

__global__ __launch_bounds__(256) void awq_silu_mul_kernel(const half_t* __restrict__ gu, half_t* __restrict__ out,
                                                           int M, int I) {
    const int per_row = I / 8;
    const int64_t total = (int64_t)M * per_row;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
        const int m = (int)(t / per_row);
        const int i = (int)(t - (int64_t)m * per_row) * 8;
        const half8_t g = *reinterpret_cast<const half8_t*>(gu + (size_t)m * 2 * I + i);
        const half8_t u = *reinterpret_cast<const half8_t*>(gu + (size_t)m * 2 * I + I + i);
        half8_t o;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float x = (float)g[e];
            o[e] = (half_t)(x / (1.0f + expf(-x)) * (float)u[e]);
        }
        *reinterpret_cast<half8_t*>(out + (size_t)m * I + i) = o;
    }
}

}  // namespace

hipError_t launch_silu_mul(const half_t* gate_up, half_t* out, int M, int I, hipStream_t stream) {
    if (M == 0) return hipSuccess;
    const int64_t items = (int64_t)M * (I / 8);
    int64_t blocks = (items + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(awq_silu_mul_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, gate_up, out, M, I);
    return hipGetLastError();
}

}  // namespace awq
