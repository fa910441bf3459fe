// Dense dequantisation W[K,N] = fp16((q - z) * s): the bit-exact check of the
// unpack + dequant device code (kernels/awq_gemm.py:14-87 computes the same
// buffer for its decode path).  One thread per packed word: it reads the word,
// its group's zero word and 8 scales (16 B), and writes 8 fp16 values (16 B).
#include "awq_kernels.h"

namespace awq {

__global__ __launch_bounds__(256) void awq_dequant_kernel(const uint32_t* __restrict__ qweight,
                                                          const uint32_t* __restrict__ qzeros,
                                                          const half_t* __restrict__ scales,
                                                          half_t* __restrict__ w, int pn, int K) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = (int64_t)K * pn;
    if (idx >= total) return;
    const int64_t k = idx / pn;
    const int64_t j = idx - k * pn;
    const int64_t g = k / kGroup;
    const int64_t n = (int64_t)pn * 8;
    const uint32_t word = qweight[idx];
    const uint32_t zw = qzeros[g * pn + j];
    const half8_t s = *reinterpret_cast<const half8_t*>(scales + g * n + 8 * j);
    *reinterpret_cast<half8_t*>(w + k * n + 8 * j) = dequant_word(word, zw, s);
}

hipError_t launch_dequant(const uint32_t* qweight, const uint32_t* qzeros, const half_t* scales,
                          half_t* w, int N, int K, hipStream_t stream) {
    const int pn = N / 8;
    const int64_t total = (int64_t)K * pn;
    if (total == 0) return hipSuccess;
    const int64_t blocks = (total + 255) / 256;
    hipLaunchKernelGGL(awq_dequant_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, qweight,
                       qzeros, scales, w, pn, K);
    return hipGetLastError();
}

}  // namespace awq
