// Prefill W4A16 AWQ GEMM (large M) for gfx950: LDS-tiled MFMA kernel.
//
// Block tile 128 (M) x 128 (N), k-step 32, 256 threads = 4 wavefronts in a
// 2 x 2 grid, each computing 64 x 64 with v_mfma_f32_16x16x32_f16.
//
// The dequantised weight is produced once per block and k-step, next to the
// load: each thread reads two qweight words (rows r, r+1 of one packed
// column), forms per-column k-pairs in registers (v_perm_b32 + magic-number
// decode), subtracts the zero and multiplies by the scale in fp16 -- the
// reference's exact fp16 weight -- and writes the pairs to LDS in a
// [n][k] layout, so that every MFMA operand fragment (8 consecutive k of one
// row) is a single 16-byte LDS read.  x is staged to LDS as [m][k] the same
// way.  The product is computed transposed, out^T = W^T x^T: the W^T fragment
// is the MFMA A operand and the x^T fragment the B operand, so each lane ends
// with 4 consecutive output columns of one row (8-byte stores).
//
// Two LDS buffers: the global loads for k-step t+1 are issued before the
// MFMAs of step t and written to the other buffer after them; one barrier per
// k-step.
#include "awq_kernels.h"

namespace awq {
namespace {
constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 32;
constexpr int PITCH = BK + 8;  // halves per LDS row; 80 B keeps 16-B fragment reads conflict-free
}  // namespace

__global__ __launch_bounds__(256) void awq_tile_kernel_v1(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) half_t As[2][BM * PITCH];
    __shared__ __attribute__((aligned(16))) half_t Bs[2][BN * PITCH];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave & 1;
    const int wn = wave >> 1;
    const int c16 = lane & 15;
    const int kq = lane >> 4;

    const int m_tiles = (a.M + BM - 1) / BM;
    const int tm = blockIdx.x % m_tiles;
    const int tn = blockIdx.x / m_tiles;
    const int m0 = tm * BM;
    const int n0 = tn * BN;
    const int pn = a.N >> 3;

    // x tile loader: 2 chunks of 8 halves per thread.
    int a_row[2], a_kc[2];
    bool a_ok[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int q = tid + 256 * r;
        a_row[r] = q >> 2;
        a_kc[r] = q & 3;
        a_ok[r] = (m0 + a_row[r]) < a.M;
    }
    // weight loader: packed column jj (0..15) of the tile, rows 2*rp, 2*rp+1 of the k-step.
    const int rp = tid & 15;
    const int jj = tid >> 4;
    const int jg = (n0 >> 3) + jj;
    const bool b_ok = jg < pn;
    const int jgc = b_ok ? jg : pn - 1;

    const int KT = a.K / BK;
    half8_t xr[2];
    uint32_t w0, w1;
    uint32_t zs[8];
    uint32_t ss[8];  // fp16 scale pairs (s, s)

    auto load_global = [&](int kt) {
        const int kb = kt * BK;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            if (a_ok[r])
                xr[r] = *reinterpret_cast<const half8_t*>(a.x + (size_t)(m0 + a_row[r]) * a.K + kb + 8 * a_kc[r]);
            else
                xr[r] = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
        }
        const uint32_t* wp = a.qweight + (size_t)(kb + 2 * rp) * pn + jgc;
        w0 = wp[0];
        w1 = wp[pn];
    };
    auto load_group = [&](int kt) {
        const int g = (kt * BK) / kGroup;
        const uint32_t zw = a.qzeros[(size_t)g * pn + jgc];
        const half8_t s8 = *reinterpret_cast<const half8_t*>(a.scales + (size_t)g * a.N + 8 * jgc);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            zs[c] = zero_splat(zw, c);
            ss[c] = as_u32(half2_t{s8[c], s8[c]});
        }
    };
    auto store_lds = [&](int buf) {
#pragma unroll
        for (int r = 0; r < 2; ++r)
            *reinterpret_cast<half8_t*>(&As[buf][a_row[r] * PITCH + 8 * a_kc[r]]) = xr[r];
        uint32_t kp[8];
        kpairs_magic(w0, w1, kp);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const half2_t v = (as_h2(kp[c]) - as_h2(zs[c])) * as_h2(ss[c]);
            const uint32_t bits = b_ok ? as_u32(v) : 0u;
            *reinterpret_cast<uint32_t*>(&Bs[buf][(8 * jj + c) * PITCH + 2 * rp]) = bits;
        }
    };

    floatx4 acc[4][4];
#pragma unroll
    for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int y = 0; y < 4; ++y) acc[x][y] = floatx4{0.f, 0.f, 0.f, 0.f};

    load_group(0);
    load_global(0);
    store_lds(0);
    __syncthreads();

    for (int kt = 0; kt < KT; ++kt) {
        const int buf = kt & 1;
        const bool has_next = kt + 1 < KT;
        if (has_next) load_global(kt + 1);

        half8_t af[4], bfr[4];
#pragma unroll
        for (int x = 0; x < 4; ++x)
            af[x] = *reinterpret_cast<const half8_t*>(&Bs[buf][(64 * wn + 16 * x + c16) * PITCH + 8 * kq]);
#pragma unroll
        for (int y = 0; y < 4; ++y)
            bfr[y] = *reinterpret_cast<const half8_t*>(&As[buf][(64 * wm + 16 * y + c16) * PITCH + 8 * kq]);
#pragma unroll
        for (int x = 0; x < 4; ++x)
#pragma unroll
            for (int y = 0; y < 4; ++y) acc[x][y] = mfma16x16x32(af[x], bfr[y], acc[x][y]);

        if (has_next) {
            if (((kt + 1) * BK) % kGroup == 0) load_group(kt + 1);
            store_lds(buf ^ 1);
        }
        __syncthreads();
    }

    // acc[x][y] lane value v: out^T[n = 16x + 4kq + v][m = 16y + c16] of this wave's 64 x 64.
#pragma unroll
    for (int y = 0; y < 4; ++y) {
        const int gm = m0 + 64 * wm + 16 * y + c16;
        if (gm >= a.M) continue;
#pragma unroll
        for (int x = 0; x < 4; ++x) {
            const int gn = n0 + 64 * wn + 16 * x + 4 * kq;
            if (gn >= a.N) continue;
            const half4_t h = {(half_t)acc[x][y][0], (half_t)acc[x][y][1], (half_t)acc[x][y][2],
                               (half_t)acc[x][y][3]};
            *reinterpret_cast<half4_t*>(a.out + (size_t)gm * a.N + gn) = h;
        }
    }
}

hipError_t launch_tile(const GemmArgs& a, const TileConfig& cfg, hipStream_t stream) {
    if (cfg.variant != 1) return hipErrorInvalidValue;
    const int64_t m_tiles = (a.M + BM - 1) / BM;
    const int64_t n_tiles = (a.N + BN - 1) / BN;
    const int64_t blocks = m_tiles * n_tiles;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(awq_tile_kernel_v1, dim3((unsigned)blocks), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace awq
