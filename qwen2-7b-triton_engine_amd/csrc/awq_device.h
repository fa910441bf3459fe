// Device helpers shared by the W4A16 AWQ kernels (gfx950 / CDNA4).
//
// AWQ packing (kernels/awq_gemm.py:5-6): logical column c of a packed int32
// word sits in nibble ORD[c], ORD = {0,4,1,5,2,6,3,7}.  Equivalently the low
// 16 bits of a word hold columns 0,2,4,6 (nibbles 0..3) and the high 16 bits
// hold columns 1,3,5,7 (nibbles 4..7).  So `(w >> 4t) & 0x000F000F` puts
// column 2t in the low half-word and column 2t+1 in the high half-word: the
// order is made for packed 16-bit arithmetic.
//
// int4 -> fp16 without conversion instructions: 0x6400 is fp16 1024.0, whose
// unit in the last place is exactly 1, so OR-ing a code c (0..15) into the
// low mantissa bits gives the fp16 value 1024 + c (Kim et al., 2022, "Who Says
// Elephants Can't Run").  (1024 + q) - (1024 + z) = q - z is then exact in
// fp16, and one fp16 multiply by the scale rounds once, to nearest even: the
// reference's fp16((q - z) * s) bit for bit (kernels/awq_gemm.py:59,223).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace awq {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kGroup = 128;          // AWQ group size served by the kernels
constexpr uint32_t kMagic2 = 0x64006400u;  // fp16 pair (1024.0, 1024.0)

__device__ __forceinline__ half2_t as_h2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }
__device__ __forceinline__ uint32_t as_u32(half2_t v) { return __builtin_bit_cast(uint32_t, v); }

// Nibble shift of logical column c (0..7): 4 * ORD[c].
__device__ __forceinline__ constexpr int col_shift(int c) { return 4 * ((c >> 1) + (c & 1) * 4); }

// (1024 + code) of logical columns (2t, 2t+1) of one word, as an fp16 pair.
__device__ __forceinline__ uint32_t pair_magic(uint32_t w, int t) {
    return ((w >> (4 * t)) & 0x000F000Fu) | kMagic2;
}

// fp16 pair (1024 + z, 1024 + z) for logical column c of a packed zero word.
__device__ __forceinline__ uint32_t zero_splat(uint32_t zw, int c) {
    const uint32_t z = (zw >> col_shift(c)) & 0xFu;
    return kMagic2 | z | (z << 16);
}

// Exact dequant of one packed word: out[c] = fp16((q_c - z_c) * s_c) in
// logical column order c = 0..7.
__device__ __forceinline__ half8_t dequant_word(uint32_t w, uint32_t zw, half8_t s) {
    half8_t out;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const half2_t d = as_h2(pair_magic(w, t)) - as_h2(pair_magic(zw, t));  // exact q - z
        const half2_t s2 = {s[2 * t], s[2 * t + 1]};
        const half2_t r = d * s2;                                             // one RNE rounding
        out[2 * t] = r.x;
        out[2 * t + 1] = r.y;
    }
    return out;
}

// k-pairs of two words a (row r) and b (row r + 1) of the same packed column:
// kp[c] = fp16 pair (1024 + q[r][c], 1024 + q[r+1][c]) for logical column c.
// v_perm_b32 gathers the low (high) half-words of a and b into one register,
// so each column's two rows land in the two halves of one 32-bit value.
__device__ __forceinline__ void kpairs_magic(uint32_t a, uint32_t b, uint32_t kp[8]) {
    const uint32_t lo = __builtin_amdgcn_perm(b, a, 0x05040100u);  // a[15:0] | b[15:0] << 16
    const uint32_t hi = __builtin_amdgcn_perm(b, a, 0x07060302u);  // a[31:16] | b[31:16] << 16
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        kp[2 * u] = ((lo >> (4 * u)) & 0x000F000Fu) | kMagic2;      // column 2u (nibble u)
        kp[2 * u + 1] = ((hi >> (4 * u)) & 0x000F000Fu) | kMagic2;  // column 2u+1 (nibble u+4)
    }
}

// (x & mask) | magic.  With the mask a literal (it goes to an SGPR) and the
// magic in a VGPR the compiler does not know the value of, this is one
// v_and_or_b32; with both literals it becomes v_and + v_or (gfx9 VOP3
// encodings carry no literal).  Written in plain C, not inline asm: the
// compiler inserts the wait states between a VALU write and an MFMA that
// reads (or is still reading or writing) the same VGPRs only for
// instructions it generated itself, never around an asm statement.
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t magic) { return (x & mask) | magic; }
// kMagic2 in a VGPR, opaque to the optimiser: a DPP row shift whose
// out-of-row lanes keep `old` (bound_ctrl off), with old = src = the
// constant, so every lane holds it.  The compiler cannot fold the DPP move,
// so and_or(x, mask, magic_vgpr()) stays one v_and_or_b32.
__device__ __forceinline__ uint32_t magic_vgpr() {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)kMagic2, (int)kMagic2, 0x111 /* row_shr:1 */, 0xF, 0xF,
                                                 false);
}

// fp16 pair (64.0, 64.0).  The unit in the last place of 64 is 1/16, so a
// code c held in mantissa bits 4..7 (the integer 16c in the mantissa field)
// reads as 64 + c: a nibble can be cut out of a word in place, without a
// shift, and still give an exact fp16 code.
constexpr uint32_t kMagic2Hi = 0x54005400u;
// kMagic2Hi in a VGPR (see magic_vgpr).
__device__ __forceinline__ uint32_t magic_hi_vgpr() {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)kMagic2Hi, (int)kMagic2Hi, 0x111 /* row_shr:1 */, 0xF, 0xF,
                                                 false);
}

// As kpairs_magic, with half the shifts by 4: nibbles 1 and 3 of each
// half-word are masked in place (mask 0x00F000F0) and read with the 64.0
// magic, which yields the fp16 value 64 + q.  Columns 2, 3, 6, 7 (c with bit
// 1 set) therefore carry the offset 64, the others 1024 (magic_base); with
// the matching zero splat (zero_splat_inplace) the difference q - z is exact
// for every column, so fp16((q - z) * s) rounds once, as the reference does.
__device__ __forceinline__ void kpairs_magic_inplace(uint32_t a, uint32_t b, uint32_t kp[8]) {
    const uint32_t magic = magic_vgpr();
    const uint32_t magic_hi = magic_hi_vgpr();
    const uint32_t lo = __builtin_amdgcn_perm(b, a, 0x05040100u);
    const uint32_t hi = __builtin_amdgcn_perm(b, a, 0x07060302u);
    const uint32_t lo8 = lo >> 8;
    const uint32_t hi8 = hi >> 8;
    kp[0] = and_or(lo, 0x000F000Fu, magic);
    kp[2] = and_or(lo, 0x00F000F0u, magic_hi);
    kp[4] = and_or(lo8, 0x000F000Fu, magic);
    kp[6] = and_or(lo8, 0x00F000F0u, magic_hi);
    kp[1] = and_or(hi, 0x000F000Fu, magic);
    kp[3] = and_or(hi, 0x00F000F0u, magic_hi);
    kp[5] = and_or(hi8, 0x000F000Fu, magic);
    kp[7] = and_or(hi8, 0x00F000F0u, magic_hi);
}

// Whether kpairs_magic_inplace reads logical column c with the 64.0 magic.
__device__ __forceinline__ constexpr bool inplace_column(int c) { return (c >> 1) & 1; }
// The offset kpairs_magic_inplace adds to the code of logical column c.
__device__ __forceinline__ constexpr float magic_base(int c) { return inplace_column(c) ? 64.0f : 1024.0f; }

// Zero splat matching kpairs_magic_inplace for logical column c: the fp16
// pair (base + z, base + z).
__device__ __forceinline__ uint32_t zero_splat_inplace(uint32_t zw, int c) {
    const uint32_t z = (zw >> col_shift(c)) & 0xFu;
    return inplace_column(c) ? (kMagic2Hi | (z << 4) | (z << 20)) : (kMagic2 | z | (z << 16));
}


__device__ __forceinline__ floatx4 mfma16x16x32(half8_t a, half8_t b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Raw buffer resources (gfx9 descriptor word 3 = 0x00020000).  Reads whose
// VGPR offset lies at or beyond num_bytes return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t num_bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)num_bytes,
                                             0x00020000);
}
__device__ __forceinline__ uint32_t buf_load_b32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}
__device__ __forceinline__ half8_t buf_load_h8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ u32x4 buf_load_u4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// Direct global->LDS loads: buffer_load_dword[x4] ... lds writes each lane's
// 4 (16) bytes to M0 + 4*lane (16*lane), so a wave fills one contiguous LDS
// block per instruction and each lane chooses which global element lands in
// its slot; no VGPR holds the data, so many can be in flight.  Issued from
// inline assembly: the compiler cannot tell which LDS bytes such a load
// writes and would otherwise wait for every outstanding load before each LDS
// read.  The caller waits itself (s_waitcnt vmcnt, then a barrier).
__device__ __forceinline__ void buffer_load_lds_x4(u32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds_base) {
    asm volatile(
        "s_mov_b32 m0, %3\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %0, %1, %2 offen lds"
        :
        : "v"(voff), "s"(rsrc), "s"(soff), "s"(lds_base)
        : "memory", "m0");
}
__device__ __forceinline__ void buffer_load_lds_x1(u32x4 rsrc, uint32_t voff, uint32_t soff, uint32_t lds_base) {
    asm volatile(
        "s_mov_b32 m0, %3\n\t"
        "s_nop 0\n\t"
        "buffer_load_dword %0, %1, %2 offen lds"
        :
        : "v"(voff), "s"(rsrc), "s"(soff), "s"(lds_base)
        : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p);
}

__device__ __forceinline__ u32x4 raw_rsrc(const void* base, uint32_t num_bytes) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    return u32x4{(uint32_t)b, (uint32_t)(b >> 32) & 0xFFFFu, num_bytes, 0x00020000u};
}

// s_waitcnt vmcnt(n * LOADS) for a wave-uniform n in 0 .. N (immediate
// operands only, hence the chain).
template <int LOADS, int N>
__device__ __forceinline__ void wait_batches(int n) {
    if constexpr (N > 0) {
        if (n >= N) {
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N * LOADS) : "memory");
            return;
        }
        wait_batches<LOADS, N - 1>(n);
    } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
}

// Device-scope (cache policy SC1) 16-byte store and load: coherent across
// the XCDs of the device without whole-L2 maintenance.
constexpr int kCpolSC1 = 16;
// Non-temporal (streaming) load hint, used for the decode kernels' weight
// loads when a workgroup streams a long K range: at most this many splits.
constexpr int kCpolNT = 2;
constexpr int kNonTemporalMaxSplit = 4;
__device__ __forceinline__ void buf_store_f4_device(floatx4 v, __amdgpu_buffer_rsrc_t r, uint32_t voff) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, voff, 0, kCpolSC1);
}
__device__ __forceinline__ floatx4 buf_load_f4_device(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
    return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, kCpolSC1));
}
// s_waitcnt vmcnt(0) (expcnt, lgkmcnt left at their maxima): every vector
// memory operation of this wave, stores included, has completed.
__device__ __forceinline__ void wait_vm_stores() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Split-K finish in one atomic per output element.
//
// Each output element owns a 64-bit slot in the workspace, zero between
// calls.  Every workgroup that holds a partial sum p of the element adds
//     (fixed(p) << 8) + 1,   fixed(p) = round(p * 2^24) as a signed integer,
// to the slot with one agent-scope atomic that returns the old value.  The
// low byte counts arrivals and the upper 56 bits sum the partials in 24-bit
// fixed point.  The workgroup whose return shows split_k arrivals holds the
// complete sum in the returned value: it writes the fp16 output and stores
// zero back into the slot.  Integer addition is exact and associative, so
// the result does not depend on arrival order (bitwise deterministic), and
// there is no separate counter, no wait for store acknowledgements and no
// reload of partials: one memory round trip after the last partial.
//
// Range: partials are clamped to +-2^22 (far beyond fp16's 65504, which
// saturates to +-inf on conversion; NaN is treated as +2^22 and so becomes
// +inf), so that the sum of up to 255 partials stays inside the 56-bit field.
// A partial with |p| >= 0.5 converts exactly; smaller ones round to 2^-24.
constexpr int kFixMaxSplit = 255;
// The word a workgroup adds for its partial p.
__device__ __forceinline__ unsigned long long fixed_point_word(float p) {
    const float clamp = 4194304.0f;  // 2^22
    const float c = p == p ? fminf(fmaxf(p, -clamp), clamp) : clamp;
    const long long f = (long long)rintf(c * 16777216.0f);
    return ((unsigned long long)f << 8) + 1ull;
}
// `now` = the slot's value after this workgroup's add (returned old value
// plus its word): the last of split_k arrivals writes the output and clears
// the slot.
// The value stored for one output element: fp16 of the fp32 sum, then, when
// given, + bias[n] and + residual[m, n], each add done in fp32 and rounded
// to fp16 -- the reference's unfused sequence (out = awq_gemm_forward(...);
// out + bias, model/qwen2.py:45-46,108-109; residual + out, :219-227; torch
// adds fp16 tensors in fp32 and rounds), so a fused epilogue and the unfused
// calls agree bit for bit.  bias_n / res point at the element (or are null).
__device__ __forceinline__ half_t epi_round(float y, const half_t* bias_n, const half_t* res) {
    half_t h = (half_t)y;
    if (bias_n) h = (half_t)((float)h + (float)*bias_n);
    if (res) h = (half_t)((float)*res + (float)h);
    return h;
}
// V consecutive outputs out[m, n .. n+V-1] (V = 4 or 8, n % V == 0) as one
// vector store, with the epilogue above.  Device-scope (write-through)
// stores: the output leaves L2 while the kernel still runs instead of in the
// write-back at its end (measured 0.5 - 4 % faster on the reduce launches
// and whole tiles).  Output byte offsets stay below 2^31 (the host checks
// M N 2 < 2^31), so one buffer resource from `out` covers every store.
template <int V>
__device__ __forceinline__ void store_out(half_t* out, const half_t* bias, const half_t* residual, int N, int m,
                                          int n, const float (&y)[V]) {
    typedef _Float16 hv_t __attribute__((ext_vector_type(V)));
    hv_t h;
    const size_t o = (size_t)m * N + n;
    if (!bias && !residual) {
#pragma unroll
        for (int i = 0; i < V; ++i) h[i] = (half_t)y[i];
    } else {
#pragma unroll
        for (int i = 0; i < V; ++i) h[i] = epi_round(y[i], bias ? bias + n + i : nullptr, residual ? residual + o + i : nullptr);
    }
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(out, 0x7FFFFFFFu);
    if constexpr (V == 8) {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, h), ro, (uint32_t)(o * 2), 0, kCpolSC1);
    } else {
        static_assert(V == 4, "4 or 8 outputs");
        typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, h), ro, (uint32_t)(o * 2), 0, kCpolSC1);
    }
}
// epi_round with the bias / residual values already loaded (has_* says
// which of them apply).
__device__ __forceinline__ half_t epi_round_vals(float y, bool has_bias, half_t bias_v, bool has_res, half_t res_v) {
    half_t h = (half_t)y;
    if (has_bias) h = (half_t)((float)h + (float)bias_v);
    if (has_res) h = (half_t)((float)res_v + (float)h);
    return h;
}
// out[o] = h as a device-scope (write-through) store, like store_out's.
__device__ __forceinline__ void store_half_device(half_t* out, size_t o, half_t h) {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, h), make_rsrc(out, 0x7FFFFFFFu),
                                          (uint32_t)(o * 2), 0, kCpolSC1);
}
// The sum held by a fixed-point slot value.
__device__ __forceinline__ float fixed_point_sum(unsigned long long now) {
    return (float)((long long)now >> 8) * (1.0f / 16777216.0f);
}
// The last step of B outputs of one thread (out[m[b], n[b]] for the b with
// ok[b]): a direct store of the fp32 sum when split_k == 1, else the
// fixed-point finish above, with every memory round trip in flight
// together -- the bias / residual values are loaded first, then all B
// atomics are issued, and only then are the returned values examined (a
// returned value read before the next atomic is issued makes the wave wait
// for it, and B outputs would cost B round trips).  The bias / residual
// reads are range-checked buffer loads (a null operand gets a zero-size
// range and reads 0), so no branch joins a loaded value with a default one,
// which also makes the wave wait for the load.  Needs M * N * 2 < 2^32
// (the callers serve M <= 16).
template <int B>
__device__ __forceinline__ void finish_batch(unsigned long long* fix, half_t* out, const half_t* bias,
                                             const half_t* residual, int M, int N, int split_k, const float (&sum)[B],
                                             const int (&m)[B], const int (&n)[B], const bool (&ok)[B]) {
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(bias, bias ? (uint32_t)N * 2u : 0u);
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(residual, residual ? (uint32_t)((size_t)M * N * 2) : 0u);
    half_t bv[B], rv[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
        const uint32_t o = (uint32_t)m[b] * (uint32_t)N + (uint32_t)n[b];
        bv[b] = __builtin_bit_cast(half_t, __builtin_amdgcn_raw_buffer_load_b16(
                                               rb, ok[b] ? (uint32_t)n[b] * 2u : 0x80000000u, 0, 0));
        rv[b] = __builtin_bit_cast(half_t, __builtin_amdgcn_raw_buffer_load_b16(rr, ok[b] ? o * 2u : 0x80000000u,
                                                                                 0, 0));
    }
    if (split_k == 1) {
#pragma unroll
        for (int b = 0; b < B; ++b)
            if (ok[b])
                store_half_device(out, (size_t)m[b] * N + n[b],
                                  epi_round_vals(sum[b], bias != nullptr, bv[b], residual != nullptr, rv[b]));
        return;
    }
    unsigned long long word[B], old[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
        word[b] = fixed_point_word(sum[b]);
        old[b] = 0ull;
        if (ok[b])
            old[b] = __hip_atomic_fetch_add(fix + (size_t)m[b] * N + n[b], word[b], __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int b = 0; b < B; ++b) {
        const unsigned long long now = old[b] + word[b];
        if (ok[b] && (int)(now & 0xFFull) == split_k) {
            const size_t o = (size_t)m[b] * N + n[b];
            store_half_device(out, o, epi_round_vals(fixed_point_sum(now), bias != nullptr, bv[b], residual != nullptr, rv[b]));
            __hip_atomic_store(fix + o, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Last-arriving workgroup of a split-K output range: for rows row0 ..
// row0+nrows and columns col0 .. col0+ncols,
// out[m, n] = fp16(sum over split of partials[split, m, n]) (partials of
// shape [split, M, N]).  Every thread of the workgroup takes part and the
// loads of many outputs are in flight together:
//  * few outputs (fewer quads than threads): each output quad gets P threads
//    that add the splits part, part+P, ... (8 loads at a time), combined
//    through LDS in a fixed order;
//  * many outputs: each thread keeps up to U quads in registers and adds
//    split after split, U loads in flight per split (U is a template
//    parameter so that callers that never have many outputs keep their
//    register footprint).
// Either way each element is summed in a fixed order, independent of timing.
// The partials are left as they are: the next split-K call writes every
// partial it reads, and the fixed-point slots live in a region of their own.
// `fin` holds blockDim.x float4.  Must be called by the whole workgroup.
// Where the partial of split q for output (row0 + r, col0 + c) lives: byte
// base + r * row_stride + 4 c + q * split_stride of the partials buffer.
struct PartLayout {
    uint32_t base, row_stride, split_stride;
};
// The [split, M, N] layout.
__device__ __forceinline__ PartLayout full_parts(int M, int N, int row0, int col0) {
    return PartLayout{(uint32_t)(((size_t)row0 * N + col0) * 4), (uint32_t)N * 4u, (uint32_t)((size_t)M * N * 4)};
}

template <int U>
__device__ __forceinline__ void splitk_finish(__amdgpu_buffer_rsrc_t rp, half_t* __restrict__ out,
                                              const half_t* bias, const half_t* residual, int M, int N,
                                              int row0, int nrows, int col0, int ncols, int split_k,
                                              floatx4* fin, PartLayout pl) {
    const int quads = ncols / 4;
    const int items = nrows * quads;
    const int nt = blockDim.x;
    const int t = threadIdx.x;
    const uint32_t stride = pl.split_stride;
    auto item_off = [&](int item, int& m, int& n) {
        const int r = item / quads;
        const int c = 4 * (item - r * quads);
        m = row0 + r;
        n = col0 + c;
        return pl.base + (uint32_t)r * pl.row_stride + (uint32_t)c * 4u;
    };
    auto store = [&](int m, int n, floatx4 s) {
        const float y[4] = {s[0], s[1], s[2], s[3]};
        store_out<4>(out, bias, residual, N, m, n, y);
    };
    if (items < nt) {
        const int P = min(8, nt / items);
        const int part = t / items;
        const int item = t - part * items;
        const bool valid = part < P;
        floatx4 s = {0.f, 0.f, 0.f, 0.f};
        int m = 0, n = 0;
        if (valid) {
            const uint32_t off = item_off(item, m, n);
#pragma unroll 8
            for (int q = part; q < split_k; q += P) s += buf_load_f4_device(rp, off + (uint32_t)q * stride);
        }
        if (P > 1) {
            if (valid) fin[t] = s;
            __syncthreads();
            if (valid && part == 0) {
                for (int p = 1; p < P; ++p) s += fin[p * items + item];
            }
        }
        if (valid && part == 0) store(m, n, s);
        return;
    }
    for (int base = 0; base < items; base += U * nt) {
        floatx4 s[U];
        uint32_t off[U];
        int mm[U], nn[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int item = base + u * nt + t;
            s[u] = floatx4{0.f, 0.f, 0.f, 0.f};
            off[u] = item < items ? item_off(item, mm[u], nn[u]) : 0u;
        }
        for (int q = 0; q < split_k; ++q) {
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (base + u * nt + t < items) s[u] += buf_load_f4_device(rp, off[u] + (uint32_t)q * stride);
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (base + u * nt + t < items) store(mm[u], nn[u], s[u]);
    }
}

// splitk_finish over the [split, M, N] partials layout.
template <int U>
__device__ __forceinline__ void splitk_finish(__amdgpu_buffer_rsrc_t rp, half_t* __restrict__ out,
                                              const half_t* bias, const half_t* residual, int M, int N,
                                              int row0, int nrows, int col0, int ncols, int split_k,
                                              floatx4* fin) {
    splitk_finish<U>(rp, out, bias, residual, M, N, row0, nrows, col0, ncols, split_k, fin,
                     full_parts(M, N, row0, col0));
}

}  // namespace awq
