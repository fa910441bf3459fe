/*
 * Plain-C restatement of the reference's AWQ dequant + matmul.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (ctypes) as an independent
 * second oracle next to the numpy one (oracle/awq_oracle.py).  The product
 * library never links or calls it.
 *
 * Reference followed: the per-column loop of inference/baseline_kernels.py:36-60
 *   for i in range(N):
 *     shift  = ((i%8 // 2) + (i%8 % 2) * 4) * 4          (:46-48)
 *     w_int4 = (qweight[:, i//8] >> shift) & 0xF           (:50)
 *     z_int4 = (qzeros[k//G, i//8] >> shift) & 0xF         (:52-53)
 *     w[:, i] = (w_int4.half() - z_int4.half()) * scales[k//G, i]   (:55-57)
 *   out = x @ w                                            (:59)
 * The fp16 arithmetic is restated here bit by bit: the subtraction of two
 * integers in 0..15 is exact, and the fp16 product is the exact product
 * (exact in binary32: 5-bit times 11-bit significands) rounded once to fp16
 * with roundTiesToEven, done by oracle_f32_to_f16 below, written from the
 * IEEE 754 binary16 definition (1 sign, 5 exponent bits with bias 15,
 * 10 fraction bits, gradual underflow, overflow to infinity).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* v / 2^s rounded to nearest, ties to even; s >= 1. */
static uint32_t shift_rne(uint32_t v, int s) {
    if (s >= 32) return 0;
    uint32_t q = v >> s;
    uint32_t rem = v & ((1u << s) - 1u);
    uint32_t halfway = 1u << (s - 1);
    if (rem > halfway || (rem == halfway && (q & 1u))) q++;
    return q;
}

uint16_t oracle_f32_to_f16(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t bexp = (u >> 23) & 0xFFu;
    const uint32_t frac = u & 0x7FFFFFu;
    if (bexp == 0xFFu) /* inf stays inf, NaN stays a quiet NaN */
        return (uint16_t)(sign | 0x7C00u | (frac ? 0x0200u | (frac >> 13) : 0u));
    if (bexp == 0u) /* binary32 zero or subnormal: far below half the fp16 subnormal unit */
        return (uint16_t)sign;
    const int e = (int)bexp - 127;        /* value = sig * 2^(e-23), sig in [2^23, 2^24) */
    const uint32_t sig = frac | 0x800000u;
    if (e > 15) return (uint16_t)(sign | 0x7C00u);
    if (e >= -14) {                        /* normal fp16 range */
        uint32_t m = shift_rne(sig, 13);   /* in [1024, 2048] */
        uint32_t he = (uint32_t)(e + 15);
        if (m == 2048u) { m = 1024u; he++; }
        if (he >= 31u) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | (he << 10) | (m & 0x3FFu));
    }
    /* subnormal fp16: count units of 2^-24; sig * 2^(e-23) = sig * 2^(e+1) units */
    const int s = -(e + 1);                /* >= 14 */
    const uint32_t m = shift_rne(sig, s);  /* 1024 rounds up into the smallest normal */
    return (uint16_t)(sign | m);
}

float oracle_f16_to_f32(uint16_t h) {
    const int neg = (h & 0x8000u) != 0;
    const int he = (h >> 10) & 0x1F;
    const int m = h & 0x3FF;
    float v;
    if (he == 0) v = ldexpf((float)m, -24);
    else if (he == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(1024 + m), he - 25);
    return neg ? -v : v;
}

/* fp16 product a*b with one roundTiesToEven rounding (exact in binary32 for
 * the operands used here: an integer in -15..15 and an fp16 value). */
uint16_t oracle_f16_mul(uint16_t a, uint16_t b) {
    return oracle_f32_to_f16(oracle_f16_to_f32(a) * oracle_f16_to_f32(b));
}

/* inference/baseline_kernels.py:48 */
static int awq_shift(int64_t col) {
    const int e = (int)(col % 8);
    return ((e / 2) + (e % 2) * 4) * 4;
}

/* Nibble at `shift` of a signed int32 word.  The reference shifts the signed
 * word arithmetically and masks with 0xF; any shift <= 28 followed by the mask
 * yields the same four bits whether the shift is arithmetic or logical, so the
 * unsigned shift here is the same function without implementation-defined C. */
static uint32_t nibble(int32_t word, int shift) {
    return ((uint32_t)word >> shift) & 0xFu;
}

void oracle_unpack(const int32_t* packed, int64_t rows, int64_t n, uint8_t* codes) {
    const int64_t pn = n / 8;
    for (int64_t i = 0; i < n; ++i)
        for (int64_t r = 0; r < rows; ++r)
            codes[r * n + i] = (uint8_t)nibble(packed[r * pn + i / 8], awq_shift(i));
}

/* w[k*N + i] = fp16((fp16(q) - fp16(z)) * s), loop over columns as the reference does. */
int oracle_dequant(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                   int64_t k, int64_t n, int32_t group_size, uint16_t* w) {
    if (group_size <= 0 || k % group_size || n % 8) return -1;
    const int64_t pn = n / 8;
    for (int64_t i = 0; i < n; ++i) {
        const int sh = awq_shift(i);
        for (int64_t r = 0; r < k; ++r) {
            const int64_t g = r / group_size;
            const int q = (int)nibble(qweight[r * pn + i / 8], sh);
            const int z = (int)nibble(qzeros[g * pn + i / 8], sh);
            /* fp16(q) - fp16(z): exact; x - x is +0 under round-to-nearest */
            const uint16_t diff = oracle_f32_to_f16((float)q - (float)z);
            w[r * n + i] = oracle_f16_mul(diff, scales[g * n + i]);
        }
    }
    return 0;
}

/* y[m*N + i] = sum_k x[m,k] * w[k,i], accumulated in binary64 in k order. */
int oracle_gemm_f64(const uint16_t* x, const int32_t* qweight, const int32_t* qzeros,
                    const uint16_t* scales, int64_t m, int64_t n, int64_t k,
                    int32_t group_size, uint16_t* w_scratch, double* y) {
    if (oracle_dequant(qweight, qzeros, scales, k, n, group_size, w_scratch)) return -1;
    for (int64_t a = 0; a < m; ++a) {
        for (int64_t i = 0; i < n; ++i) y[a * n + i] = 0.0;
        for (int64_t r = 0; r < k; ++r) {
            const double xv = (double)oracle_f16_to_f32(x[a * k + r]);
            const uint16_t* wr = w_scratch + r * n;
            for (int64_t i = 0; i < n; ++i) y[a * n + i] += xv * (double)oracle_f16_to_f32(wr[i]);
        }
    }
    return 0;
}
