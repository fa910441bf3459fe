"""Writes the golden fixtures of the W4A16 AWQ path (``awq_golden_*.npz``).

The values are computed here from the reference's definitions with plain
Python integers and floats, independently of ``oracle/``:

* nibble shift of logical column n: ``4 * ((n % 8) // 2 + (n % 8) % 2 * 4)``
  (the closed form of ``kernels/awq_gemm.py:5-6`` and
  ``inference/baseline_kernels.py:46-48``), unpack ``(word >> shift) & 0xF``;
* dequant ``fp16((q - z) * s)`` (``test/compare_benchmark.py:87-92``): the
  product of an integer in -15..15 and an fp16 scale is exact in a Python
  float (binary64), and CPython's ``struct`` 'e' format rounds it to binary16
  with round-half-to-even (overflow handled as IEEE does: +-inf);
* GEMM ``y = x @ w`` (``test/compare_benchmark.py:94``) as ``math.fsum`` of
  the exact binary64 products: the correctly rounded exact sum.

Inputs come from ``random.Random`` with fixed seeds.  Two fixtures:

* ``awq_golden_small.npz``: M=5, K=256, N=64, G=128, random codes and
  scales in [0.002, 0.02);
* ``awq_golden_edge.npz``: M=3, K=128, N=64, G=128, scales chosen to reach
  the fp16 corner cases (subnormal results, ties, weights past 4096 and up
  to the fp16 maximum, overflow to infinity, negative scales, signed zeros),
  codes hitting every nibble value in every slot, and words with the sign
  bit set.

Run from the repository root: ``python tests/golden/make_golden.py``.
"""
from __future__ import annotations

import math
import os
import random
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
G = 128


def shift_of(n: int) -> int:
    e = n % 8
    return 4 * ((e // 2) + (e % 2) * 4)


def f16_bits(v: float) -> int:
    """binary16 bits of v rounded half-to-even (+-inf past the largest finite)."""
    try:
        return struct.unpack("<H", struct.pack("<e", v))[0]
    except OverflowError:
        return 0x7C00 if v > 0 else 0xFC00


def f16_value(bits: int) -> float:
    return struct.unpack("<e", struct.pack("<H", bits))[0]


def to_int32(u: int) -> int:
    return u - (1 << 32) if u & 0x80000000 else u


def pack(codes):
    """codes[r][n] (0..15) -> int32 words[r][n // 8] under the closed-form shifts."""
    rows, n = len(codes), len(codes[0])
    words = []
    for r in range(rows):
        row = []
        for j in range(n // 8):
            u = 0
            for c in range(8):
                u |= codes[r][8 * j + c] << shift_of(8 * j + c)
            row.append(to_int32(u))
        words.append(row)
    return words


def unpack_word(word: int, n: int) -> int:
    return (word >> shift_of(n)) & 0xF  # Python's >> on a negative int is arithmetic


def compute(x_bits, qweight, qzeros, s_bits, K, N):
    M = len(x_bits)
    w_bits = [[0] * N for _ in range(K)]
    for k in range(K):
        g = k // G
        for n in range(N):
            q = unpack_word(qweight[k][n // 8], n)
            z = unpack_word(qzeros[g][n // 8], n)
            w_bits[k][n] = f16_bits((q - z) * f16_value(s_bits[g][n]))
    w_val = [[f16_value(b) for b in row] for row in w_bits]
    x_val = [[f16_value(b) for b in row] for row in x_bits]
    y = [[0.0] * N for _ in range(M)]
    for m in range(M):
        for n in range(N):
            terms = [x_val[m][k] * w_val[k][n] for k in range(K)]
            if all(math.isfinite(t) for t in terms):
                y[m][n] = math.fsum(terms)
            else:  # IEEE sum of infinities: one sign gives that infinity, both give NaN
                signs = {math.copysign(1.0, t) for t in terms if math.isinf(t)}
                nan = any(math.isnan(t) for t in terms) or len(signs) > 1
                y[m][n] = math.nan if nan else math.inf * signs.pop()
    return w_bits, y


def save(name, x_bits, qweight, qzeros, s_bits, w_bits, y):
    path = os.path.join(HERE, name)
    np.savez_compressed(
        path,
        x_f16_bits=np.array(x_bits, dtype=np.uint16),
        qweight=np.array(qweight, dtype=np.int32),
        qzeros=np.array(qzeros, dtype=np.int32),
        scales_f16_bits=np.array(s_bits, dtype=np.uint16),
        w_f16_bits=np.array(w_bits, dtype=np.uint16),
        y_f64=np.array(y, dtype=np.float64),
    )
    print("wrote", path)


def small():
    M, K, N = 5, 256, 64
    rx, rq, rz, rs = (random.Random(s) for s in (101, 102, 103, 104))
    x_bits = [[f16_bits(rx.gauss(0.0, 1.0)) for _ in range(K)] for _ in range(M)]
    qcodes = [[rq.randrange(16) for _ in range(N)] for _ in range(K)]
    zcodes = [[rz.randrange(16) for _ in range(N)] for _ in range(K // G)]
    s_bits = [[f16_bits(rs.uniform(0.002, 0.02)) for _ in range(N)] for _ in range(K // G)]
    qweight, qzeros = pack(qcodes), pack(zcodes)
    w_bits, y = compute(x_bits, qweight, qzeros, s_bits, K, N)
    save("awq_golden_small.npz", x_bits, qweight, qzeros, s_bits, w_bits, y)


def edge():
    M, K, N = 3, 128, 64
    # Scales per column: corner cases first, the rest random in [2^-14, 2).
    special = [
        0x0001,  # smallest subnormal 2^-24: (q-z)*s is an exact subnormal
        0x03FF,  # largest subnormal
        0x0400,  # smallest normal
        0x3C00,  # 1.0: w = q - z exactly
        0x3C01,  # 1 + 2^-10: 3*s is a tie, rounds to even (up)
        0x3C03,  # 1 + 3*2^-10: 3*s is a tie, rounds to even (down)
        0x7BFF,  # 65504: |q-z| >= 2 overflows to +-inf
        0x5BFF,  # 255.875: 15*s = 3838.125 rounds to 3838
        0xBC00,  # -1.0
        0x8001,  # -2^-24
        0x0000,  # +0: w is +0 or -0 by the sign of q-z
        0x8000,  # -0
        0x2E66,  # ~0.1
        0x1000,  # 2^-11
        0x7800,  # 32768: overflow for |q-z| >= 2
        0x3555,  # ~1/3
        0x6000,  # 512: |w| up to 7680, past 4096
        0x6A00,  # 3072: |w| up to 46080, finite
        0x7400,  # 16384: finite for |q-z| <= 3, 65536 rounds to inf
        0x7A01,  # 49184: finite only for |q-z| <= 1
        0x0200,  # 2^-15 (subnormal): every product subnormal
        0x0155,  # subnormal with an odd mantissa
        0x0401,  # 2^-14 (1 + 2^-10): products at the subnormal/normal boundary
    ]
    rs = random.Random(201)
    s_row = special + [f16_bits(rs.uniform(2.0 ** -14, 2.0)) for _ in range(N - len(special))]
    s_bits = [s_row]
    # Weight codes: row r, column n -> (r + 5n) % 16 runs every value through every nibble slot.
    qcodes = [[(r + 5 * n) % 16 for n in range(N)] for r in range(K)]
    # Sign-bit words: rows 0..3 set nibble 7 (columns n % 8 == 7) to 8..15.
    for r in range(4):
        for j in range(N // 8):
            qcodes[r][8 * j + 7] = 8 + (r + j) % 8
    zcodes = [[(3 * n + 7) % 16 for n in range(N)]]
    rx = random.Random(202)
    x_bits = [[f16_bits(rx.uniform(-2.0, 2.0)) for _ in range(K)] for _ in range(M)]
    qweight, qzeros = pack(qcodes), pack(zcodes)
    w_bits, y = compute(x_bits, qweight, qzeros, s_bits, K, N)
    save("awq_golden_edge.npz", x_bits, qweight, qzeros, s_bits, w_bits, y)


if __name__ == "__main__":
    small()
    edge()
