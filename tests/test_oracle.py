"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

The reference ships no golden vectors, known-answer tests or fixtures for this
path, so each oracle function is pinned here by checks chosen so that a
plausible mistake (a wrong nibble order, a dropped zero, a wrong group index,
a transposed operand, double rounding) fails at least one of them:

=====================  ====================================================
oracle function        pinned by
=====================  ====================================================
unpack_awq             hand-worked words (incl. sign-bit words); the golden
                       fixtures; round trip with pack_awq; C == numpy
pack_awq               hand-worked word 0x75316420; round trip
dequant_awq            hand-worked fp16 products (ties, subnormals,
                       overflow, signed zeros); the golden fixtures (CPython
                       struct rounding, independent of numpy); exhaustive
                       agreement of numpy, the C restatement and the fp32
                       evaluation over every (q - z) and every fp16 scale
awq_gemm_oracle        golden fixtures (math.fsum, correctly rounded);
                       one-hot rows reproduce the dequantised weight exactly;
                       integer weights give the exact integer product;
                       pure-Python brute force on a tiny shape; C == numpy
fuse_columns           fused GEMM == concatenation of the parts' GEMMs
=====================  ====================================================

``test_planted_mistakes`` checks that the checks bite: each mutant oracle
(one plausible mistake planted in a copy of the oracle) fails at least one.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import awq_oracle as O
from oracle import c_oracle as C

# The edge fixture overflows fp16 on purpose (infinities, then NaN sums).
pytestmark = [pytest.mark.filterwarnings("ignore:overflow encountered:RuntimeWarning"),
              pytest.mark.filterwarnings("ignore:invalid value encountered:RuntimeWarning")]

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _golden(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _fixture_operands(d):
    x = d["x_f16_bits"].view(np.float16)
    s = d["scales_f16_bits"].view(np.float16)
    return x, d["qweight"], d["qzeros"], s


# ---------------------------------------------------------------------------
# Hand-worked known answers
# ---------------------------------------------------------------------------

def test_unpack_known_words():
    # Nibble i of 0x76543210 holds the value i; column n reads nibble ORD[n % 8],
    # ORD = [(i // 2) + (i % 2) * 4] = [0, 4, 1, 5, 2, 6, 3, 7].
    w = np.array([[0x76543210]], dtype=np.uint32).view(np.int32)
    assert O.unpack_awq(w).tolist() == [[0, 4, 1, 5, 2, 6, 3, 7]]
    # 0xFEDCBA98 is negative as int32; nibble i holds 8 + i.  Arithmetic shift
    # then & 0xF must still give the nibbles.
    w = np.array([[0xFEDCBA98]], dtype=np.uint32).view(np.int32)
    assert int(w[0, 0]) < 0
    assert O.unpack_awq(w).tolist() == [[8, 12, 9, 13, 10, 14, 11, 15]]
    # Two words: the second word's columns are 8..15.
    w = np.array([[0x00000000, 0xF0000000]], dtype=np.uint32).view(np.int32)
    assert O.unpack_awq(w).tolist() == [[0] * 8 + [0, 0, 0, 0, 0, 0, 0, 15]]
    assert C.unpack(w).tolist() == O.unpack_awq(w).tolist()


def test_pack_known_word():
    # Columns 0..7 with values 0..7: column n goes to nibble ORD[n], so nibble
    # i holds PACK[i] = [0, 2, 4, 6, 1, 3, 5, 7] -> 0x75316420.
    codes = np.arange(8, dtype=np.uint8).reshape(1, 8)
    assert O.pack_awq(codes).view(np.uint32).tolist() == [[0x75316420]]
    codes = np.full((1, 8), 15, dtype=np.uint8)
    assert O.pack_awq(codes).view(np.uint32).tolist() == [[0xFFFFFFFF]]


def _dq_one(q, z, s_bits, dequant=None):
    """Dequantise a single (q, z, s) through a [128, 8] problem; returns fp16 bits."""
    dequant = dequant or O.dequant_awq
    codes = np.zeros((128, 8), dtype=np.uint8)
    codes[:, 3] = q
    zc = np.zeros((1, 8), dtype=np.uint8)
    zc[0, 3] = z
    s = np.zeros((1, 8), dtype=np.uint16)
    s[0, 3] = s_bits
    w = dequant(O.pack_awq(codes), O.pack_awq(zc), s.view(np.float16))
    return int(w.view(np.uint16)[5, 3])


# (q, z, scale bits, expected fp16 bits), each worked by hand.
DEQUANT_KATS = [
    (15, 0, 0x3C00, 0x4B80),  # 15 * 1.0 = 15 = 1.875 * 2^3: exp 18, frac 0x380
    (0, 15, 0x3C00, 0xCB80),  # -15
    (7, 7, 0x3C00, 0x0000),   # q == z: +0 (x - x = +0), times positive s stays +0
    (7, 7, 0xBC00, 0x8000),   # +0 times -1 is -0
    (8, 7, 0x0001, 0x0001),   # 1 * 2^-24: smallest subnormal, exact
    (15, 0, 0x0001, 0x000F),  # 15 * 2^-24: exact subnormal
    (3, 0, 0x3C01, 0x4202),   # 3 * (1 + 2^-10) = 3 + 1.5 ulp(2^-9): tie, to even -> 3 + 2^-8
    (0, 3, 0x3C01, 0xC202),   # the negative of the same tie
    (3, 0, 0x3C03, 0x4204),   # 3 * (1 + 3*2^-10) = 3 + 4.5 ulp: tie, to even -> 3 + 2^-7
    (15, 0, 0x5BFF, 0x6B7F),  # 15 * 255.875 = 3838.125 -> 3838 (ulp 2 in [2048, 4096))
    (1, 0, 0x7BFF, 0x7BFF),   # 65504 * 1: largest finite
    (2, 0, 0x7BFF, 0x7C00),   # 131008 overflows to +inf
    (0, 2, 0x7BFF, 0xFC00),   # -inf
    (5, 2, 0x3555, 0x3C00),   # 3 * 0.333251953125 = 0.999755859375 = 1 - 2^-12: tie, to even -> 1.0
]


@pytest.mark.parametrize("q,z,s_bits,expect", DEQUANT_KATS)
def test_dequant_known_products(q, z, s_bits, expect):
    assert _dq_one(q, z, s_bits) == expect
    assert _dq_one(q, z, s_bits, O.dequant_awq_f32eval) == expect
    assert _dq_one(q, z, s_bits, C.dequant) == expect


def test_c_fp16_rounding_known_values():
    assert C.f32_to_f16_bits(1.0) == 0x3C00
    assert C.f32_to_f16_bits(65504.0) == 0x7BFF
    assert C.f32_to_f16_bits(65520.0) == 0x7C00      # halfway to 2^16 rounds to even -> inf
    assert C.f32_to_f16_bits(65519.99) == 0x7BFF
    assert C.f32_to_f16_bits(2.0 ** -25) == 0x0000   # half the smallest subnormal: tie to even (0)
    assert C.f32_to_f16_bits(3 * 2.0 ** -25) == 0x0002  # 1.5 units: tie to even (2)
    assert C.f32_to_f16_bits(-0.0) == 0x8000
    assert C.f32_to_f16_bits(float("inf")) == 0x7C00


# ---------------------------------------------------------------------------
# Golden fixtures (tests/golden/make_golden.py: plain Python + struct + fsum)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["awq_golden_small.npz", "awq_golden_edge.npz"])
def test_golden_dequant_bit_exact(name):
    d = _golden(name)
    x, qw, qz, s = _fixture_operands(d)
    expect = d["w_f16_bits"]
    for dq in (O.dequant_awq, O.dequant_awq_f32eval, C.dequant):
        assert np.array_equal(dq(qw, qz, s).view(np.uint16), expect), dq.__name__


@pytest.mark.parametrize("name", ["awq_golden_small.npz", "awq_golden_edge.npz"])
def test_golden_gemm(name):
    d = _golden(name)
    x, qw, qz, s = _fixture_operands(d)
    y_ref = d["y_f64"]
    for y in (O.awq_gemm_oracle(x, qw, qz, s), C.gemm_f64(x, qw, qz, s)):
        fin = np.isfinite(y_ref)
        assert np.array_equal(np.isnan(y), np.isnan(y_ref))
        assert np.array_equal(y[np.isinf(y_ref)], y_ref[np.isinf(y_ref)])
        # fp64 accumulation in another order vs the correctly rounded sum: a few ulps of the
        # largest partial sum.
        scale = np.max(np.abs(y_ref[fin])) if fin.any() else 1.0
        assert np.max(np.abs(y[fin] - y_ref[fin])) <= 1e-12 * scale


def test_golden_edge_covers_corner_cases():
    """The edge fixture really reaches the cases it is meant to pin."""
    d = _golden("awq_golden_edge.npz")
    w = d["w_f16_bits"]
    exp = (w >> 10) & 0x1F
    frac = w & 0x3FF
    assert np.any((exp == 0) & (frac != 0))            # subnormal results
    assert np.any(w == 0x7C00) and np.any(w == 0xFC00)  # overflow both signs
    assert np.any(w == 0x0000) and np.any(w == 0x8000)  # both zeros
    assert np.any(d["qweight"] < 0)                     # sign-bit words
    codes = O.unpack_awq(d["qweight"])
    for col in range(8):  # every value in every nibble slot
        assert set(np.unique(codes[:, col::8]).tolist()) == set(range(16))


# ---------------------------------------------------------------------------
# Exhaustive and algebraic checks
# ---------------------------------------------------------------------------

def test_dequant_exhaustive_all_differences_all_scales():
    """Every (q, z) pair and every fp16 scale bit pattern: numpy fp16 arithmetic,
    the C restatement and the fp32 evaluation agree bit for bit (NaN scales
    compared as NaN)."""
    gs = 16                               # group of 16 rows: row r has q = r
    k = 16 * gs                           # group g has z = g -> q - z covers -15..15
    n = 65536                             # column n has scale bits n
    codes = np.tile((np.arange(k) % gs).astype(np.uint8)[:, None], (1, n))
    zc = np.tile(np.arange(16, dtype=np.uint8)[:, None], (1, n))
    qw, qz = O.pack_awq(codes), O.pack_awq(zc)
    s = np.tile(np.arange(n, dtype=np.uint32).astype(np.uint16)[None, :], (16, 1)).view(np.float16)
    a = O.dequant_awq(qw, qz, s, gs)
    b = O.dequant_awq_f32eval(qw, qz, s, gs)
    c = C.dequant(qw, qz, s, gs)
    nan = np.isnan(a)
    assert np.array_equal(nan, np.isnan(b)) and np.array_equal(nan, np.isnan(c))
    assert np.array_equal(a.view(np.uint16)[~nan], b.view(np.uint16)[~nan])
    assert np.array_equal(a.view(np.uint16)[~nan], c.view(np.uint16)[~nan])


def test_pack_unpack_round_trip():
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 16, size=(37, 8 * 29), dtype=np.uint8)
    packed = O.pack_awq(codes)
    assert np.array_equal(O.unpack_awq(packed), codes)
    assert np.array_equal(C.unpack(packed), codes)
    words = rng.integers(-(2 ** 31), 2 ** 31, size=(19, 23), dtype=np.int64).astype(np.int32)
    assert np.array_equal(O.pack_awq(O.unpack_awq(words)), words)


def test_one_hot_rows_reproduce_weight():
    """x = e_k makes y the k-th dequantised row exactly (1 * w is exact)."""
    _, qw, qz, s = O.make_inputs(1, 256, 48, seed=3)
    w = O.dequant_awq(qw, qz, s)
    for k in (0, 1, 127, 128, 255):
        x = np.zeros((1, 256), dtype=np.float16)
        x[0, k] = 1.0
        y = O.awq_gemm_oracle(x, qw, qz, s, accum=np.float32).astype(np.float16)
        assert np.array_equal(y.view(np.uint16)[0], w.view(np.uint16)[k])


def test_integer_weights_exact_product():
    """s = 1, z = 0, small-integer x: the GEMM is an integer matmul."""
    rng = np.random.default_rng(9)
    k, n, m = 256, 40, 3
    codes = rng.integers(0, 16, size=(k, n), dtype=np.uint8)
    xi = rng.integers(-3, 4, size=(m, k))
    qw = O.pack_awq(codes)
    qz = O.pack_awq(np.zeros((k // 128, n), dtype=np.uint8))
    s = np.ones((k // 128, n), dtype=np.float16)
    y = O.awq_gemm_oracle(xi.astype(np.float16), qw, qz, s)
    assert np.array_equal(y, (xi @ codes.astype(np.int64)).astype(np.float64))


def test_brute_force_tiny():
    """Pure-Python loops straight from the definitions on a tiny shape."""
    x, qw, qz, s = O.make_inputs(2, 128, 16, seed=21)
    y = O.awq_gemm_oracle(x, qw, qz, s)
    for m in range(2):
        for n in range(16):
            sh = 4 * ((n % 8) // 2 + (n % 8) % 2 * 4)
            z = (int(qz[0, n // 8]) >> sh) & 0xF
            acc = 0.0
            for k in range(128):
                q = (int(qw[k, n // 8]) >> sh) & 0xF
                wv = float(np.float16(float(q - z) * float(s[0, n])))
                acc += float(x[m, k]) * wv
            assert abs(acc - y[m, n]) <= 1e-12 * max(1.0, abs(acc))


def test_c_and_numpy_oracles_agree():
    x, qw, qz, s = O.make_inputs(3, 384, 72, seed=11)
    assert np.array_equal(C.dequant(qw, qz, s).view(np.uint16), O.dequant_awq(qw, qz, s).view(np.uint16))
    yc = C.gemm_f64(x, qw, qz, s)
    yn = O.awq_gemm_oracle(x, qw, qz, s)
    assert np.max(np.abs(yc - yn)) <= 1e-12 * np.max(np.abs(yn))


def test_fuse_columns_equals_parts():
    parts = [O.make_inputs(2, 256, n, seed=30 + i)[1:] for i, n in enumerate((24, 8, 40))]
    x = O.make_inputs(2, 256, 8, seed=40)[0]
    fused = O.fuse_columns(*parts)
    y = O.awq_gemm_oracle(x, *fused)
    y_parts = np.concatenate([O.awq_gemm_oracle(x, *p) for p in parts], axis=1)
    assert np.array_equal(y, y_parts)


def test_rejects_bad_shapes():
    _, qw, qz, s = O.make_inputs(1, 256, 16, seed=1)
    with pytest.raises(ValueError):
        O.dequant_awq(qw[:200], qz, s)
    with pytest.raises(ValueError):
        O.dequant_awq(qw, qz, s.astype(np.float32))
    with pytest.raises(ValueError):
        O.pack_awq(np.full((1, 8), 16, dtype=np.uint8))
    with pytest.raises(ValueError):
        O.awq_gemm_oracle(np.zeros((1, 128), dtype=np.float16), qw, qz, s)


def test_tolerance_helpers():
    y_ref = np.array([[1.0, -2.0, 4.0]])
    assert O.max_rel_err(y_ref, y_ref) == 0.0
    assert O.max_rel_err(y_ref + [[0.0, 0.0, 0.04]], y_ref) == pytest.approx(0.01)
    assert O.elementwise_violations(y_ref, y_ref) == 0
    assert O.elementwise_violations(y_ref + [[0.0, 0.5, 0.0]], y_ref) == 1


# ---------------------------------------------------------------------------
# The checks bite: plant one mistake at a time in a copy of the oracle
# ---------------------------------------------------------------------------

def _unpack_with(order):
    def unpack(packed):
        shifts = (4 * np.asarray(order, dtype=np.int32)).reshape(1, 1, 8)
        r, pn = packed.shape
        return ((packed[:, :, None] >> shifts) & 0xF).reshape(r, pn * 8).astype(np.uint8)
    return unpack


def _dequant_with(unpack=O.unpack_awq, drop_zero=False, group_shift=0, double_round=False,
                  scale_transposed=False):
    def dequant(qweight, qzeros, scales, group_size=128):
        k, pn = qweight.shape
        n = pn * 8
        g = k // group_size
        w = unpack(qweight).astype(np.float16).reshape(g, group_size, n)
        z = unpack(qzeros).astype(np.float16)
        if group_shift:
            z = np.roll(z, group_shift, axis=0)
        z = z.reshape(g, 1, n)
        s = scales[::-1] if scale_transposed else scales
        s = s.reshape(g, 1, n)
        if drop_zero:
            z = np.zeros_like(z)
        if double_round:  # round (q - z) * s through fp32 -> bf16-like truncation first
            v = ((w.astype(np.float32) - z.astype(np.float32)) * s.astype(np.float32))
            v = (v.view(np.uint32) & np.uint32(0xFFFFE000)).view(np.float32)
            return v.astype(np.float16).reshape(k, n)
        return ((w - z) * s).reshape(k, n)
    return dequant


def _gemm_with(dequant, transpose_x=False):
    def gemm(x, qweight, qzeros, scales, group_size=128):
        w = dequant(qweight, qzeros, scales, group_size).astype(np.float64)
        xx = x.astype(np.float64)
        if transpose_x:  # walk x's K axis backwards (a transposed/reversed operand)
            xx = xx[:, ::-1]
        return xx @ w
    return gemm


def _pin_failures(unpack, dequant, gemm) -> list:
    """Runs the pinning checks above against an oracle candidate; returns the names
    of the checks it fails."""
    fails = []
    w = np.array([[0x76543210]], dtype=np.uint32).view(np.int32)
    if unpack(w).tolist() != [[0, 4, 1, 5, 2, 6, 3, 7]]:
        fails.append("unpack_kat")
    for q, z, sb, expect in DEQUANT_KATS:
        if _dq_one(q, z, sb, dequant) != expect:
            fails.append("dequant_kat")
            break
    for name in ("awq_golden_small.npz", "awq_golden_edge.npz"):
        d = _golden(name)
        x, qw, qz, s = _fixture_operands(d)
        if not np.array_equal(dequant(qw, qz, s).view(np.uint16), d["w_f16_bits"]):
            fails.append(f"golden_dequant:{name}")
        y, y_ref = gemm(x, qw, qz, s), d["y_f64"]
        fin = np.isfinite(y_ref)
        if not np.allclose(y[fin], y_ref[fin], rtol=0, atol=1e-9 * np.max(np.abs(y_ref[fin]))):
            fails.append(f"golden_gemm:{name}")
    return fails


def test_real_oracle_passes_pin_checks():
    assert _pin_failures(O.unpack_awq, O.dequant_awq, _gemm_with(O.dequant_awq)) == []


MUTANTS = {
    "nibble order = pack order": dict(unpack=_unpack_with(O.AWQ_PACK_ORDER)),
    "plain nibble order": dict(unpack=_unpack_with(tuple(range(8)))),
    "zero not subtracted": dict(drop_zero=True),
    "zeros of the wrong group": dict(group_shift=1),
    "scale groups reversed": dict(scale_transposed=True),
    "extra rounding step": dict(double_round=True),
    "x reversed along K": dict(transpose_x=True),
}


@pytest.mark.parametrize("mutant", sorted(MUTANTS))
def test_planted_mistakes(mutant):
    kw = dict(MUTANTS[mutant])
    transpose_x = kw.pop("transpose_x", False)
    unpack = kw.get("unpack", O.unpack_awq)
    dequant = _dequant_with(**kw)
    gemm = _gemm_with(dequant, transpose_x=transpose_x)
    assert _pin_failures(unpack, dequant, gemm), f"planted mistake '{mutant}' passed every check"


# ---------------------------------------------------------------------------
# The timed CPU baseline (oracle/cpu_baseline.py) computes the same thing
# ---------------------------------------------------------------------------

def _cpu_baseline(x, qw, qz, s):
    import torch

    from oracle.cpu_baseline import torch_awq_gemm_cpu
    T = torch.from_numpy
    return torch_awq_gemm_cpu(T(np.ascontiguousarray(x)), T(np.ascontiguousarray(qw)),
                              T(np.ascontiguousarray(qz)), T(np.ascontiguousarray(s))).numpy()


def test_cpu_baseline_one_hot_reproduces_oracle_weight():
    """One-hot rows through the timed torch-CPU baseline return the oracle's
    fp16 weight bit for bit, on random scales and on the edge fixture's
    finite columns: the baseline's unpack order, zero subtraction, group
    indexing and single fp16 rounding are the oracle's."""
    _, qw, qz, s = O.make_inputs(1, 384, 136, seed=81)
    d = _golden("awq_golden_edge.npz")
    _, qw_e, qz_e, s_e = _fixture_operands(d)
    keep = np.isfinite(d["w_f16_bits"].view(np.float16)).all(axis=0)
    for qw_, qz_, s_, cols in ((qw, qz, s, slice(None)), (qw_e, qz_e, s_e, keep)):
        k = qw_.shape[0]
        x = np.eye(k, dtype=np.float16)
        y = _cpu_baseline(x, qw_, qz_, s_)[:, cols]
        w = O.dequant_awq(qw_, qz_, s_)[:, cols]
        assert np.array_equal((y + np.float16(0)).view(np.uint16), (w + np.float16(0)).view(np.uint16))


@pytest.mark.parametrize("name", ["awq_golden_small.npz"])
def test_cpu_baseline_matches_golden_gemm(name):
    d = _golden(name)
    x, qw, qz, s = _fixture_operands(d)
    y = _cpu_baseline(x, qw, qz, s).astype(np.float64)
    assert O.max_rel_err(y, d["y_f64"]) <= 1e-3
    assert O.elementwise_violations(y, d["y_f64"], 1e-2) == 0


def test_cpu_baseline_matches_oracle_random():
    for m, k, n in ((1, 1024, 512), (5, 512, 264), (33, 256, 64)):
        x, qw, qz, s = O.make_inputs(m, k, n, seed=82 + m)
        y = _cpu_baseline(x, qw, qz, s).astype(np.float64)
        y_ref = O.awq_gemm_oracle(x, qw, qz, s).astype(np.float64)
        assert O.max_rel_err(y, y_ref) <= 1e-2 and O.elementwise_violations(y, y_ref, 1e-2) == 0
