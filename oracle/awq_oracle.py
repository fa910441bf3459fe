"""numpy restatement of the reference's AWQ W4A16 dequant + matmul.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): used by ``tests/`` as
the checker and by ``bench.py``'s ``cpu_baseline`` leg; never by the product.

Reference semantics followed, function by function:

* ``AWQ_UNPACK_ORDER`` -- ``kernels/awq_gemm.py:5-6``: logical column ``n`` of
  a packed int32 sits in nibble ``ORD[n % 8]`` (shift ``4*ORD[n % 8]``).
* ``unpack_awq``       -- ``test/compare_benchmark.py:80-85``: arithmetic
  right shift of the signed int32 word, then ``& 0xF``.
* ``dequant_awq``      -- ``test/compare_benchmark.py:87-92`` (and
  ``kernels/awq_gemm.py:59``): ``w = (fp16(q) - fp16(z)) * s`` evaluated in
  fp16, i.e. an exact subtraction followed by one round-to-nearest-even.
* ``awq_gemm_oracle``  -- ``kernels/awq_gemm.py:223-224``: the fp16 dequantised
  weight multiplied by fp16 activations with a wide (fp32 or fp64)
  accumulator; the fp16 output is one final rounding.
* ``pack_awq``         -- inverse of ``unpack_awq``: the AutoAWQ packing that
  produced the checkpoints the reference loads (``model/qwen2.py:34-36``);
  the reference itself never packs, so this is pinned by round trips and by
  hand-worked words.
* ``fuse_columns``     -- ``model/qwen2.py:79-85,174-178``: QKV and gate||up
  fusion is ``torch.cat(dim=1)`` on the *packed* tensors.
"""
from __future__ import annotations

import numpy as np

# kernels/awq_gemm.py:5-6 -- order[i] = (i // 2) + (i % 2) * 4
AWQ_UNPACK_ORDER = (0, 4, 1, 5, 2, 6, 3, 7)
# The inverse permutation: nibble slot i holds logical column AWQ_PACK_ORDER[i].
AWQ_PACK_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)

GROUP_SIZE = 128


def pack_awq(codes: np.ndarray) -> np.ndarray:
    """Pack int4 codes ``[R, N]`` (values 0..15) into int32 ``[R, N // 8]``.

    Column ``n`` goes to nibble ``AWQ_UNPACK_ORDER[n % 8]`` of word ``n // 8``.
    """
    codes = np.asarray(codes)
    if codes.ndim != 2 or codes.shape[1] % 8:
        raise ValueError("codes must be [R, N] with N % 8 == 0")
    if codes.size and (codes.min() < 0 or codes.max() > 15):
        raise ValueError("int4 codes must lie in 0..15")
    r, n = codes.shape
    c = codes.reshape(r, n // 8, 8).astype(np.uint32)
    word = np.zeros((r, n // 8), dtype=np.uint32)
    for col in range(8):
        word |= c[:, :, col] << np.uint32(4 * AWQ_UNPACK_ORDER[col])
    return word.view(np.int32)


def unpack_awq(packed: np.ndarray) -> np.ndarray:
    """Unpack int32 ``[R, N // 8]`` into int4 codes ``[R, N]`` (uint8).

    Follows ``test/compare_benchmark.py:80-85``: ``(word >> 4*ORD) & 0xF`` on
    the signed word (arithmetic shift, then mask).
    """
    packed = np.asarray(packed)
    if packed.dtype != np.int32 or packed.ndim != 2:
        raise ValueError("packed must be a 2-D int32 array")
    r, pn = packed.shape
    shifts = (4 * np.asarray(AWQ_UNPACK_ORDER, dtype=np.int32)).reshape(1, 1, 8)
    codes = (packed[:, :, None] >> shifts) & 0xF
    return codes.reshape(r, pn * 8).astype(np.uint8)


def dequant_awq(qweight: np.ndarray, qzeros: np.ndarray, scales: np.ndarray,
                group_size: int = GROUP_SIZE) -> np.ndarray:
    """fp16 ``[K, N]`` dequantised weight, ``fp16((q - z) * s)``.

    ``test/compare_benchmark.py:87-92``: the codes are cast to fp16, the zero
    is subtracted in fp16 (exact: the difference lies in -15..15) and the
    product with the fp16 scale is rounded once to fp16 (round to nearest
    even; numpy evaluates fp16 products exactly in fp32 and rounds once).
    """
    k, pn = qweight.shape
    n = pn * 8
    if scales.dtype != np.float16 or scales.shape != (k // group_size, n):
        raise ValueError("scales must be fp16 [K/G, N]")
    if k % group_size:
        raise ValueError("K must be a multiple of group_size")
    if qzeros.shape != (k // group_size, pn):
        raise ValueError("qzeros must be int32 [K/G, N/8]")
    g = k // group_size
    w = unpack_awq(qweight).astype(np.float16).reshape(g, group_size, n)
    z = unpack_awq(qzeros).astype(np.float16).reshape(g, 1, n)
    s = scales.reshape(g, 1, n)
    return ((w - z) * s).reshape(k, n)


def dequant_awq_f32eval(qweight: np.ndarray, qzeros: np.ndarray, scales: np.ndarray,
                        group_size: int = GROUP_SIZE) -> np.ndarray:
    """``dequant_awq`` evaluated in float32, for large shapes.

    Same bits as ``dequant_awq``: ``q - z`` is an integer in -15..15 and the
    product of it with an fp16 scale has at most 16 significant bits, so the
    float32 product is exact and the single cast to fp16 is the one
    round-to-nearest-even that fp16 arithmetic performs.  The bit-identity is
    checked in tests/test_oracle.py.
    """
    k, pn = qweight.shape
    n = pn * 8
    g = k // group_size
    q = unpack_awq(qweight).astype(np.int16).reshape(g, group_size, n)
    z = unpack_awq(qzeros).astype(np.int16).reshape(g, 1, n)
    s = scales.astype(np.float32).reshape(g, 1, n)
    return ((q - z).astype(np.float32) * s).astype(np.float16).reshape(k, n)


def awq_gemm_oracle(x: np.ndarray, qweight: np.ndarray, qzeros: np.ndarray,
                    scales: np.ndarray, group_size: int = GROUP_SIZE,
                    accum=np.float64) -> np.ndarray:
    """``x @ dequant(W)`` with a wide accumulator; returns the unrounded result.

    ``kernels/awq_gemm.py:223-224``: fp16 dequantised weight, fp16
    activations, ``tl.dot`` accumulating in fp32.  ``accum=np.float64`` gives
    the reference value used by the tolerance gate.  Round to fp16 with
    ``.astype(np.float16)`` for the reference's output dtype.
    """
    x = np.asarray(x)
    if x.dtype != np.float16:
        raise ValueError("x must be fp16")
    k = qweight.shape[0]
    x2 = x.reshape(-1, x.shape[-1])
    if x2.shape[1] != k:
        raise ValueError("x last dim must equal K")
    w = dequant_awq(qweight, qzeros, scales, group_size).astype(accum)
    y = x2.astype(accum) @ w
    return y.reshape(*x.shape[:-1], w.shape[1])


def fuse_columns(*parts):
    """Concatenate several AWQ projections along N (``model/qwen2.py:79-85``).

    Each part is ``(qweight, qzeros, scales)``; packed words are whole
    8-column units, so concatenating packed tensors along dim 1 is exact.
    """
    qw = np.concatenate([p[0] for p in parts], axis=1)
    qz = np.concatenate([p[1] for p in parts], axis=1)
    sc = np.concatenate([p[2] for p in parts], axis=1)
    return qw, qz, sc


# ---------------------------------------------------------------------------
# Seeded synthetic inputs (the value distributions of the Qwen2-7B shape
# configurations): x ~ N(0,1) fp16; int4 weight and zero codes ~ U{0..15};
# scales ~ U[0.002, 0.02] fp16; group 128.  One generator per tensor, seeded
# seed+0 .. seed+3, so any tensor can be regenerated on its own.
# ---------------------------------------------------------------------------

def make_inputs(m: int, k: int, n: int, group_size: int = GROUP_SIZE, seed: int = 0,
                scale_lo: float = 0.002, scale_hi: float = 0.02):
    if k % group_size or n % 8:
        raise ValueError("need K % group_size == 0 and N % 8 == 0")
    g = k // group_size
    x = np.random.default_rng(seed + 0).standard_normal((m, k), dtype=np.float32).astype(np.float16)
    qcodes = np.random.default_rng(seed + 1).integers(0, 16, size=(k, n), dtype=np.uint8)
    zcodes = np.random.default_rng(seed + 2).integers(0, 16, size=(g, n), dtype=np.uint8)
    scales = np.random.default_rng(seed + 3).uniform(scale_lo, scale_hi, size=(g, n)).astype(np.float16)
    return x, pack_awq(qcodes), pack_awq(zcodes), scales


# ---------------------------------------------------------------------------
# Tolerance: max|y - y_ref| / max|y_ref| <= rtol, with y_ref the fp64
# accumulation of the exact fp16 dequantised weight.
# ---------------------------------------------------------------------------

def max_rel_err(y: np.ndarray, y_ref: np.ndarray) -> float:
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    denom = float(np.max(np.abs(y_ref))) if y_ref.size else 0.0
    num = float(np.max(np.abs(y - y_ref))) if y_ref.size else 0.0
    if denom == 0.0:
        return 0.0 if num == 0.0 else float("inf")
    return num / denom


def elementwise_violations(y: np.ndarray, y_ref: np.ndarray, rtol: float = 1e-2) -> int:
    """Count of elements with ``|y - y_ref| > rtol*|y_ref| + rtol*rms(y_ref)``."""
    y = np.asarray(y, dtype=np.float64)
    y_ref = np.asarray(y_ref, dtype=np.float64)
    if not y_ref.size:
        return 0
    rms = float(np.sqrt(np.mean(y_ref * y_ref)))
    return int(np.count_nonzero(np.abs(y - y_ref) > rtol * np.abs(y_ref) + rtol * rms))
