"""Algorithmic work of one W4A16 AWQ GEMM and the MI355X peaks it is priced at.

Bytes one GEMM must move at minimum (each operand read or written once):

    B = K*N/2            int4 weight codes (qweight)
      + (K/G)*(N/8)*4    packed zeros (qzeros)
      + (K/G)*N*2        fp16 scales
      + M*K*2            fp16 activations x
      + M*N*2            fp16 output

Flops: F = 2*M*N*K.  Decode shapes (small M) are priced against HBM
bandwidth, prefill shapes against dense fp16 MFMA throughput.
"""
from __future__ import annotations

HBM_PEAK_BPS = 8.0e12                 # MI355X HBM3E, bytes/s
MFMA_F16_DENSE_PEAK_FLOPS = 2.5166e15  # MI355X dense fp16 MFMA, flop/s (256 CU x 2.4 GHz x 4096)
RIDGE_FLOP_PER_BYTE = MFMA_F16_DENSE_PEAK_FLOPS / HBM_PEAK_BPS


def algorithmic_bytes(M: int, N: int, K: int, group_size: int = 128) -> int:
    g = K // group_size
    return K * N // 2 + g * (N // 8) * 4 + g * N * 2 + M * K * 2 + M * N * 2


def flops(M: int, N: int, K: int) -> int:
    return 2 * M * N * K


def bound(M: int, N: int, K: int, group_size: int = 128) -> str:
    """'hbm' when the arithmetic intensity is below the ridge point, else 'mfma'."""
    ai = flops(M, N, K) / algorithmic_bytes(M, N, K, group_size)
    return "hbm" if ai < RIDGE_FLOP_PER_BYTE else "mfma"


def roofline_fraction(M: int, N: int, K: int, seconds: float, group_size: int = 128):
    """(bound, achieved, peak, unit, fraction) for one GEMM taking ``seconds``."""
    b = bound(M, N, K, group_size)
    if b == "hbm":
        achieved = algorithmic_bytes(M, N, K, group_size) / seconds / 1e9
        peak = HBM_PEAK_BPS / 1e9
        unit = "GB/s"
    else:
        achieved = flops(M, N, K) / seconds / 1e12
        peak = MFMA_F16_DENSE_PEAK_FLOPS / 1e12
        unit = "TFLOP/s"
    return b, achieved, peak, unit, achieved / peak


# Per-layer linear shapes of Qwen2-7B (hidden 3584, 28 Q heads / 4 KV heads of
# 128, intermediate 18944): (name, K, N).  The fused entries are the shapes
# the reference engine actually calls (model/qwen2.py:79-85,174-178).
QWEN2_7B_LINEARS = (
    ("q_proj", 3584, 3584),
    ("k_proj", 3584, 512),
    ("v_proj", 3584, 512),
    ("o_proj", 3584, 3584),
    ("gate_proj", 3584, 18944),
    ("up_proj", 3584, 18944),
    ("down_proj", 18944, 3584),
)
QWEN2_7B_FUSED = (
    ("qkv_proj", 3584, 4608),
    ("gate_up_proj", 3584, 37888),
)
