"""SiLU * up on a hand-written gfx950 kernel (``awq_silu_mul``).

The reference splits the fused gate||up projection into two ``.contiguous()``
copies and runs its Triton ``silu_mul`` (``model/qwen2.py:187-194``,
``kernels/silu_mul.py:17-39``: ``x * sigmoid(x) * y`` in fp32, fp16 out).
``silu_mul_gate_up`` reads the fused output in place -- one pass instead of
three::

    silu_mul_gate_up(gate_up[..., 2I]) -> fp16 [..., I]
    silu_mul_forward(gate, up)          # the reference's two-operand form
"""
from __future__ import annotations

import ctypes

import torch

from . import _native
from .awq_gemm import _check_device, _ptr, _OnDevice, _aligned16

__all__ = ["silu_mul_gate_up", "silu_mul_forward"]


def silu_mul_gate_up(gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``silu(gate_up[..., :I]) * gate_up[..., I:]`` in fp32, rounded once to fp16."""
    if gate_up.dtype != torch.float16:
        raise ValueError(f"gate_up must be float16, got {gate_up.dtype}")
    two_i = gate_up.shape[-1]
    if two_i % 16 != 0:
        raise ValueError(f"the last dimension (2I = {two_i}) must be a multiple of 16")
    dev = _check_device(gate_up)
    I = two_i // 2
    g = _aligned16(gate_up.reshape(-1, two_i).contiguous())
    M = g.shape[0]
    if out is None:
        out = torch.empty((M, I), dtype=torch.float16, device=dev)
    elif out.dtype != torch.float16 or out.numel() != M * I or not out.is_contiguous() or out.device != dev:
        raise ValueError("out must be a contiguous fp16 tensor of M*I elements on the operand's device")
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    with _OnDevice(dev):
        st = _native.lib().awq_silu_mul(_ptr(g), _ptr(out), M, I, stream)
    _native.check(st, "awq_silu_mul")
    return out.view(*gate_up.shape[:-1], I)


def silu_mul_forward(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """The reference's ``silu_mul_forward(gate, up)`` (``kernels/silu_mul.py``)."""
    if gate.shape != up.shape:
        raise ValueError(f"gate {tuple(gate.shape)} and up {tuple(up.shape)} differ")
    return silu_mul_gate_up(torch.cat([gate, up], dim=-1))
