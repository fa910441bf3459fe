"""fp16 output projection (lm_head) on a hand-written gfx950 GEMV.

The reference computes logits with ``nn.Linear(hidden_size, vocab_size,
bias=False)`` (``model/qwen2.py:253``, applied at ``:280``) over every
position and then keeps the last one (``inference/engine.py:93,127``).  At
decode the product is a GEMV over a 152064 x 3584 fp16 weight -- 1.09 GB per
token, the largest single read of a Qwen2-7B decode step.  This module
serves the positions actually needed (M <= 8 rows, e.g. the last position of
each sequence) through ``awq_fp16_linear`` of ``lib/libawq_w4a16.so``::

    lm_head_forward(x, weight) -> Tensor      # == F.linear(x, weight), fp16

* ``x``       fp16 ``[..., K]``, at most 8 rows once flattened
* ``weight``  fp16 ``[N, K]`` (``nn.Linear.weight``: ``[out, in]``)
* returns a new fp16 ``[..., N]``, fp32 accumulation, rounded once

Bad operands raise ``ValueError``; there is no torch fallback.
"""
from __future__ import annotations

import ctypes

import torch

from . import _native
from .awq_gemm import _check_device, _ptr, _OnDevice, _aligned16

__all__ = ["lm_head_forward", "MAX_ROWS"]

# Rows of x one call serves (the library's limit for this kernel).
MAX_ROWS = 8


def lm_head_forward(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``x @ weight.T`` in fp16 with fp32 accumulation (``F.linear`` without bias)."""
    if x.dtype != torch.float16 or weight.dtype != torch.float16:
        raise ValueError(f"x and weight must be float16, got {x.dtype}/{weight.dtype}")
    if weight.dim() != 2 or x.dim() < 1:
        raise ValueError("weight must be 2-D [N, K] and x at least 1-D")
    N, K = weight.shape
    if x.shape[-1] != K:
        raise ValueError(f"x has K = {x.shape[-1]}, weight has K = {K}")
    dev = _check_device(x, weight)
    in_shape = x.shape
    x_flat = _aligned16(x.reshape(-1, K).contiguous())
    M = x_flat.shape[0]
    if M > MAX_ROWS:
        raise ValueError(f"lm_head_forward serves at most {MAX_ROWS} rows, got {M}")
    weight = _aligned16(weight.contiguous())
    if out is None:
        out = torch.empty((M, N), dtype=torch.float16, device=dev)
    elif out.dtype != torch.float16 or tuple(out.shape) != (M, N) or not out.is_contiguous() or out.device != dev:
        raise ValueError("out must be a contiguous fp16 [M, N] tensor on the operands' device")
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    with _OnDevice(dev):
        st = _native.lib().awq_fp16_linear(_ptr(x_flat), _ptr(weight), _ptr(out), M, N, K, stream)
    if st in (_native.AWQ_ERR_BAD_DIMS, _native.AWQ_ERR_TOO_LARGE, _native.AWQ_ERR_PATH,
              _native.AWQ_ERR_MISALIGNED):
        raise ValueError(f"awq_fp16_linear rejected M={M} N={N} K={K}: {_native.error_string(st)}")
    _native.check(st, "awq_fp16_linear")
    return out.view(*in_shape[:-1], N)
