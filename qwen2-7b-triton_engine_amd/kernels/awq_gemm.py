"""W4A16 AWQ GEMM/GEMV: drop-in for ``kernels/awq_gemm.py`` of
Qwen2-7B-Triton_Engine, running hand-written gfx950 HIP kernels through the C
ABI of ``lib/libawq_w4a16.so`` (``include/awq_w4a16.h``).

Same entry point, argument meaning and result as the reference
(``kernels/awq_gemm.py:237-284``)::

    awq_gemm_forward(x, qweight, qzeros, scales, group_size=128) -> Tensor

* ``x``        fp16 ``[..., K]`` (any leading shape; flattened to ``[M, K]``)
* ``qweight``  int32 ``[K, N/8]``, AWQ nibble order (column n in nibble
  ``[0,4,1,5,2,6,3,7][n % 8]``)
* ``qzeros``   int32 ``[K/G, N/8]``, same packing
* ``scales``   fp16 ``[K/G, N]``; ``N = scales.shape[1]`` as in the reference
* returns a new fp16 ``[..., N]`` = ``x @ dequant(W)``, fp32 accumulation.

Differences from the reference, all on the error side: operands are checked
and a bad call raises ``ValueError`` (the reference launches anyway and lets
Triton's masks hide out-of-range reads); only ``group_size == 128`` is served
(the value the reference always uses, ``model/config.py:22``).  The work runs
on the caller's current stream: one kernel launch per call, or two when the
plan adds its split-K partials in a second, reduce launch (tile variants 7,
8, 9 and stream variant 3 with more than one split).  There is no
Triton, no torch dequant and no other fallback: without the HIP library the
call raises.

Workspace: like the reference's module-global ``_dequant_buffer``
(kernels/awq_gemm.py:234,255-262) one buffer per device, grown on demand,
held by the torch binding's registry and shared by every entry point -- here
it holds split-K partial sums, the kernels' arrival counters and fixed-point
slots (zero-filled once; each call leaves the counters and slots zero).  Calls that
share a device must therefore not run concurrently on different streams, the
same single-stream use the reference makes of its buffer.  The buffer is
graph-capture safe once it is large enough: capture after one eager call of
the largest shape, as the reference's engine warms up before capturing
(inference/engine.py:43-52); growing it during a capture raises.
"""
from __future__ import annotations

import ctypes

import torch

from . import _native

__all__ = ["awq_gemm_forward", "awq_gemm_forward_ex", "_dequant_to_fp16", "plan"]


_F16, _I32 = torch.float16, torch.int32


def _check_operands(x: torch.Tensor, qweight: torch.Tensor, qzeros: torch.Tensor,
                    scales: torch.Tensor, group_size: int):
    """Shape/dtype checks shared by every entry point; returns (K, N)."""
    if x.dtype is not _F16:
        raise ValueError(f"x must be float16, got {x.dtype}")
    if qweight.dtype is not _I32 or qzeros.dtype is not _I32:
        raise ValueError(f"qweight/qzeros must be int32, got {qweight.dtype}/{qzeros.dtype}")
    if scales.dtype is not _F16:
        raise ValueError(f"scales must be float16, got {scales.dtype}")
    if group_size != 128:
        raise ValueError(f"group_size {group_size} is not served (only 128)")
    ws, zs, ss = qweight.shape, qzeros.shape, scales.shape
    if len(ws) != 2 or len(zs) != 2 or len(ss) != 2 or x.dim() < 1:
        raise ValueError("qweight, qzeros and scales must be 2-D and x at least 1-D")
    K = x.shape[-1]
    N = ss[1]
    if N % 8 != 0 or N == 0:
        raise ValueError(f"N = scales.shape[1] = {N} must be a positive multiple of 8")
    if K == 0 or K % group_size != 0:
        raise ValueError(f"K = {K} must be a positive multiple of group_size {group_size}")
    if ws != (K, N // 8):
        raise ValueError(f"qweight shape {tuple(ws)} != (K, N/8) = {(K, N // 8)}")
    if zs != (K // group_size, N // 8):
        raise ValueError(f"qzeros shape {tuple(zs)} != (K/G, N/8) = {(K // group_size, N // 8)}")
    if ss != (K // group_size, N):
        raise ValueError(f"scales shape {tuple(ss)} != (K/G, N) = {(K // group_size, N)}")
    return K, N


def _check_device(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise ValueError(f"operands must be on a ROCm device, got {dev}")
    for t in tensors[1:]:
        if t.device != dev:
            raise ValueError(f"all operands must be on {dev}, got {t.device}")
    return dev


def _ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


# Per-device workspace buffers live in the torch binding's registry, shared
# by every entry point; earlier (smaller) buffers stay referenced so that
# graphs captured with them keep valid memory.
def _workspace(dev: torch.device, nbytes: int) -> torch.Tensor:
    """The device's workspace buffer, grown to at least ``nbytes`` (zero
    filled; refused while the current stream is being captured)."""
    return _native.binding().workspace(dev.index, int(nbytes))


def _workspace_buffers(dev: torch.device) -> list:
    """Every workspace buffer the device holds, oldest first."""
    return _native.binding().workspace_buffers(dev.index)


def _aligned16(t: torch.Tensor) -> torch.Tensor:
    """``t`` itself when its data starts on a 16-byte boundary, else a copy
    (a fresh allocation is aligned).  The kernels read x, scales and out with
    16-byte loads and stores and the C ABI refuses other addresses; the
    reference's Triton path takes any fp16 view, so an odd storage offset is
    copied here rather than refused."""
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _prepare(x, qweight, qzeros, scales, group_size):
    K, N = _check_operands(x, qweight, qzeros, scales, group_size)
    dev = _check_device(x, qweight, qzeros, scales)
    in_shape = x.shape
    x_flat = x if len(in_shape) == 2 else x.reshape(-1, K)     # kernels/awq_gemm.py:244-246
    # The reference passes strides to Triton; the C ABI takes dense operands.
    x_flat = _aligned16(x_flat.contiguous())
    qweight = qweight.contiguous()
    qzeros = qzeros.contiguous()
    scales = _aligned16(scales.contiguous())
    return in_shape, x_flat, qweight, qzeros, scales, K, N, dev


def _shaped(out: torch.Tensor, in_shape, N: int) -> torch.Tensor:
    """``out`` [M, N] viewed as ``[*in_shape[:-1], N]`` (kernels/awq_gemm.py:284)."""
    return out if len(in_shape) == 2 else out.view(*in_shape[:-1], N)


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_handle(dev: torch.device) -> int:
    """The current stream of ``dev`` as a raw hipStream_t value."""
    if _raw_stream is not None:
        return _raw_stream(dev.index)
    return torch.cuda.current_stream(dev).cuda_stream


# Plans of the AUTO dispatcher (or a forced path) per (M, N, K, group size,
# path, device): the planner's choice depends only on these and on the
# device's compute-unit count, so an eager call looks it up once instead of
# planning in C on every call.  Bounded: cleared when it grows past _PLAN_CACHE_MAX.
_plans: dict = {}
_PLAN_CACHE_MAX = 4096


class _OnDevice:
    """``torch.cuda.device(dev)`` unless ``dev`` is already current (the
    context manager costs a device switch and back on every call)."""

    __slots__ = ("idx", "prev")

    def __init__(self, dev: torch.device):
        self.idx = dev.index if dev.index is not None else torch.cuda.current_device()
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if cur != self.idx:
            self.prev = cur
            torch.cuda.set_device(self.idx)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False


def _plan_cached(M: int, N: int, K: int, group_size: int, path: int, dev: torch.device):
    """(plan, ctypes reference to it) for the shape on ``dev``."""
    key = (M, N, K, group_size, path, dev.index)
    e = _plans.get(key)
    if e is None:
        with _OnDevice(dev):
            p = _native.plan_for(M, N, K, group_size, path)
        if len(_plans) >= _PLAN_CACHE_MAX:
            _plans.clear()
        e = _plans[key] = (p, ctypes.byref(p))
    return e


def _launch(x_flat, qweight, qzeros, scales, out, M, N, K, group_size, dev, path=None, plan_obj=None,
            bias=None, residual=None):
    L = _native.lib()
    if plan_obj is not None:
        p, pref = plan_obj, ctypes.byref(plan_obj)
    else:
        p, pref = _plan_cached(M, N, K, group_size, _native.PATH_AUTO if path is None else path, dev)
    ws_bytes = p.workspace_bytes
    ws_ptr = 0
    if ws_bytes:
        ws = _workspace(dev, ws_bytes)
        ws_ptr, ws_bytes = ws.data_ptr(), ws.numel() * 4
    stream = _stream_handle(dev)
    with _OnDevice(dev):
        if bias is not None or residual is not None:
            st = L.awq_w4a16_gemm_epilogue(x_flat.data_ptr(), qweight.data_ptr(), qzeros.data_ptr(),
                                           scales.data_ptr(), 0 if bias is None else bias.data_ptr(),
                                           0 if residual is None else residual.data_ptr(), out.data_ptr(),
                                           M, N, K, group_size, ws_ptr, ws_bytes, pref, stream)
            where = "awq_w4a16_gemm_epilogue"
        else:
            st = L.awq_w4a16_gemm_planned(x_flat.data_ptr(), qweight.data_ptr(), qzeros.data_ptr(),
                                          scales.data_ptr(), out.data_ptr(), M, N, K, group_size, ws_ptr,
                                          ws_bytes, pref, stream)
            where = "awq_w4a16_gemm_planned"
    if st:
        _native.check(st, where)


def awq_gemm_forward(x: torch.Tensor, qweight: torch.Tensor, qzeros: torch.Tensor,
                     scales: torch.Tensor, group_size: int = 128) -> torch.Tensor:
    """``x @ dequant(qweight, qzeros, scales)`` in fp16 (kernels/awq_gemm.py:237-284).

    One call into the torch binding: the same checks as ``awq_gemm_forward_ex``
    (ValueError for a bad operand), the [M, K] flattening, the fp16 output, the
    AUTO plan (cached per shape and device), the shared workspace and the
    current stream, then the C ABI's ``awq_w4a16_gemm_planned``."""
    return _gemm(x, qweight, qzeros, scales, group_size)


def _gemm(x, qweight, qzeros, scales, group_size):
    global _gemm
    _gemm = _native.binding().awq_gemm_forward   # bound once: later calls go straight to C++
    return _gemm(x, qweight, qzeros, scales, group_size)


def awq_gemm_forward_ex(x: torch.Tensor, qweight: torch.Tensor, qzeros: torch.Tensor,
                        scales: torch.Tensor, group_size: int = 128, path: int | None = None,
                        plan_obj: "_native.Plan | None" = None, out: torch.Tensor | None = None,
                        bias: torch.Tensor | None = None, residual: torch.Tensor | None = None) -> torch.Tensor:
    """``awq_gemm_forward`` with the kernel path forced (``_native.PATH_*``) or an
    explicit plan (``_native.plan_skinny`` / ``plan``), optionally into ``out``,
    and optionally with the reference's follow-up adds fused into the store:
    ``bias`` fp16 ``[N]`` (``out + bias``, model/qwen2.py:45-46,108-109) and
    ``residual`` fp16 ``[..., N]`` (``residual + out``, :219-227), bit-identical
    to the unfused torch adds.  ``residual`` may be ``out`` itself."""
    in_shape, x_flat, qweight, qzeros, scales, K, N, dev = _prepare(x, qweight, qzeros, scales, group_size)
    M = x_flat.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.float16, device=dev)
    elif out.dtype != torch.float16 or out.numel() != M * N or not out.is_contiguous() or out.device != dev:
        raise ValueError("out must be a contiguous fp16 [M, N] tensor on the operands' device")
    elif out.data_ptr() % 16 != 0:
        # The kernels store 16-byte vectors: compute into an aligned buffer and copy back.
        if residual is not None and residual.data_ptr() == out.data_ptr():
            residual = residual.clone()
        tmp = awq_gemm_forward_ex(x, qweight, qzeros, scales, group_size, path=path, plan_obj=plan_obj,
                                  bias=bias, residual=residual)
        out.view(tmp.shape).copy_(tmp)
        return out.view(*in_shape[:-1], N)
    if bias is not None:
        if bias.dtype != torch.float16 or bias.numel() != N or bias.device != dev:
            raise ValueError(f"bias must be an fp16 [N={N}] tensor on {dev}")
        bias = bias.contiguous()
    if residual is not None:
        if residual.dtype != torch.float16 or residual.numel() != M * N or residual.device != dev:
            raise ValueError(f"residual must be an fp16 tensor of M*N = {M * N} elements on {dev}")
        residual = residual.contiguous()
    _launch(x_flat, qweight, qzeros, scales, out, M, N, K, group_size, dev, path=path, plan_obj=plan_obj,
            bias=bias, residual=residual)
    return out.view(*in_shape[:-1], N)


def _dequant_to_fp16(qweight: torch.Tensor, qzeros: torch.Tensor, scales: torch.Tensor,
                     out_buf: torch.Tensor, group_size: int = 128) -> torch.Tensor:
    """Dense fp16 ``[K, N]`` weight ``(q - z) * s`` into ``out_buf``, bit-exact
    (kernels/awq_gemm.py:66-87)."""
    K = qweight.shape[0]
    N = scales.shape[1]
    dummy_x = torch.empty((0, K), dtype=torch.float16, device=qweight.device)
    _check_operands(dummy_x, qweight, qzeros, scales, group_size)
    dev = _check_device(qweight, qzeros, scales, out_buf)
    if out_buf.dtype != torch.float16 or tuple(out_buf.shape) != (K, N) or not out_buf.is_contiguous():
        raise ValueError(f"out_buf must be a contiguous fp16 tensor of shape {(K, N)}")
    qweight, qzeros, scales = qweight.contiguous(), qzeros.contiguous(), _aligned16(scales.contiguous())
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    with _OnDevice(dev):
        st = _native.lib().awq_w4a16_dequant(_ptr(qweight), _ptr(qzeros), _ptr(scales), _ptr(out_buf),
                                             N, K, group_size, stream)
    _native.check(st, "awq_w4a16_dequant")
    return out_buf


def plan(M: int, N: int, K: int, group_size: int = 128, path: int = _native.PATH_AUTO) -> dict:
    """What the shape dispatcher launches for ``[M, K] x [K, N]`` (host only)."""
    return _native.plan_for(M, N, K, group_size, path).as_dict()
