"""ctypes binding of ``lib/libawq_w4a16.so`` (C ABI: ``include/awq_w4a16.h``).

Loading fails loudly when the library is missing: there is no fallback path.
Build it with ``python qwen2-7b-triton_engine_amd/build.py``.
"""
from __future__ import annotations

import ctypes
import os

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_ROOT, "lib", "libawq_w4a16.so")

ABI_VERSION = 2

AWQ_OK = 0
AWQ_ERR_NULL_POINTER = -1
AWQ_ERR_BAD_DIMS = -2
AWQ_ERR_GROUP_SIZE = -3
AWQ_ERR_MISALIGNED = -4
AWQ_ERR_WORKSPACE = -5
AWQ_ERR_LAUNCH = -6
AWQ_ERR_PATH = -7
AWQ_ERR_TOO_LARGE = -8
AWQ_ERR_SCRATCH = -9
AWQ_ERR_CAPTURE = -10
NOALLOC_SCRATCH_BYTES = 32 << 20
SLOT_BYTES = 2 << 20   # fixed-point slot region of a workspace (AWQ_W4A16_SLOT_BYTES)

PATH_AUTO = 0
PATH_SKINNY = 1
PATH_TILE = 2
PATH_GEMV = 3
PATH_STREAM = 5
PATH_NAMES = {PATH_AUTO: "auto", PATH_SKINNY: "skinny", PATH_TILE: "tile", PATH_GEMV: "gemv", PATH_STREAM: "stream"}


class Plan(ctypes.Structure):
    """Mirror of ``awq_w4a16_plan``."""

    _fields_ = [
        ("path", ctypes.c_int32),
        ("variant", ctypes.c_int32),
        ("tile_m", ctypes.c_int32),
        ("tile_n", ctypes.c_int32),
        ("rows_per_wave", ctypes.c_int32),
        ("k_waves", ctypes.c_int32),
        ("split_k", ctypes.c_int32),
        ("block_threads", ctypes.c_int32),
        ("factored_scale", ctypes.c_int32),
        ("depth", ctypes.c_int32),
        ("grid", ctypes.c_int64),
        ("workspace_bytes", ctypes.c_uint64),
        ("lds_bytes", ctypes.c_uint64),
    ]

    def as_dict(self) -> dict:
        d = {name: getattr(self, name) for name, _ in self._fields_}
        d["path_name"] = PATH_NAMES.get(self.path, "?")
        return d


# Every symbol include/awq_w4a16.h declares, with its ctypes signature.
_VP = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
SIGNATURES = {
    "awq_w4a16_abi_version": (ctypes.c_int, []),
    "awq_w4a16_error_string": (ctypes.c_char_p, [ctypes.c_int]),
    "awq_w4a16_plan_for": (ctypes.c_int, [_I64, _I64, _I64, _I32, _I32, ctypes.POINTER(Plan)]),
    "awq_w4a16_plan_skinny": (ctypes.c_int, [_I64, _I64, _I64, _I32, _I32, _I32, _I32, _I32,
                                             ctypes.POINTER(Plan)]),
    "awq_w4a16_counter_bytes": (ctypes.c_size_t, []),
    "awq_w4a16_plan_gemv": (ctypes.c_int, [_I64, _I64, _I64, _I32, _I32, _I32, _I32, _I32, _I32, _I32,
                                           ctypes.POINTER(Plan)]),
    "awq_w4a16_plan_tile": (ctypes.c_int, [_I64, _I64, _I64, _I32, _I32, _I32, ctypes.POINTER(Plan)]),
    "awq_w4a16_plan_stream": (ctypes.c_int, [_I64, _I64, _I64, _I32, _I32, _I32, _I32, _I32, _I32,
                                              ctypes.POINTER(Plan)]),
    "awq_w4a16_workspace_bytes": (ctypes.c_size_t, [_I64, _I64, _I64, _I32]),
    "awq_w4a16_workspace_bytes_ex": (ctypes.c_size_t, [_I64, _I64, _I64, _I32, _I32]),
    "awq_w4a16_validate": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I32, _VP,
                                          ctypes.c_size_t, _I32]),
    "awq_w4a16_gemm": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I32, _VP,
                                      ctypes.c_size_t, _VP]),
    "awq_w4a16_gemm_ex": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I32, _VP,
                                         ctypes.c_size_t, _I32, _VP]),
    "awq_w4a16_gemm_planned": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I32, _VP,
                                              ctypes.c_size_t, ctypes.POINTER(Plan), _VP]),
    "awq_w4a16_dequant": (ctypes.c_int, [_VP, _VP, _VP, _VP, _I64, _I64, _I32, _VP]),
    "awq_fp16_linear": (ctypes.c_int, [_VP, _VP, _VP, _I64, _I64, _I64, _VP]),
    "awq_w4a16_gemm_epilogue": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I32, _VP,
                                               ctypes.c_size_t, ctypes.POINTER(Plan), _VP]),
    "awq_silu_mul": (ctypes.c_int, [_VP, _VP, _I64, _I64, _VP]),
    "awq_w4a16_gemm_noalloc": (ctypes.c_int, [_VP, _VP, _VP, _VP, _VP, _I64, _I64, _I64, _I32, _VP]),
}

_lib = None
_binding = None


def binding():
    """The torch binding of the eager entry point (``lib/_awq_torch*.so``,
    built from ``csrc/awq_torch_binding.cpp``): ``awq_gemm_forward`` with
    checks, allocation, plan and workspace in C++, and the per-device
    workspace registry every entry point shares.  Missing, it raises: there
    is no fallback path."""
    global _binding
    if _binding is None:
        import importlib.util
        import sysconfig

        import torch  # noqa: F401  (the binding links torch's libraries)

        lib()  # the C ABI it calls, ABI-checked first
        path = os.path.join(_PKG_ROOT, "lib", "_awq_torch" + sysconfig.get_config_var("EXT_SUFFIX"))
        if not os.path.exists(path):
            raise RuntimeError(f"torch binding not found at {path}; build it with "
                               "`python qwen2-7b-triton_engine_amd/build.py` (there is no fallback path)")
        spec = importlib.util.spec_from_file_location("_awq_torch", path)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        if mod.abi_version() != ABI_VERSION:
            raise RuntimeError(f"{path} was built against ABI {mod.abi_version()}, expected {ABI_VERSION}")
        _binding = mod
    return _binding


class AwqNativeError(RuntimeError):
    """A nonzero status from the HIP library."""

    def __init__(self, status: int, where: str):
        self.status = status
        super().__init__(f"{where}: status {status}: {error_string(status)}")


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"W4A16 AWQ HIP library not found at {LIB_PATH}; build it with "
                "`python qwen2-7b-triton_engine_amd/build.py` (there is no fallback path)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        if L.awq_w4a16_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI {L.awq_w4a16_abi_version()}, expected {ABI_VERSION}")
        _lib = L
    return _lib


def error_string(status: int) -> str:
    return lib().awq_w4a16_error_string(status).decode()


def check(status: int, where: str) -> None:
    if status != AWQ_OK:
        raise AwqNativeError(status, where)


def plan_for(M: int, N: int, K: int, group_size: int = 128, path: int = PATH_AUTO) -> Plan:
    p = Plan()
    check(lib().awq_w4a16_plan_for(M, N, K, group_size, path, ctypes.byref(p)), "awq_w4a16_plan_for")
    return p


def plan_skinny(M: int, N: int, K: int, rows_per_wave: int, k_waves: int, variant: int = 2,
                factored_scale: int | None = None, group_size: int = 128) -> Plan:
    if factored_scale is None:
        factored_scale = 0 if M > 32 else 1
    p = Plan()
    check(lib().awq_w4a16_plan_skinny(M, N, K, group_size, rows_per_wave, k_waves, variant, factored_scale,
                                      ctypes.byref(p)), "awq_w4a16_plan_skinny")
    return p


def plan_gemv(M: int, N: int, K: int, rows_per_wave: int, k_waves: int, variant: int = 5, split_k: int = 1,
              depth: int = 2, tile_n: int = 512, group_size: int = 128) -> Plan:
    """GEMV-path plan.  Variant 5 (MFMA column sums, fixed-point split-K):
    ``tile_n`` is the strip width -- 512 (column quads, M <= 2), 256 (pairs,
    M <= 4) or 128 (singles, M <= 8); variant 6 (singles with 16 rows of x,
    9 <= M <= 16, fp32 partials and a reduce launch): ``tile_n`` 128, depth 2;
    variant 2 (K-streaming): ``tile_n`` 512, ``rows_per_wave`` 16 or 32."""
    p = Plan()
    check(lib().awq_w4a16_plan_gemv(M, N, K, group_size, variant, tile_n, rows_per_wave, k_waves, split_k, depth,
                                    ctypes.byref(p)), "awq_w4a16_plan_gemv")
    return p


def plan_stream(M: int, N: int, K: int, k_waves: int, split_k: int, variant: int = 1, depth: int = 2,
                layout: str = "half", group_size: int = 128) -> Plan:
    """Stream path (M <= 16): 16x16x32 MFMA, zero and scale folded once per
    group.  ``layout`` "row" (M <= 8: whole 256-byte row segments per load,
    ``k_waves`` waves sharing every group, 1, 2, 4 or 8 with depth 2 or 4 or
    8 with depth 1) or "half" (M <= 16: wave pairs on the two halves of each
    row segment, ``k_waves`` pairs, 1 .. 4 with depth 2, 1 .. 2 with depth 4
    or 6); split-K finish by fixed-point slots (variant 1), fp32 partials
    added by the last-arriving workgroup of a strip (2) or by a second launch
    (3)."""
    rows = {"row": 16, "half": 32}[layout]
    p = Plan()
    check(lib().awq_w4a16_plan_stream(M, N, K, group_size, rows, variant, k_waves, split_k, depth, ctypes.byref(p)),
          "awq_w4a16_plan_stream")
    return p


def plan_tile(M: int, N: int, K: int, variant: int = 6, split_k: int = 1, group_size: int = 128) -> Plan:
    p = Plan()
    check(lib().awq_w4a16_plan_tile(M, N, K, group_size, variant, split_k, ctypes.byref(p)), "awq_w4a16_plan_tile")
    return p


def counter_bytes() -> int:
    return int(lib().awq_w4a16_counter_bytes())


def workspace_bytes(M: int, N: int, K: int, group_size: int = 128, path: int = PATH_AUTO) -> int:
    return int(lib().awq_w4a16_workspace_bytes_ex(M, N, K, group_size, path))
