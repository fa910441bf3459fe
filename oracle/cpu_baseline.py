"""The reference's CPU dequant + matmul, restated on torch-CPU.

TEST INFRASTRUCTURE ONLY: this is the ``cpu_baseline`` leg that ``bench.py``
times on the host cores next to the GPU kernel (``kind: "port"``).  It is
never the thing measured as the product and never a fallback.

Follows ``test/compare_benchmark.py:72-95`` (``torch_awq_gemm``), the
vectorised "Pure PyTorch" AWQ GEMM the reference swaps in for its baseline
runs (``test/compare_benchmark.py:120``):

1. unpack qweight / qzeros with shifts ``4*[0,4,1,5,2,6,3,7]`` on the signed
   int32 words, ``& 0xF`` (``:80-85``);
2. ``w = (q - z) * s`` in fp16 with the zero and scale broadcast over each
   128-row group (``:87-92``);
3. ``torch.matmul`` of fp16 x with the fp16 weight (``:94``).
"""
from __future__ import annotations

import os
import platform
import time

import torch

_ORDER = (0, 4, 1, 5, 2, 6, 3, 7)


def torch_awq_gemm_cpu(x: torch.Tensor, qweight: torch.Tensor, qzeros: torch.Tensor,
                       scales: torch.Tensor, group_size: int = 128) -> torch.Tensor:
    in_shape = x.shape
    x2 = x.reshape(-1, x.shape[-1])
    k = x2.shape[1]
    n = scales.shape[1]
    g = k // group_size
    shifts = (torch.tensor(_ORDER, dtype=torch.int32) * 4).view(1, 1, 8)
    w = ((qweight.view(k, n // 8, 1) >> shifts) & 0xF).reshape(k, n).to(torch.float16)
    z = ((qzeros.view(g, n // 8, 1) >> shifts) & 0xF).reshape(g, n).to(torch.float16)
    w = (w.view(g, group_size, n) - z.view(g, 1, n)) * scales.view(g, 1, n)
    out = torch.matmul(x2, w.view(k, n))
    return out.view(*in_shape[:-1], n)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def time_cpu_baseline(x, qweight, qzeros, scales, group_size=128, reps=5, warmup=1,
                      threads=None, budget_s=None):
    """Median wall time (s) of ``torch_awq_gemm_cpu`` on CPU tensors.

    One warm-up, then ``reps`` timed repetitions (stopping early once
    ``budget_s`` of timed work is spent, after at least one repetition).
    """
    if threads is not None:
        torch.set_num_threads(int(threads))
    for _ in range(warmup):
        torch_awq_gemm_cpu(x, qweight, qzeros, scales, group_size)
    times = []
    spent = 0.0
    for _ in range(reps):
        t0 = time.perf_counter()
        torch_awq_gemm_cpu(x, qweight, qzeros, scales, group_size)
        dt = time.perf_counter() - t0
        times.append(dt)
        spent += dt
        if budget_s is not None and spent >= budget_s:
            break
    times.sort()
    return {
        "median_s": times[len(times) // 2],
        "reps": len(times),
        "threads": torch.get_num_threads(),
        "os_cpu_count": os.cpu_count(),
        "cpu_model": cpu_model(),
    }
