"""CPU oracle for the W4A16 AWQ GEMM path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library and the
``kernels.awq_gemm`` host module) imports, links or calls anything here.  The
only permitted users are ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``, and there only as the checker or as the
timed CPU baseline, never as the thing measured or shipped.

Two independent restatements of the reference's numerics live here:

* ``awq_oracle.py``  -- numpy, vectorised, following
  ``test/compare_benchmark.py:72-95`` (``torch_awq_gemm``);
* ``awq_oracle.c``   -- plain C, per-column loop, following
  ``inference/baseline_kernels.py:36-60``, with its own IEEE fp16
  round-to-nearest-even conversion.

``cpu_baseline.py`` restates ``torch_awq_gemm`` on torch-CPU (fp16 dequant,
then ``torch.matmul`` in fp16): this is the CPU path timed next to the GPU.

How each function is pinned (known answers worked by hand, closed forms,
exhaustive checks, brute force) is listed in ``tests/test_oracle.py``.
"""
