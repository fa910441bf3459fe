"""MI355X-native W4A16 AWQ GEMM: the ``kernels.awq_gemm`` module of
Qwen2-7B-Triton_Engine, rebuilt on hand-written HIP kernels for gfx950.

Put the directory that holds this package on ``sys.path`` and the reference's
call sites (``kernels.awq_gemm.awq_gemm_forward(...)``, ``model/qwen2.py:44,
104-107,183-186``) resolve to this implementation unchanged.
"""
