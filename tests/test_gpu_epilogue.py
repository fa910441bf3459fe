"""Fused epilogues (``awq_w4a16_gemm_epilogue``, ``awq_silu_mul``): the
reference's follow-ups of the GEMM (QKV bias add, residual adds after o/down,
SiLU * up, model/qwen2.py:45-46,108-109,187-194,219-227).

Bars: the fused bias / residual result equals the unfused sequence -- the
same plan's GEMM, then torch's fp16 ``y + bias`` and ``residual + y`` --
bit for bit, on every kernel family and every split-K finish (direct store,
fixed-point slots, last arriver, reduce launch), also with the residual
aliasing the output.  SiLU * up equals torch's ``silu(g) * u`` in fp32
rounded to fp16 within one fp16 ulp (both take exp from the device math
library)."""
import numpy as np
import pytest
import torch

from kernels import _native
from kernels.awq_gemm import awq_gemm_forward, awq_gemm_forward_ex
from kernels.silu_mul import silu_mul_forward, silu_mul_gate_up
from oracle import awq_oracle as O

pytestmark = pytest.mark.gpu


def _plans(m, n, k):
    """The AUTO plan, every path's own plan, and forced variants that cover
    each split-K finish (fixed-point slots, last arriver, reduce launch)."""
    makers = [("auto", lambda: _native.plan_for(m, n, k))]
    for path in (_native.PATH_GEMV, _native.PATH_STREAM, _native.PATH_SKINNY, _native.PATH_TILE):
        makers.append((_native.PATH_NAMES[path], lambda path=path: _native.plan_for(m, n, k, path=path)))
    if m <= 2:
        makers += [(f"gemv quad v{v} s{sp}", lambda v=v, sp=sp: _native.plan_gemv(m, n, k, 0, 4, variant=v, split_k=sp))
                   for v in (5,) for sp in (1, 3, 16)]
    if m <= 16:
        makers += [(f"stream v{v} s4", lambda v=v: _native.plan_stream(m, n, k, 2, 4, variant=v)) for v in (1, 2, 3)]
    if 9 <= m <= 16:
        makers += [(f"gemv singles reduce s{sp}",
                    lambda sp=sp: _native.plan_gemv(m, n, k, 0, 8, variant=6, split_k=sp, tile_n=128))
                   for sp in (4, 9)]
    if m > 16:
        makers += [(f"tile v{v} s{sp}", lambda v=v, sp=sp: _native.plan_tile(m, n, k, v, sp))
                   for v, sp in ((6, 1), (6, 2), (7, 3), (8, 2), (9, 4), (13, 2), (14, 3), (15, 1), (15, 2))]
    out = []
    for label, make in makers:
        try:
            out.append((label, make()))
        except _native.AwqNativeError:
            pass  # this path or plan does not serve the shape
    assert len(out) >= 4, (m, [l for l, _ in out])
    return out


@pytest.mark.parametrize("m", [1, 2, 4, 16, 100, 300, 2048])
def test_bias_residual_epilogue_bit_exact(gpu, m):
    k, n = 3584, 4608
    x, qw, qz, s = O.make_inputs(m, k, n, seed=40 + m)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)  # noqa: E731
    xt, qwt, qzt, st = t(x), t(qw), t(qz), t(s)
    g = torch.Generator(device=gpu)
    g.manual_seed(m)
    bias = (torch.randn(n, generator=g, device=gpu) * 0.5).half()
    res = (torch.randn((m, n), generator=g, device=gpu) * 4).half()
    for label, p in _plans(m, n, k):
        print(f"epilogue M={m} {label} split={p.split_k}", flush=True)
        y = awq_gemm_forward_ex(xt, qwt, qzt, st, plan_obj=p)
        want_b = y + bias
        want_br = res + want_b
        want_r = res + y
        got_b = awq_gemm_forward_ex(xt, qwt, qzt, st, plan_obj=p, bias=bias)
        got_br = awq_gemm_forward_ex(xt, qwt, qzt, st, plan_obj=p, bias=bias, residual=res)
        got_r = awq_gemm_forward_ex(xt, qwt, qzt, st, plan_obj=p, residual=res)
        inplace = res.clone()
        awq_gemm_forward_ex(xt, qwt, qzt, st, plan_obj=p, bias=bias, residual=inplace, out=inplace)
        torch.cuda.synchronize()
        for what, a, b in (("bias", got_b, want_b), ("bias+res", got_br, want_br), ("res", got_r, want_r),
                           ("in place", inplace, want_br)):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"{label} {what}"


def test_epilogue_auto_path_and_leading_dims(gpu):
    m, k, n = 6, 3584, 3584
    x, qw, qz, s = O.make_inputs(m, k, n, seed=3)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)  # noqa: E731
    xt = t(x).view(2, 3, k)
    res = torch.randn((2, 3, n), device=gpu).half()
    got = awq_gemm_forward_ex(xt, t(qw), t(qz), t(s), residual=res)
    want = res + awq_gemm_forward(xt, t(qw), t(qz), t(s))
    torch.cuda.synchronize()
    assert got.shape == (2, 3, n) and torch.equal(got, want)
    with pytest.raises(ValueError):
        awq_gemm_forward_ex(xt, t(qw), t(qz), t(s), bias=torch.zeros(n + 8, dtype=torch.float16, device=gpu))


@pytest.mark.parametrize("m,i", [(1, 18944), (4, 18944), (37, 256), (2048, 512)])
def test_silu_mul_gate_up(gpu, m, i):
    g = torch.Generator(device=gpu)
    g.manual_seed(i + m)
    gu = (torch.randn((m, 2 * i), generator=g, device=gpu) * 3).half()
    out = silu_mul_gate_up(gu)
    gate, up = gu[:, :i].float(), gu[:, i:].float()
    ref = (torch.nn.functional.silu(gate) * up).half()
    torch.cuda.synchronize()
    diff = (out.view(torch.int16).int() - ref.view(torch.int16).int()).abs()
    assert int(diff.max()) <= 1, f"max {int(diff.max())} ulp"
    two = silu_mul_forward(gu[:, :i], gu[:, i:])
    torch.cuda.synchronize()
    assert torch.equal(two, out)
