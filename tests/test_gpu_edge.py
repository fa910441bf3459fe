"""GPU parity at the edges of the operand ranges.

* One-hot rows of x through every kernel path and split-K finish at extreme
  fp16 scales (subnormal scales and products, ties, weights past 4096 up to
  46080): each output is one dequantised weight, so it must equal the
  oracle's fp16((q - z) * s) bit for bit (zeros compared without their sign:
  an accumulator that starts at +0 turns -0 into +0, as fp16 matmul does).
* Outlier activations (a few channels at +-1000, the rest N(0, 1)) on every
  AUTO route of the Qwen2-7B shapes, decode and prefill, against the oracle
  at the GEMM tolerance.
* A NaN or an infinity in x makes its own output row non-finite on every
  route (the reference's fp16 matmul gives NaN or +-inf there) and leaves the
  other rows exact to the tolerance.
"""
import numpy as np
import pytest
import torch

from kernels import _native
from kernels.awq_gemm import awq_gemm_forward_ex
from kernels.awq_roofline import QWEN2_7B_FUSED, QWEN2_7B_LINEARS
from oracle import awq_oracle as O

pytestmark = pytest.mark.gpu

RTOL = 1e-2
_SHAPES = {name: (k, n) for name, k, n in QWEN2_7B_LINEARS + QWEN2_7B_FUSED}

# fp16 scale bit patterns whose weights (q - z) * s stay finite for every
# |q - z| <= 15: subnormal scales (every product subnormal, odd mantissas),
# the subnormal/normal boundary, ties to even, signed zeros, negative
# scales, and large scales whose weights lie between 4096 and 65504.
FINITE_EDGE_SCALES = np.array(
    [0x0001, 0x0155, 0x0200, 0x03FF, 0x0400, 0x0401, 0x1000, 0x2E66, 0x3555, 0x3C00, 0x3C01, 0x3C03,
     0xBC00, 0x8001, 0x0000, 0x8000, 0x5BFF, 0x6000, 0x67FF, 0x6A00, 0xEA00],
    dtype=np.uint16)


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _run(dev, x, qw, qz, s, path=None, plan_obj=None):
    y = awq_gemm_forward_ex(_t(x, dev), _t(qw, dev), _t(qz, dev), _t(s, dev), 128, path=path, plan_obj=plan_obj)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def _assert_close(y, y_ref, what):
    err = O.max_rel_err(y, y_ref)
    bad = O.elementwise_violations(y, y_ref, RTOL)
    assert np.isfinite(y).all(), f"{what}: non-finite output"
    assert err <= RTOL and bad == 0, f"{what}: max rel err {err:.3e}, {bad} element violations"


def _try(make):
    try:
        return make()
    except _native.AwqNativeError:
        return None


def _every_plan(m, n, k):
    """AUTO, each path's own plan, and forced variants covering every kernel
    and split-K finish that serves this shape."""
    makers = [lambda: _native.plan_for(m, n, k)]
    makers += [lambda p=p: _native.plan_for(m, n, k, path=p)
               for p in (_native.PATH_GEMV, _native.PATH_STREAM, _native.PATH_SKINNY, _native.PATH_TILE)]
    for sp in (1, 2):
        makers += [lambda v=v, sp=sp: _native.plan_gemv(m, n, k, 0, 4, variant=v, split_k=sp) for v in (5,)]
        makers += [lambda sp=sp: _native.plan_gemv(m, n, k, 16, 8, variant=2, split_k=sp, depth=2)]
        makers += [lambda v=v, sp=sp: _native.plan_stream(m, n, k, 2, sp, variant=v) for v in (1, 2, 3)]
        makers += [lambda v=v, sp=sp: _native.plan_stream(m, n, k, 4, sp, variant=v, layout="row")
                   for v in (1, 2, 3)]
        makers += [lambda v=v, sp=sp: _native.plan_tile(m, n, k, v, sp) for v in (6, 7, 8, 9, 15)]
    makers += [lambda f=f: _native.plan_skinny(m, n, k, 128, 2, 2, f) for f in (0, 1)]
    plans, seen = [], set()
    for make in makers:
        p = _try(make)
        if p is None:
            continue
        key = tuple(getattr(p, f) for f, _ in p._fields_)
        if key not in seen:
            seen.add(key)
            plans.append(p)
    return plans


@pytest.mark.parametrize("m", [1, 2, 4, 8, 16, 40, 130])
def test_one_hot_edge_scales_every_plan(gpu, m):
    k, n = 256, 288
    rng = np.random.default_rng(40 + m)
    qcodes = rng.integers(0, 16, size=(k, n), dtype=np.uint8)
    zcodes = rng.integers(0, 16, size=(k // 128, n), dtype=np.uint8)
    s = rng.choice(FINITE_EDGE_SCALES, size=(k // 128, n)).view(np.float16)
    qw, qz = O.pack_awq(qcodes), O.pack_awq(zcodes)
    w = O.dequant_awq(qw, qz, s)
    assert np.isfinite(w).all() and np.abs(w.astype(np.float64)).max() > 4096
    rows = rng.integers(0, k, size=m)
    x = np.zeros((m, k), dtype=np.float16)
    x[np.arange(m), rows] = 1.0
    want = (w[rows] + np.float16(0)).view(np.uint16)
    plans = _every_plan(m, n, k)
    assert len(plans) >= 3
    for p in plans:
        what = f"one-hot edge M={m} {_native.PATH_NAMES[p.path]} v{p.variant} split={p.split_k}"
        print(what, flush=True)
        y = _run(gpu, x, qw, qz, s, plan_obj=p)
        assert np.array_equal((y + np.float16(0)).view(np.uint16), want), what


def _outlier_x(m, k, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    ch = rng.choice(k, size=4, replace=False)
    x[:, ch] = np.array([1000.0, -1000.0, 1000.0, -1000.0], dtype=np.float32)
    return x.astype(np.float16)


_ROUTES = ([(name, m) for name in ("qkv_proj", "o_proj", "gate_up_proj", "down_proj") for m in (1, 2, 3, 4, 8, 16)] +
           [("down_proj", 64), ("qkv_proj", 64), ("o_proj", 512), ("down_proj", 512), ("gate_up_proj", 2048),
            ("qkv_proj", 2048), ("o_proj", 1025), ("o_proj", 2560), ("down_proj", 3072)])


@pytest.mark.parametrize("name,m", _ROUTES)
def test_outlier_activations_auto_routes(gpu, name, m):
    k, n = _SHAPES[name]
    _, qw, qz, s = O.make_inputs(1, k, n, seed=60)
    x = _outlier_x(m, k, seed=61 + m)
    rows = np.arange(m) if m <= 64 else np.random.default_rng(m).choice(m, size=32, replace=False)
    w = O.dequant_awq_f32eval(qw, qz, s).astype(np.float64 if m <= 16 else np.float32)
    y_ref = x[rows].astype(w.dtype) @ w
    p = _native.plan_for(m, n, k)
    what = f"outliers {name} M={m} auto={_native.PATH_NAMES[p.path]} v{p.variant} split={p.split_k}"
    print(what, flush=True)
    y = _run(gpu, x, qw, qz, s)
    _assert_close(y[rows], y_ref, what)


@pytest.mark.parametrize("name,m", [(nm, m) for nm in ("qkv_proj", "gate_up_proj", "down_proj")
                                    for m in (1, 2, 4, 16)] + [("down_proj", 64), ("o_proj", 512)])
def test_nonfinite_activation_stays_in_its_row(gpu, name, m):
    k, n = _SHAPES[name]
    _, qw, qz, s = O.make_inputs(1, k, n, seed=70)
    x = np.random.default_rng(71).standard_normal((m, k)).astype(np.float16)
    x[0, 5] = np.float16(np.nan)
    if m > 1:
        x[m - 1, k - 3] = np.float16(np.inf)
    p = _native.plan_for(m, n, k)
    what = f"non-finite x {name} M={m} auto={_native.PATH_NAMES[p.path]} v{p.variant} split={p.split_k}"
    print(what, flush=True)
    y = _run(gpu, x, qw, qz, s)
    assert not np.isfinite(y[0]).any(), f"{what}: NaN row has finite outputs"
    if m > 1:
        assert not np.isfinite(y[m - 1]).any(), f"{what}: inf row has finite outputs"
    if m > 2:
        w = O.dequant_awq_f32eval(qw, qz, s).astype(np.float32)
        _assert_close(y[1:m - 1], x[1:m - 1].astype(np.float32) @ w, what)
