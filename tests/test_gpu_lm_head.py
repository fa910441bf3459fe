"""GPU parity of the fp16 output-projection GEMV (``awq_fp16_linear``,
``kernels/lm_head.py``), the lm_head of model/qwen2.py:253,280.

Bars: one-hot activations give the weight column bit-exactly (a single
product 1 * w is exact, and the fp32 sum of it and zeros rounds back to w);
otherwise max|y - y_ref| / max|y_ref| <= 1e-2 and the element-wise bound of
the GEMM tests, y_ref = x @ W^T in fp64 (numpy) or, at the full
152064 x 3584 shape, in fp32 on the GPU (its own error ~1e-6).
"""
import numpy as np
import pytest
import torch

from kernels import _native
from kernels.lm_head import MAX_ROWS, lm_head_forward
from oracle import awq_oracle as O

pytestmark = pytest.mark.gpu

RTOL = 1e-2


def _inputs(m, n, k, seed):
    g = np.random.default_rng(seed)
    x = g.standard_normal((m, k)).astype(np.float16)
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float16)
    return x, w


def _assert_close(y, y_ref, what):
    err = O.max_rel_err(y, y_ref)
    bad = O.elementwise_violations(y, y_ref, RTOL)
    assert np.isfinite(y).all(), f"{what}: non-finite output"
    assert err <= RTOL and bad == 0, f"{what}: max rel err {err:.3e}, {bad} element violations"


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("n,k", [(1000, 3584), (129, 1024), (37, 200), (4099, 4096), (64, 8)])
def test_lm_head_parity(gpu, m, n, k):
    x, w = _inputs(m, n, k, seed=m * 131 + n)
    print(f"lm_head M={m} N={n} K={k}", flush=True)
    y = lm_head_forward(torch.from_numpy(x).to(gpu), torch.from_numpy(w).to(gpu))
    torch.cuda.synchronize()
    y_ref = x.astype(np.float64) @ w.astype(np.float64).T
    _assert_close(y.cpu().numpy(), y_ref, f"lm_head M={m} N={n} K={k}")


@pytest.mark.parametrize("m", [1, 4])
def test_lm_head_qwen2_7b_shape(gpu, m):
    """The real projection: vocab 152064, hidden 3584 (1.09 GB of fp16)."""
    n, k = 152064, 3584
    print(f"lm_head full shape M={m}", flush=True)
    g = torch.Generator(device=gpu)
    g.manual_seed(5 + m)
    x = torch.randn((m, k), generator=g, device=gpu).half()
    w = (torch.randn((n, k), generator=g, device=gpu) * 0.02).half()
    y = lm_head_forward(x, w)
    y_ref = x.float() @ w.float().T
    torch.cuda.synchronize()
    _assert_close(y.cpu().numpy(), y_ref.cpu().numpy().astype(np.float64), f"lm_head full M={m}")
    del w


def test_lm_head_one_hot_bit_exact(gpu):
    n, k = 3000, 3584
    _, w = _inputs(1, n, k, seed=11)
    w[5, 7] = np.float16(65504.0)    # largest finite
    w[6, 7] = np.float16(-6.1e-5)    # subnormal-adjacent
    cols = [0, 7, 1234, k - 1, 3583, 8, 9, 2047]
    x = np.zeros((MAX_ROWS, k), dtype=np.float16)
    x[np.arange(MAX_ROWS), cols] = 1.0
    for m in (1, 3, MAX_ROWS):
        print(f"lm_head one-hot M={m}", flush=True)
        y = lm_head_forward(torch.from_numpy(x[:m]).to(gpu), torch.from_numpy(w).to(gpu))
        torch.cuda.synchronize()
        y = y.cpu().numpy()
        for i in range(m):
            assert np.array_equal(y[i].view(np.uint16), w[:, cols[i]].view(np.uint16)), (m, i)


def test_lm_head_leading_dims_empty_and_out(gpu):
    x, w = _inputs(6, 300, 512, seed=3)
    xt, wt = torch.from_numpy(x).to(gpu), torch.from_numpy(w).to(gpu)
    y = lm_head_forward(xt.view(2, 3, 512), wt)
    assert tuple(y.shape) == (2, 3, 300)
    y2 = lm_head_forward(xt, wt)
    torch.cuda.synchronize()
    assert torch.equal(y.reshape(6, 300), y2)
    empty = lm_head_forward(xt[:0], wt)
    assert tuple(empty.shape) == (0, 300)
    out = torch.empty((6, 300), dtype=torch.float16, device=gpu)
    assert lm_head_forward(xt, wt, out=out).data_ptr() == out.data_ptr()
    torch.cuda.synchronize()
    assert torch.equal(out, y2)


def test_lm_head_errors(gpu):
    x, w = _inputs(9, 64, 256, seed=4)
    xt, wt = torch.from_numpy(x).to(gpu), torch.from_numpy(w).to(gpu)
    with pytest.raises(ValueError):
        lm_head_forward(xt, wt)                      # 9 rows
    with pytest.raises(ValueError):
        lm_head_forward(xt[:2].float(), wt)          # dtype
    with pytest.raises(ValueError):
        lm_head_forward(xt[:2, :128], wt)            # K mismatch
    with pytest.raises(ValueError):
        lm_head_forward(xt[:2], torch.zeros((64, 8192), dtype=torch.float16, device=gpu)[:, :8190])  # K % 8


def test_lm_head_graph_replay(gpu):
    x, w = _inputs(1, 5000, 3584, seed=9)
    xt, wt = torch.from_numpy(x).to(gpu), torch.from_numpy(w).to(gpu)
    ref = lm_head_forward(xt, wt).clone()
    out = torch.empty_like(ref)
    lm_head_forward(xt, wt, out=out)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        lm_head_forward(xt, wt, out=out)
    torch.cuda.current_stream().wait_stream(side)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
