"""The allocation-free entry point, awq_w4a16_gemm_noalloc, called through
the C ABI, against awq_w4a16_gemm (the entry point that takes a caller
workspace) on the same operands.

Where both launch the same plan the outputs must be bit-identical; where the
static scratch bound lowered a tile plan's split-K count (down_proj at
M = 2048 needs 56 MB of partials, the scratch holds 32 MiB) they must agree
to the GEMM tolerance.  Each case makes two calls in a row, the second with
a smaller input, and checks both: a scratch left dirty by the first call
(counters, fixed-point slots, partials) would corrupt the second.
"""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from kernels import _native
from kernels.awq_gemm import awq_gemm_forward
from oracle import awq_oracle as O

pytestmark = pytest.mark.gpu

RTOL = 1e-2


def _operands(dev, k, n, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    qw = torch.randint(-2**31, 2**31 - 1, (k, n // 8), generator=g, device=dev, dtype=torch.int32)
    qz = torch.randint(-2**31, 2**31 - 1, (k // 128, n // 8), generator=g, device=dev, dtype=torch.int32)
    s = (torch.rand((k // 128, n), generator=g, device=dev) * 0.018 + 0.002).half()
    return qw, qz, s


def _noalloc(x, qw, qz, s):
    m, k = x.shape
    n = s.shape[1]
    out = torch.empty((m, n), dtype=torch.float16, device=x.device)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
    st = _native.lib().awq_w4a16_gemm_noalloc(P(x), P(qw), P(qz), P(s), P(out), m, n, k, 128, stream)
    _native.check(st, "awq_w4a16_gemm_noalloc")
    return out


# (name, K, N, first M, second M): the first call's plan, then a smaller one.
CASES = [
    ("qkv_proj", 3584, 4608, 16, 1),        # 32-row tile split 14 + reduce launch; GEMV fixed-point slots
    ("gate_up_proj", 3584, 37888, 4, 2),    # stream fixed-point slots, at M = 4 and 2
    ("down_proj", 18944, 3584, 16, 8),      # 16-row column singles split 8 + reduce launch; 8-row ones at M = 8
    ("o_proj", 3584, 3584, 300, 5),         # tile split-K (reduce launch); column-single GEMV at M = 5
    ("down_proj", 18944, 3584, 2048, 512),  # 512-column tile plans lowered to the 256-column tile: split 1, then 4 (28 MB)
    ("qkv_proj", 3584, 4608, 2048, 1025),   # hybrid tiles (compact partials, last arrivers)
    ("k_proj", 3584, 512, 16, 4),           # 16-row column singles split 64 + reduce; slim singles split 28
    ("gate_proj", 3584, 18944, 2, 1),       # column pairs split 3 (fixed-point slots), at M = 2 and 1
]


@pytest.mark.parametrize("name,k,n,m1,m2", CASES)
def test_noalloc_matches_workspace_entry(gpu, name, k, n, m1, m2):
    qw, qz, s = _operands(gpu, k, n, seed=k + n + m1)
    x = torch.randn((m1, k), device=gpu).half()
    for m in (m1, m2):
        p = _native.plan_for(m, n, k)
        fits = p.workspace_bytes <= _native.NOALLOC_SCRATCH_BYTES
        what = (f"noalloc {name} M={m} auto={_native.PATH_NAMES[p.path]} v{p.variant} split={p.split_k} "
                f"ws={p.workspace_bytes} fits={fits}")
        print(what, flush=True)
        got = _noalloc(x[:m].contiguous(), qw, qz, s)
        want = awq_gemm_forward(x[:m], qw, qz, s)
        torch.cuda.synchronize()
        g, w = got.cpu().numpy(), want.cpu().numpy()
        assert np.isfinite(g).all(), what
        if fits:
            assert np.array_equal(g.view(np.uint16), w.view(np.uint16)), what
        else:
            err = O.max_rel_err(g, w.astype(np.float64))
            assert err <= RTOL and O.elementwise_violations(g, w.astype(np.float64), RTOL) == 0, (what, err)


def test_noalloc_repeats_and_graph_replay(gpu):
    """Repeated calls leave the scratch clean (same bits every time), and a
    captured call replays correctly several times with eager work in between."""
    k, n = 3584, 4608
    qw, qz, s = _operands(gpu, k, n, seed=5)
    x = torch.randn((16, k), device=gpu).half()
    ref = awq_gemm_forward(x, qw, qz, s)
    for _ in range(3):
        got = _noalloc(x, qw, qz, s)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        out_static = _noalloc(x, qw, qz, s)  # warm: set-up done before capture
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            out_static = _noalloc(x, qw, qz, s)
    torch.cuda.current_stream().wait_stream(side)
    for i in range(3):
        out_static.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_static, ref), f"replay {i}"
        eager = _noalloc(x[:4].contiguous(), qw, qz, s)
        torch.cuda.synchronize()
        assert torch.equal(eager, awq_gemm_forward(x[:4], qw, qz, s))


_FRESH_PROCESS = r"""
import ctypes, sys
sys.path[:0] = sys.argv[1:3]
import torch
from kernels import _native
from kernels.awq_gemm import awq_gemm_forward

dev = torch.device("cuda:0")
k, n, m = 3584, 4608, 16
g = torch.Generator(device=dev)
g.manual_seed(3)
qw = torch.randint(-2**31, 2**31 - 1, (k, n // 8), generator=g, device=dev, dtype=torch.int32)
qz = torch.randint(-2**31, 2**31 - 1, (k // 128, n // 8), generator=g, device=dev, dtype=torch.int32)
s = (torch.rand((k // 128, n), generator=g, device=dev) * 0.018 + 0.002).half()
x = torch.randn((m, k), generator=g, device=dev).half()
out = torch.zeros((m, n), dtype=torch.float16, device=dev)
assert _native.plan_for(m, n, k).workspace_bytes > 0
P = lambda t: ctypes.c_void_p(t.data_ptr())
L = _native.lib()

def call(stream):
    return L.awq_w4a16_gemm_noalloc(P(x), P(qw), P(qz), P(s), P(out), m, n, k, 128,
                                    ctypes.c_void_p(stream.cuda_stream))

side = torch.cuda.Stream()
side.wait_stream(torch.cuda.current_stream())
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph, stream=side):
    out.zero_()
    st_captured_first = call(side)
torch.cuda.synchronize()
print("first call under capture:", st_captured_first, flush=True)
assert st_captured_first == _native.AWQ_ERR_CAPTURE, st_captured_first
st = call(torch.cuda.current_stream())
torch.cuda.synchronize()
assert st == _native.AWQ_OK, st
ref = awq_gemm_forward(x, qw, qz, s)
torch.cuda.synchronize()
assert torch.equal(out, ref)
graph2 = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph2, stream=side):
    st2 = call(side)
assert st2 == _native.AWQ_OK, st2
for i in range(3):
    out.zero_()
    graph2.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, ref), i
print("ok", flush=True)
"""


def test_noalloc_first_call_under_capture_is_refused(gpu):
    """In a fresh process (no earlier call has set the scratch up): the first
    split-K call of the allocation-free entry point, made under graph
    capture, is refused with AWQ_ERR_CAPTURE and records nothing; after one
    eager call on the device (which sets the scratch up) the same call
    matches awq_w4a16_gemm and can be captured and replayed."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    pkg = os.path.join(root, "qwen2-7b-triton_engine_amd")
    print("noalloc capture refusal: fresh process", flush=True)
    r = subprocess.run([sys.executable, "-c", _FRESH_PROCESS, pkg, root], capture_output=True, text=True,
                       timeout=300)
    print(r.stdout, flush=True)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout + r.stderr
