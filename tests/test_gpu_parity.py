"""GPU parity of the HIP W4A16 AWQ kernels against the CPU oracle.

Bars (the reference's own dequant + matmul semantics):
* unpack + dequant: bit-exact (``awq_w4a16_dequant`` vs the oracle's
  ``fp16((q - z) * s)``), and bit-exact through the GEMM kernels via one-hot
  activations;
* GEMM: max|y - y_ref| / max|y_ref| <= 1e-2 (RTOL below), y_ref the oracle's
  exact fp16 weight accumulated in fp64 (fp32 for the largest shapes, whose
  own error is ~1e-6), plus the element-wise bound
  |y - y_ref| <= 1e-2*|y_ref| + 1e-2*rms(y_ref) on every element.
"""
import numpy as np
import pytest
import torch

from kernels import _native
from kernels.awq_gemm import _dequant_to_fp16, awq_gemm_forward, awq_gemm_forward_ex
from kernels.awq_roofline import QWEN2_7B_FUSED, QWEN2_7B_LINEARS
from oracle import awq_oracle as O
from oracle import c_oracle as C

pytestmark = pytest.mark.gpu

RTOL = 1e-2  # max relative error: fp32 accumulate, fp16 out


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _run(dev, x, qw, qz, s, path=None, plan_obj=None):
    y = awq_gemm_forward_ex(_t(x, dev), _t(qw, dev), _t(qz, dev), _t(s, dev), 128, path=path,
                            plan_obj=plan_obj)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def _assert_close(y, y_ref, what):
    err = O.max_rel_err(y, y_ref)
    bad = O.elementwise_violations(y, y_ref, RTOL)
    assert np.isfinite(y).all(), f"{what}: non-finite output"
    assert err <= RTOL and bad == 0, f"{what}: max rel err {err:.3e}, {bad} element violations"
    return err


def _paths_for(m, n=None):
    paths = [_native.PATH_TILE]
    if m <= 64:
        paths.insert(0, _native.PATH_SKINNY)
    if m <= 16 and (n is None or n % 32 == 0):
        paths.insert(0, _native.PATH_STREAM)
    if m <= 2:
        paths.insert(0, _native.PATH_GEMV)
    return paths


# --------------------------------------------------------------------------
# Dequant: bit-exact
# --------------------------------------------------------------------------

@pytest.mark.parametrize("k,n", [(128, 8), (256, 64), (3584, 512), (3584, 4608), (18944, 3584)])
def test_dequant_bit_exact(gpu, k, n):
    print(f"dequant K={k} N={n}", flush=True)
    _, qw, qz, s = O.make_inputs(1, k, n, seed=11)
    out = torch.empty((k, n), dtype=torch.float16, device=gpu)
    _dequant_to_fp16(_t(qw, gpu), _t(qz, gpu), _t(s, gpu), out)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    want = O.dequant_awq_f32eval(qw, qz, s).view(np.uint16)
    assert np.array_equal(got, want)


def test_dequant_edge_scales_bit_exact(gpu):
    """Every code pair against scales that exercise fp16 rounding: ties,
    subnormal scales and products, overflow to inf, negative scales."""
    print("dequant edge scales", flush=True)
    k, n = 128 * 16, 256
    rng = np.random.default_rng(5)
    qcodes = rng.integers(0, 16, size=(k, n), dtype=np.uint8)
    zcodes = rng.integers(0, 16, size=(k // 128, n), dtype=np.uint8)
    special = np.array([0x3C01, 0x0001, 0x0201, 0x03FF, 0x0400, 0x7BFF, 0xBC01, 0x8001, 0x3555,
                        0x1400, 0x2E66, 0x5BFF, 0x0000, 0x8000, 0x3C00, 0x4900], dtype=np.uint16)
    sbits = rng.choice(special, size=(k // 128, n))
    s = sbits.view(np.float16)
    qw, qz = O.pack_awq(qcodes), O.pack_awq(zcodes)
    out = torch.empty((k, n), dtype=torch.float16, device=gpu)
    _dequant_to_fp16(_t(qw, gpu), _t(qz, gpu), _t(s, gpu), out)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    want = C.dequant(qw, qz, s).view(np.uint16)
    assert np.array_equal(got, want)


# --------------------------------------------------------------------------
# GEMM: small shapes against fp64 brute force, every path
# --------------------------------------------------------------------------

@pytest.mark.parametrize("m", [1, 2, 5, 16, 17, 31, 33, 64, 65, 100, 129, 300])
@pytest.mark.parametrize("k,n", [(128, 8), (256, 64), (384, 136), (512, 264)])
def test_gemm_small(gpu, m, k, n):
    x, qw, qz, s = O.make_inputs(m, k, n, seed=m * 7 + n)
    y_ref = C.gemm_f64(x, qw, qz, s)
    for path in [None] + _paths_for(m, n):
        print(f"gemm small M={m} K={k} N={n} path={path}", flush=True)
        y = _run(gpu, x, qw, qz, s, path=path)
        _assert_close(y, y_ref, f"M={m} K={k} N={n} path={path}")


def test_one_hot_bit_exact(gpu):
    """x = e_k makes y the dequantised row k, bit for bit, through each GEMM kernel."""
    k, n = 512, 264
    _, qw, qz, s = O.make_inputs(1, k, n, seed=3)
    w = O.dequant_awq(qw, qz, s)
    for m in (1, 16, 40, 130):
        rows = np.random.default_rng(m).integers(0, k, size=m)
        x = np.zeros((m, k), dtype=np.float16)
        x[np.arange(m), rows] = 1.0
        for path in _paths_for(m, n):
            print(f"one-hot M={m} path={path}", flush=True)
            y = _run(gpu, x, qw, qz, s, path=path)
            assert np.array_equal(y.view(np.uint16), w[rows].view(np.uint16)), f"M={m} path={path}"


def test_integer_exact(gpu):
    """Scale 1, zero 0 and small integer x: every product and partial sum is an
    exact integer below 2048, so the fp16 output is exact."""
    k, n = 256, 128
    rng = np.random.default_rng(9)
    q = rng.integers(0, 4, size=(k, n), dtype=np.uint8)
    qw = O.pack_awq(q)
    qz = O.pack_awq(np.zeros((k // 128, n), dtype=np.uint8))
    s = np.ones((k // 128, n), dtype=np.float16)
    for m in (1, 7, 64, 200):
        x = rng.integers(-2, 3, size=(m, k)).astype(np.float16)
        want = x.astype(np.int64) @ q.astype(np.int64)
        assert np.abs(want).max() < 2048
        for path in _paths_for(m, n):
            y = _run(gpu, x, qw, qz, s, path=path)
            assert np.array_equal(y.astype(np.int64), want), f"M={m} path={path}"


# --------------------------------------------------------------------------
# GEMM: Qwen2-7B shapes (the decode sweep, down M-sweep, fused shapes, prefill)
# --------------------------------------------------------------------------

_SHAPES = {name: (k, n) for name, k, n in QWEN2_7B_LINEARS + QWEN2_7B_FUSED}


@pytest.mark.parametrize("name", ["q_proj", "k_proj", "gate_proj", "down_proj", "qkv_proj", "gate_up_proj"])
@pytest.mark.parametrize("m", [1, 2, 4, 16])
def test_gemm_decode_shapes(gpu, name, m):
    k, n = _SHAPES[name]
    x, qw, qz, s = O.make_inputs(m, k, n, seed=0)
    y_ref = x.astype(np.float64) @ O.dequant_awq_f32eval(qw, qz, s).astype(np.float64)
    for path in ((None, _native.PATH_SKINNY) + ((_native.PATH_STREAM,) if m <= 16 else ()) +
                 ((_native.PATH_GEMV,) if m <= 2 else ())):
        print(f"decode {name} M={m} path={path}", flush=True)
        y = _run(gpu, x, qw, qz, s, path=path)
        _assert_close(y, y_ref, f"{name} M={m} path={path}")


@pytest.mark.parametrize("m,k,n,path,variant,k_waves", [
    (5, 3584, 4608, "gemv", 5, 8), (8, 18944, 3584, "gemv", 5, 8), (9, 18944, 3584, "gemv", 6, 8),
    (16, 8192, 2080, "gemv", 6, 8),
    (8, 3584, 3592, "tile", 9, None), (13, 2048, 4104, "tile", 9, None), (16, 1152, 6144, "tile", 9, None),
    (9, 3584, 8224, "stream", 3, 3), (13, 8192, 1056, "stream", 3, 3), (12, 2048, 16384, "stream", 3, 2)])
def test_auto_small_m_routes(gpu, m, k, n, path, variant, k_waves):
    """The AUTO routes for 5 <= M <= 16: the column-single GEMV (eight rows of
    x, eight waves) up to M = 8 on narrow weights of 3584 - 4608 columns;
    the 32-row tile split along K on other narrow shallow weights (N not a
    multiple of 256, splits that do not divide K evenly) and above M = 8; on
    deep narrow ones at M = 9 - 16 column singles with 16 rows of x and the
    reduce launch (last strip partly filled at N = 2080); the half-strip
    stream kernel with two or three wave pairs on wide or deep
    ones; each against the oracle."""
    p = _native.plan_for(m, n, k)
    assert _native.PATH_NAMES[p.path] == path and p.variant == variant
    if k_waves is not None:
        assert p.k_waves == k_waves
    x, qw, qz, s = O.make_inputs(m, k, n, seed=m + n)
    y_ref = x.astype(np.float64) @ O.dequant_awq_f32eval(qw, qz, s).astype(np.float64)
    print(f"auto route M={m} K={k} N={n} {path} v{p.variant} split={p.split_k}", flush=True)
    _assert_close(_run(gpu, x, qw, qz, s), y_ref, f"auto M={m} K={k} N={n}")


@pytest.mark.parametrize("m,k,n,tile_n,variant", [
    (1, 3584, 512, 128, 5), (3, 3584, 512, 128, 5), (8, 3584, 512, 128, 5), (12, 3584, 512, 128, 6),
    (16, 3584, 512, 128, 6), (2, 2048, 1056, 128, 5), (9, 2048, 1056, 128, 6),
    (1, 3584, 18944, 256, 5), (2, 3584, 18944, 256, 5), (3, 3584, 18944, 128, 5), (8, 3584, 18944, 128, 5),
    (1, 3584, 8224, 256, 5), (5, 3584, 8224, 128, 5)])
def test_auto_strip_class_routes(gpu, m, k, n, tile_n, variant):
    """AUTO's column-strip GEMV on slim weights (1 - 7 strips of 256 columns:
    k_proj / v_proj 3584 x 512, and 2048 x 1056 whose last strip is partly
    filled) -- column singles, the 16-row singles above M = 8 -- and on wide
    shallow ones (gate_proj / up_proj 3584 x 18944; 3584 x 8224) -- column
    pairs at M <= 2, singles above; each against the oracle on three
    512-column slices (first, middle, last)."""
    p = _native.plan_for(m, n, k)
    print(f"strip-class route M={m} K={k} N={n}: {_native.PATH_NAMES[p.path]} v{p.variant} "
          f"tile_n={p.tile_n} split={p.split_k} k_waves={p.k_waves}", flush=True)
    assert p.path == _native.PATH_GEMV and p.variant == variant and p.tile_n == tile_n
    x, qw, qz, s = O.make_inputs(m, k, n, seed=70 + m)
    y = _run(gpu, x, qw, qz, s)
    for c0 in sorted({0, n // 2 - 256, n - 512}):
        w = O.dequant_awq_f32eval(qw[:, c0 // 8:(c0 + 512) // 8], qz[:, c0 // 8:(c0 + 512) // 8],
                                  s[:, c0:c0 + 512]).astype(np.float64)
        _assert_close(y[:, c0:c0 + 512], x.astype(np.float64) @ w, f"strip class M={m} N={n} columns {c0}..")


@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_auto_vocab_wide(gpu, m):
    """AUTO on a vocab-wide weight (3584 x 152064, the Qwen2-7B LM head's
    shape) at decode sizes, where the split plans' fixed-point slots
    (M x N x 8 bytes) may not fit their region and the planner takes an fp32
    partials finish instead.  Checked against the oracle on three 512-column
    slices (first, middle, last: each packed column dequantises on its own)."""
    k, n = 3584, 152064
    x, qw, qz, s = O.make_inputs(m, k, n, seed=90 + m)
    p = _native.plan_for(m, n, k)
    print(f"vocab-wide M={m} auto={_native.PATH_NAMES[p.path]} v{p.variant} split={p.split_k}", flush=True)
    y = _run(gpu, x, qw, qz, s)
    for c0 in (0, n // 2 - 256, n - 512):
        w = O.dequant_awq_f32eval(qw[:, c0 // 8:(c0 + 512) // 8], qz[:, c0 // 8:(c0 + 512) // 8],
                                  s[:, c0:c0 + 512]).astype(np.float64)
        _assert_close(y[:, c0:c0 + 512], x.astype(np.float64) @ w, f"vocab-wide M={m} columns {c0}..")


def test_decode_plans_sized_by_the_device(gpu):
    """The planner sizes its grids by the current device's compute units (read
    once per device): the GEMV and stream plans of the Qwen2-7B shapes put at
    most one workgroup on each CU and keep more than half of them busy; on
    down_proj at M = 16 the column singles with 16 rows of x take one split
    fewer than fills the CUs."""
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    print(f"device compute units: {cus}", flush=True)
    for m, k, n in [(1, 3584, 4608), (1, 3584, 37888), (4, 3584, 4608), (4, 18944, 3584), (8, 18944, 3584),
                    (16, 18944, 3584)]:
        p = _native.plan_for(m, n, k)
        assert cus // 2 < p.grid <= cus, (m, k, n, p.grid, cus)
    p = _native.plan_for(16, 3584, 18944)
    assert p.path == _native.PATH_GEMV and p.variant == 6 and p.split_k == cus // 28 - 1, (p.path, p.split_k, cus)


@pytest.mark.parametrize("m", [1, 8, 64, 512, 2048])
def test_gemm_down_m_sweep(gpu, m):
    k, n = _SHAPES["down_proj"]
    x, qw, qz, s = O.make_inputs(m, k, n, seed=1)
    rows = np.arange(m) if m <= 64 else np.random.default_rng(m).choice(m, size=64, replace=False)
    w = O.dequant_awq_f32eval(qw, qz, s).astype(np.float32)
    y_ref = x[rows].astype(np.float32) @ w
    for path in [None] + _paths_for(m, n):
        print(f"down M={m} path={path}", flush=True)
        y = _run(gpu, x, qw, qz, s, path=path)
        _assert_close(y[rows], y_ref, f"down M={m} path={path}")


def test_gemm_prefill_gate_up(gpu):
    m = 2048
    k, n = _SHAPES["gate_up_proj"]
    x, qw, qz, s = O.make_inputs(m, k, n, seed=2)
    rows = np.random.default_rng(0).choice(m, size=48, replace=False)
    w = O.dequant_awq_f32eval(qw, qz, s).astype(np.float32)
    y_ref = x[rows].astype(np.float32) @ w
    print("prefill gate_up M=2048", flush=True)
    y = _run(gpu, x, qw, qz, s)
    _assert_close(y[rows], y_ref, "gate_up M=2048")
    # size-independent property: column sums of y equal (sum of x rows) @ W
    colsum = y.astype(np.float64).sum(axis=0)
    want = (x.astype(np.float64).sum(axis=0).astype(np.float32) @ w).astype(np.float64)
    rel = np.abs(colsum - want).max() / np.abs(want).max()
    assert rel < 1e-3, rel


# --------------------------------------------------------------------------
# Split-K plans, determinism, API behaviour
# --------------------------------------------------------------------------

@pytest.mark.parametrize("m", [1, 3, 16, 20, 32, 64])
def test_skinny_plans_agree(gpu, m):
    """Every skinny main-loop variant, scale mode, K range per wave and K
    wave count gives the same result within tolerance (split-K included)."""
    k, n = 3584, 520
    x, qw, qz, s = O.make_inputs(m, k, n, seed=4)
    y_ref = O.awq_gemm_oracle(x, qw, qz, s)
    tried = 0
    for variant in (1, 2):
        for factored in (0, 1):
            for rpw in (32, 64, 128, 256, 384, 3584):
                for kw in (1, 2, 4):
                    try:
                        p = _native.plan_skinny(m, n, k, rpw, kw, variant, factored)
                    except _native.AwqNativeError:
                        continue
                    print(f"skinny plan M={m} v={variant} f={factored} rows_per_wave={rpw} k_waves={kw}", flush=True)
                    y = _run(gpu, x, qw, qz, s, plan_obj=p)
                    _assert_close(y, y_ref, f"M={m} v={variant} f={factored} rpw={rpw} kw={kw}")
                    tried += 1
    assert tried >= 12


@pytest.mark.parametrize("m", [1, 2])
def test_gemv_plans_agree(gpu, m):
    """K-streaming GEMV (variant 2, the route for N % 32 != 0): every split
    count that divides the 28 groups into whole chunks, every ring depth."""
    k, n = 3584, 1032
    x, qw, qz, s = O.make_inputs(m, k, n, seed=14)
    y_ref = O.awq_gemm_oracle(x, qw, qz, s)
    for rpw, depths in ((16, (2, 3, 4)), (32, (2, 3))):
        for depth in depths:
            for split in (1, 2, 3, 4, 7, 14, 28):
                p = _native.plan_gemv(m, n, k, rpw, 128 // rpw, variant=2, split_k=split, depth=depth)
                print(f"gemv stream plan M={m} rows_per_wave={rpw} depth={depth} split={split}", flush=True)
                y = _run(gpu, x, qw, qz, s, plan_obj=p)
                _assert_close(y, y_ref, f"gemv stream M={m} rpw={rpw} depth={depth} split={split}")


@pytest.mark.parametrize("m,k,n", [(65, 1024, 1032), (200, 3584, 520), (512, 2048, 264), (130, 18944, 128)])
def test_tile_plans_agree(gpu, m, k, n):
    """Every tile variant, and split-K counts from 1 up, give the same result."""
    x, qw, qz, s = O.make_inputs(m, k, n, seed=15)
    y_ref = O.awq_gemm_oracle(x, qw, qz, s)
    plans = [(v, sk) for v in (6, 7, 8, 9, 15) for sk in (1, 2, 3, 5, 8)]
    for variant, sk in plans:
        try:
            p = _native.plan_tile(m, n, k, variant, sk)
        except _native.AwqNativeError:
            continue
        print(f"tile plan M={m} K={k} N={n} variant={variant} split_k={sk}", flush=True)
        y = _run(gpu, x, qw, qz, s, plan_obj=p)
        _assert_close(y, y_ref, f"tile M={m} v={variant} split={sk}")


@pytest.mark.parametrize("m,k,n", [(512, 18944, 3584), (1000, 8192, 1000), (300, 3584, 2800), (513, 2048, 3000)])
def test_512_column_tile_matches_256_column_tile(gpu, m, k, n):
    """Variant 15 (eight waves on 512-column tiles) computes every output as
    variant 7 does: one wave over the same K order within a split, the splits
    summed in split order by the same reduce launch.  So at every split both
    accept the two must be bit-identical -- with ragged M, and ragged N where a
    512-column tile's second half starts at or beyond N (N = 1000, 2800, 3000)
    -- and within tolerance of the oracle; one-hot rows of x give each weight
    exactly."""
    x, qw, qz, s = O.make_inputs(m, k, n, seed=18)
    w = O.dequant_awq(qw, qz, s)
    y_ref = x.astype(np.float32) @ w.astype(np.float32)
    rows = np.random.default_rng(19).integers(0, k, size=m)
    x1 = np.zeros((m, k), dtype=np.float16)
    x1[np.arange(m), rows] = 1.0
    want = (w[rows] + np.float16(0)).view(np.uint16)
    tried = 0
    for sk in (1, 2, 3, 4, 8):
        try:
            p15 = _native.plan_tile(m, n, k, 15, sk)
            p7 = _native.plan_tile(m, n, k, 7, sk)
        except _native.AwqNativeError:
            continue
        print(f"512-column tile M={m} K={k} N={n} split_k={sk} grid={p15.grid}", flush=True)
        y15 = _run(gpu, x, qw, qz, s, plan_obj=p15)
        _assert_close(y15, y_ref, f"tile v15 M={m} split={sk}")
        y7 = _run(gpu, x, qw, qz, s, plan_obj=p7)
        assert np.array_equal(y15.view(np.uint16), y7.view(np.uint16)), f"v15 != v7 M={m} N={n} split={sk}"
        y1 = _run(gpu, x1, qw, qz, s, plan_obj=p15)
        assert np.array_equal((y1 + np.float16(0)).view(np.uint16), want), f"one-hot v15 split={sk}"
        tried += 1
    assert tried >= 3


@pytest.mark.parametrize("m,k,n", [(2048, 3584, 4608), (2100, 1024, 4104), (2600, 1280, 3584)])
def test_tile_hybrid_plans(gpu, m, k, n):
    """The hybrid tiles (variants 13, 14: a whole tile per CU slot, the leftover
    tiles split along K with compact partials and a last-arriver finish), on
    every output against the oracle, with ragged M and N, and bit-exact with
    one-hot rows of x (each output is one weight: every tile and K piece must
    land in its own place)."""
    x, qw, qz, s = O.make_inputs(m, k, n, seed=16)
    w = O.dequant_awq(qw, qz, s)
    y_ref = x.astype(np.float32) @ w.astype(np.float32)
    rows = np.random.default_rng(17).integers(0, k, size=m)
    x1 = np.zeros((m, k), dtype=np.float16)
    x1[np.arange(m), rows] = 1.0
    want = (w[rows] + np.float16(0)).view(np.uint16)
    tried = 0
    for variant in (13, 14):
        for sk in (2, 3, 4, 5, 7):
            try:
                p = _native.plan_tile(m, n, k, variant, sk)
            except _native.AwqNativeError:
                continue
            print(f"hybrid tile M={m} K={k} N={n} variant={variant} split_k={sk} grid={p.grid}", flush=True)
            _assert_close(_run(gpu, x, qw, qz, s, plan_obj=p), y_ref, f"hybrid M={m} v={variant} split={sk}")
            y1 = _run(gpu, x1, qw, qz, s, plan_obj=p)
            assert np.array_equal((y1 + np.float16(0)).view(np.uint16), want), f"one-hot hybrid v={variant} split={sk}"
            tried += 1
    assert tried >= 4


def _random_shapes(count, seed, kind="any"):
    """(M, K, N) drawn from a fixed seed.  "any": M over the decode, small-M
    and prefill routes, K any multiple of 128 up to 4992, N any multiple of 8
    up to 9592, at most 3e9 multiply-adds each; "decode": M <= 16 and N a
    multiple of 32 (the GEMV and stream routes); "prefill": M from 512 to
    2100, K up to 4992, N up to 12800 (the tile routes and hybrids);
    "strips": M <= 16, N a multiple of 32 from 256 to 8160, K from 2048 to
    12800 (the column-strip GEMV classes, 16-row singles included), at most
    40 M weights."""
    rng = np.random.default_rng(seed)
    ms = {"any": [1, 2, 3, 4, 5, 6, 7, 8, 9, 11, 13, 16, 17, 20, 24, 31, 33, 48, 64, 65, 100, 129, 200, 257, 513,
                  1000],
          "decode": list(range(1, 17)), "prefill": [512, 600, 1024, 1500, 2048, 2100],
          "strips": list(range(1, 17))}[kind]
    out = []
    while len(out) < count:
        if kind == "strips":
            m, k, n = int(rng.choice(ms)), 128 * int(rng.integers(16, 101)), 32 * int(rng.integers(8, 256))
            if k * n <= 40e6:
                out.append((m, k, n))
            continue
        m, k = int(rng.choice(ms)), 128 * int(rng.integers(1, 40))
        n = 32 * int(rng.integers(1, 400)) if kind == "decode" else 8 * int(rng.integers(1, 1600 if kind == "prefill"
                                                                                           else 1200))
        if kind != "any" or m * n * k <= 3e9:
            out.append((m, k, n))
    return out


@pytest.mark.parametrize("m,k,n", _random_shapes(40, 2027) + _random_shapes(16, 2028, "decode") +
                         _random_shapes(6, 2029, "prefill") + _random_shapes(12, 2030, "strips"))
def test_auto_random_shapes(gpu, m, k, n):
    """AUTO on shapes no other test fixes, drawn at random: every output
    against the oracle's dequantised product, whichever route and split the
    dispatcher takes for the shape (N not a multiple of 32 or of a tile,
    K of a few groups, M between the routes' bounds, strip widths and K of
    the column-strip GEMV classes)."""
    x, qw, qz, s = O.make_inputs(m, k, n, seed=m + k + n)
    w = O.dequant_awq(qw, qz, s)
    y_ref = x.astype(np.float32) @ w.astype(np.float32)
    p = _native.plan_for(m, n, k)
    print(f"random shape M={m} K={k} N={n}: {_native.PATH_NAMES[p.path]} v{p.variant} split={p.split_k}", flush=True)
    _assert_close(_run(gpu, x, qw, qz, s), y_ref, f"random M={m} K={k} N={n}")


def test_auto_many_random_shapes_against_fp32(gpu):
    """AUTO on 300 seeded random shapes at once (M from 1 to 2100, K any
    multiple of 128 up to 18944, N any multiple of 8 up to 40000, at most
    1.5e11 multiply-adds): the output against a plain PyTorch fp32 product of
    the same operands (x in fp32 times the weight dequantised by
    awq_w4a16_dequant, which the tests above pin bit for bit to the oracle),
    and the fused bias + residual epilogue bit-identical to torch's fp16 adds
    on the GEMM's own output.  Covers every route, variant and split-K finish
    AUTO takes over that range (the GEMV, skinny, stream and tile kernels and
    the hybrids)."""
    rng = np.random.default_rng(303)
    ms = list(range(1, 17)) + [17, 20, 24, 31, 32, 33, 40, 48, 63, 64, 65, 80, 96, 100, 128, 129, 200, 256, 257,
                               384, 500, 512, 513, 700, 1000, 1024, 1500, 2048, 2100]
    routes, done = set(), 0
    while done < 300:
        m, k, n = int(rng.choice(ms)), 128 * int(rng.integers(1, 149)), 8 * int(rng.integers(1, 5000))
        if m * k * n > 1.5e11 or k * n > 6e8:
            continue
        g = torch.Generator(device=gpu)
        g.manual_seed(done)
        x = torch.randn((m, k), generator=g, device=gpu).half()
        qw = torch.randint(-2**31, 2**31 - 1, (k, n // 8), generator=g, device=gpu, dtype=torch.int32)
        qz = torch.randint(-2**31, 2**31 - 1, (k // 128, n // 8), generator=g, device=gpu, dtype=torch.int32)
        sc = (torch.rand((k // 128, n), generator=g, device=gpu) * 0.018 + 0.002).half()
        bias = (torch.randn(n, generator=g, device=gpu) * 0.5).half()
        res = (torch.randn((m, n), generator=g, device=gpu) * 4).half()
        y = awq_gemm_forward(x, qw, qz, sc)
        w = torch.empty((k, n), dtype=torch.float16, device=gpu)
        _dequant_to_fp16(qw, qz, sc, w)
        ref = torch.matmul(x.float(), w.float())
        fused = awq_gemm_forward_ex(x, qw, qz, sc, bias=bias, residual=res)
        unfused = res + (y + bias)
        torch.cuda.synchronize()
        p = _native.plan_for(m, n, k)
        what = f"random M={m} K={k} N={n} ({_native.PATH_NAMES[p.path]} v{p.variant} split={p.split_k})"
        _assert_close(y.float().cpu().numpy(), ref.cpu().numpy(), what)
        assert torch.equal(fused.view(torch.int16), unfused.view(torch.int16)), what + ": epilogue"
        routes.add((p.path, p.variant, p.split_k > 1))
        done += 1
    print(f"{done} random shapes over {len(routes)} routes", flush=True)
    assert len(routes) >= 12, routes


@pytest.mark.parametrize("m", [1, 2])
def test_gemv_quad_plans_agree(gpu, m):
    """Column-quad GEMV (balanced K split, fixed-point split-K finish): split
    counts from 1 up to one 16-row step per workgroup, every wave count, on
    an N whose last 512-column strip holds a single quad."""
    k, n = 3584, 1056
    x, qw, qz, s = O.make_inputs(m, k, n, seed=24)
    y_ref = O.awq_gemm_oracle(x, qw, qz, s)
    tried = 0
    for variant in (5,):
        for split in (1, 2, 3, 5, 16, 37, 100, 112):
            for kw in (1, 2, 3, 4, 8):
                for depth in (2, 3, 4):
                    try:
                        p = _native.plan_gemv(m, n, k, 0, kw, variant=variant, split_k=split, depth=depth)
                    except _native.AwqNativeError:
                        continue  # too many groups per workgroup for this wave count
                    print(f"gemv quad plan M={m} variant={variant} split={split} k_waves={kw} depth={depth}",
                          flush=True)
                    y = _run(gpu, x, qw, qz, s, plan_obj=p)
                    _assert_close(y, y_ref, f"gemv quad M={m} v={variant} split={split} kw={kw} d={depth}")
                    tried += 1
    assert tried >= 80


@pytest.mark.parametrize("tile_n,m", [(256, 1), (256, 2), (256, 3), (256, 4), (128, 1), (128, 2), (128, 3), (128, 4),
                                      (128, 5), (128, 7), (128, 8)])
def test_gemv_pair_plans_agree(gpu, m, tile_n):
    """Column-pair and column-single GEMV (256- and 128-column strips, up to 4
    and 8 rows of x -- above 4, lanes of two k-blocks hold the rows --,
    fixed-point split-K finish): split counts from 1 up to one 32-row chunk
    per workgroup, wave counts 1 - 8, ring depths 2 and 3, on an N whose last
    strip is partly filled (1056 = 4 x 256 + 32 = 8 x 128 + 32)."""
    k, n = 3584, 1056
    x, qw, qz, s = O.make_inputs(m, k, n, seed=25 + m)
    y_ref = O.awq_gemm_oracle(x, qw, qz, s)
    tried = 0
    for split in (1, 2, 3, 5, 16, 37, 100, 112):
        for kw in (1, 2, 4, 8):
            for depth in (2, 3):
                try:
                    p = _native.plan_gemv(m, n, k, 0, kw, variant=5, split_k=split, depth=depth, tile_n=tile_n)
                except _native.AwqNativeError:
                    continue
                print(f"gemv {tile_n}-column strips M={m} split={split} k_waves={kw} depth={depth}", flush=True)
                y = _run(gpu, x, qw, qz, s, plan_obj=p)
                _assert_close(y, y_ref, f"gemv {tile_n} M={m} split={split} kw={kw} d={depth}")
                tried += 1
    assert tried >= 40


@pytest.mark.parametrize("m", [9, 12, 16])
def test_gemv_singles_reduce_plans_agree(gpu, m):
    """Column singles with fp32 partials added by a second reduce launch
    (GEMV variant 6, 128-column strips, 9 - 16 rows of x in the lanes of all
    four k-blocks): split counts from 1 (direct finish, two row batches) up to
    one 32-row chunk per workgroup, wave counts 1 - 8, on an N whose last
    strip is partly filled."""
    k, n = 2048, 1056
    x, qw, qz, s = O.make_inputs(m, k, n, seed=41 + m)
    y_ref = O.awq_gemm_oracle(x, qw, qz, s)
    tried = 0
    for split in (1, 2, 3, 9, 37, 64):
        for kw in (1, 2, 4, 8):
            try:
                p = _native.plan_gemv(m, n, k, 0, kw, variant=6, split_k=split, depth=2, tile_n=128)
            except _native.AwqNativeError:
                continue
            print(f"gemv singles + reduce M={m} split={split} k_waves={kw}", flush=True)
            y = _run(gpu, x, qw, qz, s, plan_obj=p)
            _assert_close(y, y_ref, f"gemv singles reduce M={m} split={split} kw={kw}")
            tried += 1
    assert tried >= 12


@pytest.mark.parametrize("m", [1, 3, 4, 5, 8, 9, 16])
def test_stream_plans_agree(gpu, m):
    """Stream path (16x16x32 MFMA, zero/scale folded per group), both layouts
    (row: whole row segments per load, M <= 8; half-strip wave pairs): every
    split-K finish (fixed-point slots, last-arriving workgroup, second reduce
    launch), split counts from 1 to one group per workgroup, wave counts and
    ring depths, on an N whose last 512-column strip holds a single packed-
    column pair of each half."""
    k, n = 3584, 1056
    x, qw, qz, s = O.make_inputs(m, k, n, seed=25 + m)
    y_ref = O.awq_gemm_oracle(x, qw, qz, s)
    tried = 0
    shapes = [("half", kw, d) for kw, d in ((1, 2), (2, 2), (3, 2), (4, 2), (1, 4), (2, 4), (1, 6), (2, 6))]
    if m <= 8:
        shapes += [("row", kw, 2) for kw in (1, 2, 4, 8)] + [("row", kw, 1) for kw in (4, 8)]
    for variant in (1, 2, 3):
        for split in (1, 2, 3, 5, 9, 14, 28):
            for layout, kw, depth in shapes:
                try:
                    p = _native.plan_stream(m, n, k, kw, split, variant=variant, depth=depth, layout=layout)
                except _native.AwqNativeError:
                    continue  # too many groups per workgroup for this wave count
                what = f"stream M={m} {layout} v={variant} split={split} k_waves={kw} depth={depth}"
                print(what, flush=True)
                y = _run(gpu, x, qw, qz, s, plan_obj=p)
                _assert_close(y, y_ref, what)
                tried += 1
    assert tried >= (170 if m <= 8 else 120)


def test_stream_and_quad_one_hot_bit_exact(gpu):
    """One-hot rows of x reproduce the dequantised rows bit for bit through the
    stream kernel and the column-quad GEMV, with and without split-K: with one
    nonzero x the group sums are 1024 + q' and 1, the folded result
    s' (1024 + q') - s' (1024 + z') = s (q - z) is exact in fp32, and the
    fixed-point and partial finishes add exact zeros.  The tile kernels form
    the fp16 weight itself."""
    k, n = 512, 288
    _, qw, qz, s = O.make_inputs(1, k, n, seed=33)
    w = O.dequant_awq(qw, qz, s)
    for m in (1, 2, 4, 16):
        rows = np.random.default_rng(m).integers(0, k, size=m)
        x = np.zeros((m, k), dtype=np.float16)
        x[np.arange(m), rows] = 1.0
        plans = [_native.plan_stream(m, n, k, kw, sp, variant=v, depth=d) for v in (1, 2, 3) for sp in (1, 2, 4)
                 for kw, d in ((1, 2), (4, 2), (2, 4), (2, 6))]
        if m <= 8:
            plans += [_native.plan_stream(m, n, k, kw, sp, variant=v, depth=d, layout="row") for v in (1, 2, 3)
                      for sp in (1, 2, 4) for kw, d in ((1, 2), (8, 2), (4, 2), (8, 1))]
        if m <= 2:
            plans += [_native.plan_gemv(m, n, k, 0, 4, variant=5, split_k=sp) for sp in (1, 3, 16)]
        if m == 16:
            plans += [_native.plan_tile(m, n, k, v, sp) for v in (6, 7, 8, 9, 15) for sp in (1, 2, 4)]
        for p in plans:
            print(f"one-hot M={m} path={_native.PATH_NAMES[p.path]} v={p.variant} split={p.split_k}", flush=True)
            y = _run(gpu, x, qw, qz, s, plan_obj=p)
            assert np.array_equal(y.view(np.uint16), w[rows].view(np.uint16)), (m, p.path, p.split_k)


def test_split_k_workspace_left_zero(gpu):
    """Every split-K finish leaves the counter block and the fixed-point
    slot region of the shared workspace zero (arrival counters reset, slots
    cleared), so it is ready for the next call of any path and for graph
    replays.  The partials region is never cleared: every call writes each
    partial it reads.  To show that no finish reads a partial before writing
    it, each case runs on a zeroed workspace, then again with the whole
    partials region filled with NaN, and the two outputs must be finite and
    bit-identical."""
    from kernels import awq_gemm as G
    k, n = 3584, 4608
    cases = [(m, _native.plan_for(m, n, k, path=path))
             for m, path in ((1, _native.PATH_GEMV), (4, _native.PATH_SKINNY),
                             (100, _native.PATH_TILE), (16, _native.PATH_STREAM), (3, _native.PATH_STREAM))]
    cases += [(m, _native.plan_stream(m, n, k, 4, sp, variant=v)) for m, v, sp in ((2, 1, 28), (4, 2, 8), (16, 2, 2))]
    cases += [(m, _native.plan_stream(m, n, k, kw, sp, variant=v, layout="row", depth=d))
              for m, v, sp, kw, d in ((3, 1, 28, 8, 1), (5, 2, 6, 8, 2), (8, 3, 28, 8, 1))]
    cases += [(m, _native.plan_stream(m, n, k, 3, 14, variant=3)) for m in (9, 16)]
    cases += [(m, _native.plan_gemv(m, n, k, 16, 8, variant=2, split_k=sp, depth=3)) for m, sp in ((1, 7), (2, 14))]
    cases += [(m, _native.plan_gemv(m, n, k, 0, 8, variant=6, split_k=sp, tile_n=128)) for m, sp in ((9, 6), (16, 9))]
    cases += [(m, _native.plan_tile(m, n, k, v, sp)) for m, v, sp in
              ((100, 6, 4), (200, 7, 3), (100, 8, 4), (70, 9, 7), (2048, 13, 2), (2048, 14, 3))]
    ws = G._workspace(gpu, max(int(p.workspace_bytes) for _, p in cases))
    kept_zero = (_native.counter_bytes() + _native.SLOT_BYTES) // 4
    for m, p in cases:
        x, qw, qz, s = O.make_inputs(m, k, n, seed=6)
        assert p.split_k > 1, (m, p.path)
        name = f"{_native.PATH_NAMES[p.path]} v={p.variant} M={m} split={p.split_k}"
        print(f"workspace check {name}", flush=True)
        ws.zero_()
        y = _run(gpu, x, qw, qz, s, plan_obj=p)
        assert G._workspace_buffers(gpu)[-1].data_ptr() == ws.data_ptr(), "the workspace was replaced"
        assert int((ws.view(torch.int32)[:kept_zero] != 0).sum().item()) == 0, name
        ws[kept_zero:].fill_(float("nan"))
        y2 = _run(gpu, x, qw, qz, s, plan_obj=p)
        assert int((ws.view(torch.int32)[:kept_zero] != 0).sum().item()) == 0, name
        assert np.isfinite(y).all() and np.isfinite(y2).all(), name
        assert np.array_equal(y.view(np.uint16), y2.view(np.uint16)), name


def test_deterministic(gpu):
    for m, (k, n) in [(1, _SHAPES["down_proj"]), (16, _SHAPES["q_proj"]), (300, (1024, 1024))]:
        x, qw, qz, s = O.make_inputs(m, k, n, seed=8)
        a = _run(gpu, x, qw, qz, s)
        b = _run(gpu, x, qw, qz, s)
        assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), f"M={m}"


def test_leading_dims_and_empty(gpu):
    k, n = 256, 64
    x, qw, qz, s = O.make_inputs(6, k, n, seed=12)
    y_ref = C.gemm_f64(x, qw, qz, s)
    x3 = _t(x, gpu).view(2, 3, k)
    y = awq_gemm_forward(x3, _t(qw, gpu), _t(qz, gpu), _t(s, gpu))
    assert tuple(y.shape) == (2, 3, n)
    _assert_close(y.reshape(6, n).cpu().numpy(), y_ref, "3-D x")
    e = awq_gemm_forward(torch.empty((0, k), dtype=torch.float16, device=gpu), _t(qw, gpu), _t(qz, gpu),
                         _t(s, gpu))
    assert tuple(e.shape) == (0, n)


def test_noncontiguous_operands(gpu):
    k, n = 256, 128
    x, qw, qz, s = O.make_inputs(3, k, n, seed=13)
    y_ref = C.gemm_f64(x, qw, qz, s)
    qw_t = _t(np.ascontiguousarray(qw.T), gpu).t()
    s_t = _t(np.ascontiguousarray(s.T), gpu).t()
    x_wide = torch.zeros((3, 2 * k), dtype=torch.float16, device=gpu)
    x_wide[:, :k] = _t(x, gpu)
    y = awq_gemm_forward(x_wide[:, :k], qw_t, _t(qz, gpu), s_t)
    _assert_close(y.cpu().numpy(), y_ref, "non-contiguous")


def test_misaligned_operands_are_copied(gpu):
    """x, scales and a caller's out= at storage offsets that are not 16-byte
    aligned (the reference's Triton path takes any fp16 view): the entry
    points copy to aligned buffers instead of raising, and the results are
    bit-identical to the aligned call, including an in-place residual add
    into a misaligned out."""
    k, n, m = 3584, 4608, 3
    x, qw, qz, s = O.make_inputs(m, k, n, seed=17)
    X, QW, QZ, S = (_t(a, gpu) for a in (x, qw, qz, s))
    want = awq_gemm_forward(X, QW, QZ, S)
    xbuf = torch.empty(m * k + 1, dtype=torch.float16, device=gpu)
    xo = xbuf[1:].view(m, k)
    xo.copy_(X)
    sbuf = torch.empty(S.numel() + 3, dtype=torch.float16, device=gpu)
    so = sbuf[3:].view(S.shape)
    so.copy_(S)
    assert xo.data_ptr() % 16 and so.data_ptr() % 16
    for xx, ss, what in ((xo, S, "x"), (X, so, "scales"), (xo, so, "x and scales")):
        got = awq_gemm_forward(xx, QW, QZ, ss)
        torch.cuda.synchronize()
        assert torch.equal(got, want), what
    obuf = torch.empty(m * n + 1, dtype=torch.float16, device=gpu)
    oo = obuf[1:].view(m, n)
    got = awq_gemm_forward_ex(xo, QW, QZ, S, out=oo)
    assert got.data_ptr() == oo.data_ptr() and torch.equal(oo, want), "out="
    res = torch.randn((m, n), device=gpu).half()
    oo.copy_(res)
    awq_gemm_forward_ex(X, QW, QZ, S, out=oo, residual=oo)
    torch.cuda.synchronize()
    assert torch.equal(oo, (res.float() + want.float()).half()), "out= with residual=out"


def test_errors_raise(gpu):
    k, n = 256, 64
    x, qw, qz, s = O.make_inputs(2, k, n)
    X, QW, QZ, S = (_t(a, gpu) for a in (x, qw, qz, s))
    with pytest.raises(ValueError):
        awq_gemm_forward(X.float(), QW, QZ, S)
    with pytest.raises(ValueError):
        awq_gemm_forward(X, QW[:, :4], QZ, S)
    with pytest.raises(ValueError):
        awq_gemm_forward(X, QW, QZ, S, group_size=64)
    with pytest.raises(_native.AwqNativeError):
        awq_gemm_forward_ex(torch.zeros((100, k), dtype=torch.float16, device=gpu), QW, QZ, S,
                            path=_native.PATH_SKINNY)


def test_graph_capture_replay(gpu):
    """Captured into a graph (split-K workspace included), every replay matches
    eager bit for bit: the GEMV, the stream kernels (M = 2, 4), the 32-row
    tile with its reduce launch (M = 16), a small-M tile and the hybrid tile
    (M = 2048)."""
    shapes = [(1, 3584, 512), (2, 3584, 4608), (4, 3584, 3584), (16, 3584, 4608), (200, 1024, 1024),
              (2048, 3584, 4608)]
    inputs = []
    for m, k, n in shapes:
        x, qw, qz, s = O.make_inputs(m, k, n, seed=m)
        inputs.append(tuple(_t(a, gpu) for a in (x, qw, qz, s)))
    eager = [awq_gemm_forward(*t) for t in inputs]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for t in inputs:  # warm-up on the capture stream
            awq_gemm_forward(*t)
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = [awq_gemm_forward(*t) for t in inputs]
    for rep in range(3):
        for o in outs:
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        # unrelated eager work between replays
        _ = awq_gemm_forward(*inputs[0]) + 1
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), f"replay {rep}"


# --------------------------------------------------------------------------
# Golden fixtures (tests/golden/make_golden.py: plain-Python values)
# --------------------------------------------------------------------------

def _golden(name):
    import os

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", name)
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", ["awq_golden_small.npz", "awq_golden_edge.npz"])
def test_golden_dequant_bit_exact(gpu, name):
    print(f"golden dequant {name}", flush=True)
    d = _golden(name)
    qw, qz = d["qweight"], d["qzeros"]
    s = d["scales_f16_bits"].view(np.float16)
    k, n = qw.shape[0], s.shape[1]
    out = torch.empty((k, n), dtype=torch.float16, device=gpu)
    _dequant_to_fp16(_t(qw, gpu), _t(qz, gpu), _t(s, gpu), out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint16), d["w_f16_bits"])


def test_golden_small_gemm_every_path(gpu):
    """The fixture's correctly rounded products, through every kernel path and
    every row count the fixture's 5 rows allow."""
    d = _golden("awq_golden_small.npz")
    x = d["x_f16_bits"].view(np.float16)
    qw, qz = d["qweight"], d["qzeros"]
    s = d["scales_f16_bits"].view(np.float16)
    for m in (1, 2, 5):
        for path in _paths_for(m, s.shape[1]):
            print(f"golden gemm M={m} path={_native.PATH_NAMES[path]}", flush=True)
            y = _run(gpu, x[:m], qw, qz, s, path=path)
            _assert_close(y, d["y_f64"][:m], f"golden M={m} path={path}")


def test_golden_edge_gemm_finite_columns(gpu):
    """Edge-case scales (subnormal, ties, negative, signed zeros) through every
    path, element by element: |y - y_ref| <= 1.1 * 2^-10 * sum_k |x_k w_k|
    + 2^-23, which covers the fp16 rounding of the output (2^-11 relative, and
    the subnormal quantum 2^-24), the per-weight fp16 rounding that the GEMV
    and factored skinny paths skip by scaling the fp32 group sum (2^-11
    relative per term) and the fp32 accumulation (K * 2^-24 relative).
    Outputs beyond the fp16 range must be infinities of the right sign.
    Columns whose fp16 weights overflow to +-inf are left out: the reference's
    output there is inf/NaN, while the paths that scale the group sum stay
    finite."""
    d = _golden("awq_golden_edge.npz")
    x = d["x_f16_bits"].view(np.float16)
    qw, qz = d["qweight"], d["qzeros"]
    s = d["scales_f16_bits"].view(np.float16)
    w = d["w_f16_bits"].view(np.float16).astype(np.float64)
    keep = np.isfinite(w).all(axis=0)
    assert 0 < keep.sum() < w.shape[1]
    for m in (1, 2, 3):
        y_ref = d["y_f64"][:m][:, keep]
        mag = (np.abs(x[:m].astype(np.float64)) @ np.abs(w[:, keep]))
        tol = 1.1 * 2.0 ** -10 * mag + 2.0 ** -23
        big = np.abs(y_ref) > 65600.0
        small = np.abs(y_ref) < 65400.0
        for path in _paths_for(m, s.shape[1]):
            print(f"golden edge gemm M={m} path={_native.PATH_NAMES[path]}", flush=True)
            y = _run(gpu, x[:m], qw, qz, s, path=path)[:, keep].astype(np.float64)
            assert np.all(np.isinf(y[big]) & (np.sign(y[big]) == np.sign(y_ref[big]))), f"M={m} path={path}"
            err = np.abs(y[small] - y_ref[small])
            assert np.all(err <= tol[small]), (
                f"M={m} path={path}: worst excess {np.max(err - tol[small]):.3e}")
