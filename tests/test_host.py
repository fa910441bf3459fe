"""Host-side tests that need no GPU: the C ABI library loads and exports what
include/awq_w4a16.h declares, the shape dispatcher and plan validation, the
argument checks of the C ABI and of the Python entry point (every call here
fails validation, or has M = 0, before any device work), the roofline
arithmetic and the bench's one-GPU contract."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest
import torch

from kernels import _native
from kernels import awq_roofline as R

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "awq_w4a16.h")

SHAPES = [(k, n) for _, k, n in R.QWEN2_7B_LINEARS + R.QWEN2_7B_FUSED]


@pytest.fixture(scope="module")
def L():
    if not os.path.exists(_native.LIB_PATH):
        import importlib.util

        spec = importlib.util.spec_from_file_location(
            "_awq_build", os.path.join(ROOT, "qwen2-7b-triton_engine_amd", "build.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    return _native.lib()


def _declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(awq_(?:w4a16_|fp16_|silu_)[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(L):
    declared = _declared_symbols()
    assert len(declared) >= 10
    for name in declared:
        assert hasattr(L, name), f"{name} declared in include/awq_w4a16.h but not exported"
    assert sorted(_native.SIGNATURES) == declared


def test_abi_version_and_error_strings(L):
    assert L.awq_w4a16_abi_version() == _native.ABI_VERSION
    codes = [_native.AWQ_OK, _native.AWQ_ERR_NULL_POINTER, _native.AWQ_ERR_BAD_DIMS,
             _native.AWQ_ERR_GROUP_SIZE, _native.AWQ_ERR_MISALIGNED, _native.AWQ_ERR_WORKSPACE,
             _native.AWQ_ERR_LAUNCH, _native.AWQ_ERR_PATH, _native.AWQ_ERR_TOO_LARGE,
             _native.AWQ_ERR_SCRATCH, _native.AWQ_ERR_CAPTURE]
    msgs = [_native.error_string(c) for c in codes]
    assert len(set(msgs)) == len(msgs)
    assert _native.error_string(-99) == "unknown status"


def test_plan_struct_matches_header():
    # 10 int32 fields, one int64, two uint64: 64 bytes, no padding.
    assert ctypes.sizeof(_native.Plan) == 64
    text = open(HEADER).read()
    body = re.search(r"typedef struct awq_w4a16_plan\s*\{(.*?)\}\s*awq_w4a16_plan;", text, re.S).group(1)
    fields = re.findall(r"\b(int32_t|int64_t|uint64_t)\s+(\w+);", body)
    assert [f for _, f in fields] == [f for f, _ in _native.Plan._fields_]


# ---------------------------------------------------------------------------
# Shape dispatcher
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("k,n", SHAPES)
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 7, 8, 12, 16, 17, 33, 64, 65, 128, 512, 2048, 2049])
def test_auto_plan_invariants(L, m, k, n):
    p = _native.plan_for(m, n, k)
    strips = -(-(n // 8) // 64)            # 512-column strips of the stream path
    stream = n % 32 == 0 and m <= 16 and (m <= 4 or strips >= 16 or k >= 8192)
    # 9 <= M <= 16 on deep, narrow weights: column singles with 16 rows of x
    # and the reduce launch, one split fewer than fills the CUs (256 without
    # a GPU); else the 32-row tile with five groups per split where that grid
    # covers every CU and fits two workgroups per CU
    strips128 = -(-(n // 8) // 16)
    strips256 = -(-(n // 8) // 32)
    deep_gemv = (9 <= m <= 16 and k >= 8192 and n % 32 == 0 and strips < 16 and strips256 >= 8
                 and 256 // strips128 - 1 >= 2)
    deep_split = -(-(k // 128) // 5)
    deep_tile = 9 <= m <= 16 and k >= 8192 and strips < 16 and 256 <= -(-n // 256) * deep_split <= 512
    # column singles (128-column strips) on narrow weights at M <= 8
    pairs = n % 32 == 0 and strips < 16 and strips256 >= 8 and m <= 8
    # slim weights (1 - 7 strips of 256, 2048 <= K < 8192): singles with two
    # waves and four chunks per workgroup at M <= 8, the 16-row singles with
    # one workgroup per CU above; wide shallow ones with >= 3 splits of the
    # 256-column strips per CU: pairs at M <= 2, singles to M = 8
    slim = n % 32 == 0 and n >= 256 and strips256 < 8 and 2048 <= k < 8192 and m <= 16
    wide = n % 32 == 0 and strips >= 16 and k < 8192 and 256 // strips256 >= 3 and m <= 8
    if pairs:
        assert p.path == _native.PATH_GEMV and p.variant == 5 and p.tile_m >= m and p.tile_n == 128
        assert 0.5 * 256 < p.grid <= 256
    elif slim:
        assert p.path == _native.PATH_GEMV and p.tile_n == 128
        if m <= 8:
            assert p.variant == 5 and p.k_waves == 2 and p.split_k == min((k // 32) // 4, 256 // strips128)
        else:
            assert p.variant == 6 and p.k_waves == 8 and p.split_k == 256 // strips128
    elif wide:
        assert p.path == _native.PATH_GEMV and p.variant == 5 and p.split_k == 256 // strips256
        assert p.tile_n == (256 if m <= 2 else 128)
    elif m == 1 or (m == 2 and n % 32 != 0):
        assert p.path == _native.PATH_GEMV
    elif deep_gemv:
        assert p.path == _native.PATH_GEMV and p.variant == 6 and p.tile_n == 128 and p.k_waves == 8
        assert p.split_k == 256 // strips128 - 1 and p.grid == strips128 * p.split_k <= 256
    elif deep_tile:
        assert p.path == _native.PATH_TILE and p.variant == 9 and p.split_k == deep_split
    elif stream:
        assert p.path == _native.PATH_STREAM
        assert p.tile_m >= m
        assert p.split_k <= k // 128
    elif m <= 16:
        # 5 <= M <= 16: the 32-row tile split 14 ways along K where its grid
        # covers half the CUs, else the skinny kernel
        units = k // 128
        split = min(14, units)
        split = -(-units // -(-units // split))
        small_tile = m >= 5 and -(-n // 256) * split * 2 >= 256
        if small_tile:
            assert p.path == _native.PATH_TILE and p.variant == 9 and p.split_k == split
        else:
            assert p.path == _native.PATH_SKINNY
            assert p.tile_m >= m
    else:
        assert p.path == _native.PATH_TILE
        if m <= 1024 and -(-m // 128) * -(-n // 256) < 512:
            assert p.variant >= 6           # the register-dequant tiles, by the cost model
            assert p.variant in (7, 8, 9, 13, 14, 15)   # by the cost model; 6 = 7 with the one-launch finish
    assert p.grid > 0 and p.block_threads % 64 == 0 and p.block_threads <= 1024
    if p.split_k > 1:
        if (p.path == _native.PATH_GEMV and p.variant in (4, 5)) or (p.path == _native.PATH_STREAM and p.variant == 1):
            # one 64-bit fixed-point slot per output element
            assert p.workspace_bytes == _native.counter_bytes() + m * n * 8
            assert p.split_k <= 255
        elif p.path == _native.PATH_TILE and p.variant in (13, 14):
            # hybrid: compact partials of the leftover tiles only
            tm = 128 if p.variant == 13 else 64
            tiles = -(-m // tm) * -(-n // 256)
            left = tiles % 256
            assert p.grid == tiles - left + left * p.split_k
            assert p.workspace_bytes == (_native.counter_bytes() + _native.SLOT_BYTES +
                                         p.split_k * left * tm * 256 * 4)
        elif p.path == _native.PATH_TILE and p.variant in (7, 8, 9, 15):
            # reduce launch: fragment-native units of 16 rows x 256 columns
            assert p.workspace_bytes == (_native.counter_bytes() + _native.SLOT_BYTES +
                                         p.split_k * -(-m // 16) * 16 * -(-n // 256) * 256 * 4)
        else:
            assert p.workspace_bytes == _native.counter_bytes() + _native.SLOT_BYTES + p.split_k * m * n * 4
    else:
        assert p.workspace_bytes == 0
    assert _native.workspace_bytes(m, n, k) == p.workspace_bytes


@pytest.mark.parametrize("m,n,k", [(1, 262144, 4096), (2, 152064, 3584), (2, 262144, 4096), (3, 262144, 3584),
                                   (4, 152064, 3584), (4, 65536, 18944)])
def test_auto_plan_falls_back_when_slots_do_not_fit(L, m, n, k):
    """Where the fixed-point slots of a split plan (M x N x 8 bytes) exceed the
    slot region, AUTO still serves the shape, with an fp32-partials finish or
    without a split, and never asks for more slots than the region holds."""
    p = _native.plan_for(m, n, k)
    fixed_point = (p.path == _native.PATH_GEMV and p.variant in (4, 5)) or \
                  (p.path == _native.PATH_STREAM and p.variant == 1)
    if p.split_k > 1 and fixed_point:
        assert m * n * 8 <= _native.SLOT_BYTES
    if m * n * 8 > _native.SLOT_BYTES and p.split_k > 1:
        assert not fixed_point
        assert p.workspace_bytes == _native.counter_bytes() + _native.SLOT_BYTES + p.split_k * m * n * 4


def test_stream_split_keeps_a_group_and_a_half_per_split(L):
    """The stream planner (AUTO's choice at M = 2 .. 4 on wide weights, and
    the explicit stream path elsewhere): K = 3584 (28 groups) at M = 2 .. 4
    gets 18 splits, the cap of 2 x groups / 3; M = 2 takes the half-strip
    layout with two wave pairs there, the row layout with four waves on deep
    weights (148 groups, 36 splits)."""
    S = _native.PATH_STREAM
    for m in (2, 3, 4):
        for n in (4608, 3584):
            p = _native.plan_for(m, n, 3584, path=S)
            assert p.path == S and p.split_k == 18
        p = _native.plan_for(m, 37888, 3584)
        assert p.path == S and p.split_k == 3
    p = _native.plan_for(2, 4608, 3584, path=S)
    assert (p.rows_per_wave, p.k_waves, p.depth, p.variant) == (32, 2, 2, 1)
    p = _native.plan_for(2, 3584, 18944, path=S)
    assert (p.rows_per_wave, p.k_waves, p.depth, p.split_k) == (16, 4, 2, 36)


@pytest.mark.parametrize("k,n", SHAPES)
def test_tile_plans_cover_k_exactly(L, k, n):
    """Every split-K plan gives each split a whole number of 64-row k-steps
    (variants 6..9, 13, 14, 15: of 128-row groups) and covers K exactly; the tile count fits
    the arrival-counter block.  The hybrids (13, 14) put `full` whole tiles on
    each of the 256 CUs (fewer than a CU holds) and split the leftover tiles,
    at most one piece per CU, with compact partials.  Variant numbers without a
    kernel are refused."""
    for m in (512, 2048):
        for variant in range(1, 17):
            for split in (1, 2, 3, 4, 5, 8):
                try:
                    p = _native.plan_tile(m, n, k, variant, split)
                except _native.AwqNativeError as e:
                    # no such kernel or split, or partials beyond 2^31 bytes (M = 2048, 8 splits)
                    assert e.status in (_native.AWQ_ERR_PATH, _native.AWQ_ERR_TOO_LARGE)
                    continue
                assert variant in (6, 7, 8, 9, 13, 14, 15)
                per = p.rows_per_wave
                assert per % 128 == 0
                assert (split - 1) * per < k <= split * per
                tm = {6: 128, 7: 128, 8: 64, 9: 32, 14: 64}.get(variant, 128)
                tn = 512 if variant == 15 else 256
                assert (p.tile_m, p.tile_n, p.block_threads) == (tm, tn, 512 if variant == 15 else 256)
                tiles = -(-m // tm) * -(-n // tn)
                if variant in (13, 14):
                    full, left = tiles // 256, tiles % 256
                    assert split >= 2 and 1 <= full <= (1 if variant == 13 else 2) and 1 <= left and left * split <= 256
                    assert p.grid == full * 256 + left * split
                    assert p.workspace_bytes == (_native.counter_bytes() + _native.SLOT_BYTES +
                                                 split * left * tm * 256 * 4)
                else:
                    assert p.grid == tiles * split
                if split > 1:
                    assert tiles * 4 <= _native.counter_bytes()


def test_deep_weights_take_the_512_column_tile(L):
    """On deep weights (K >= 8192) at M >= 512, AUTO takes the eight-wave
    512-column tile (variant 15) at the largest split (of whole 128-row
    groups, at most 32) whose grid fits one workgroup per CU, where that grid
    covers at least 7/8 of the 256 CUs; otherwise it keeps the 256-column
    tiles: below M = 512, on shallow weights, where even one split needs more
    than 256 workgroups (M = 8192 on down_proj), and where the best fit leaves
    CUs idle (M = 2760, N = 2896: 132 workgroups at split 1)."""
    for k, n in ((18944, 3584), (8192, 1000), (18944, 3000), (11520, 2896)):
        groups = k // 128
        for m in (256, 511, 512, 768, 1000, 1024, 1536, 2048, 2760, 4096, 8192):
            p = _native.plan_for(m, n, k)
            tiles = -(-m // 128) * -(-n // 512)
            valid = [s for s in range(1, min(groups, 32) + 1) if -(-groups // -(-groups // s)) == s]
            fits = [s for s in valid if tiles * s <= 256]
            if m >= 512 and fits and tiles * max(fits) * 8 >= 256 * 7:
                assert (p.path, p.variant, p.split_k) == (_native.PATH_TILE, 15, max(fits)), (m, k, n)
                assert p.grid == tiles * p.split_k <= 256 and p.block_threads == 512 and p.tile_n == 512
            else:
                assert not (p.path == _native.PATH_TILE and p.variant == 15), (m, k, n)
    for m in (512, 2048, 4096):
        for k, n in ((3584, 37888), (3584, 4608), (3584, 3584)):
            assert _native.plan_for(m, n, k).variant != 15


@pytest.mark.parametrize("m,n,bm,waves", [(16, 4608, 32, 4), (64, 3584, 64, 4), (70, 264, 64, 4), (300, 1032, 128, 4),
                                         (64, 3584, 128, 8), (300, 1032, 128, 8), (70, 2800, 128, 8)])
def test_tile_fragment_partials_layout_agrees(m, n, bm, waves):
    """The layout contract between the tile kernel's fragment-native partial
    stores and the tile reduce kernel (both in csrc/awq_tile.hip), restated
    from each side: the store side addresses lane l's value r of fragment
    (wave, c, f) of a tile, the reduce side addresses the 8-column piece of a
    thread.  Every output of every split must be read from exactly the bytes
    written for it, every written byte of a row below M read once, and no two
    stores may write the same bytes.  Eight-wave tiles (512 columns) write two
    256-column units, waves 4 .. 7 the second, and none where it starts at or
    beyond N (N = 1032 and 2800 end inside a 512-column tile's first half)."""
    split = 3
    rb_n, nt = -(-m // 16), -(-n // 256)
    bn = 64 * waves
    # Store side: (split, tile, wave, f, c, lane, r) -> byte offset, output (row, col).
    store, offsets = {}, []
    for s in range(split):
        for m0 in range(0, m, bm):
            for n0 in range(0, -(-n // bn) * bn, bn):
                for f in range(bm // 16):
                    if m0 + 16 * f >= m:
                        break
                    for w in range(waves):
                        tn = n0 // 256 + (w >> 2)
                        if tn >= nt:
                            continue
                        unit = (s * rb_n + m0 // 16 + f) * nt + tn
                        for c in range(4):
                            for lane in range(64):
                                kb = lane // 16
                                for r in range(4):
                                    row = m0 + 16 * f + lane % 16
                                    col = n0 + 64 * w + 16 * c + 8 * (kb >> 1) + 2 * r + (kb & 1)
                                    off = unit * 16384 + (4 * (w & 3) + c) * 1024 + lane * 16 + 4 * r
                                    store[(s, row, col)] = off
                                    offsets.append(off)
    assert len(set(offsets)) == len(offsets)
    # Reduce side: piece -> its output row and 8 columns, the float4s it reads per split.
    read = {}
    for piece in range(rb_n * nt * 512):
        u, rem = piece >> 9, piece & 511
        wc, j, n16 = rem >> 5, (rem >> 4) & 1, rem & 15
        rb, tn = u // nt, u % nt
        row, col = 16 * rb + n16, 256 * tn + 64 * (wc >> 2) + 16 * (wc & 3) + 8 * j
        if row >= m or col >= n:
            continue
        for s in range(split):
            base = (s * rb_n * nt * 1024 + u * 1024 + 64 * wc + 32 * j + n16) * 16
            for r in range(4):
                read[(s, row, col + 2 * r)] = base + 4 * r
                read[(s, row, col + 2 * r + 1)] = base + 16 * 16 + 4 * r
    live = {k: v for k, v in store.items() if k[1] < m and k[2] < n}
    assert len(read) == split * m * n
    assert live == read
    assert len(set(read.values())) == len(read)
    assert max(store.values()) < split * rb_n * nt * 16384


def test_build_rejects_register_spills():
    """build.py reads hipcc's per-kernel resource remarks and refuses kernels
    that spill registers to scratch memory."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("_awq_build_check",
                                                  os.path.join(ROOT, "qwen2-7b-triton_engine_amd", "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    remarks = ("a.hip:1:1: remark: Function Name: _Z4goodv [-Rpass-analysis=kernel-resource-usage]\n"
               "a.hip:1:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]\n"
               "a.hip:9:1: remark: Function Name: _Z5spillv [-Rpass-analysis=kernel-resource-usage]\n"
               "a.hip:9:1: remark:     ScratchSize [bytes/lane]: 88 [-Rpass-analysis=kernel-resource-usage]\n")
    assert mod._spills(remarks) == [("_Z5spillv", 88)]
    assert "-Rpass-analysis=kernel-resource-usage" in mod.RESOURCE_FLAGS


def test_skinny_and_gemv_plan_rejections():
    with pytest.raises(_native.AwqNativeError) as e:
        _native.plan_gemv(3, 512, 3584, 0, 4)           # GEMV serves M <= 2
    assert e.value.status == _native.AWQ_ERR_PATH
    with pytest.raises(_native.AwqNativeError):
        _native.plan_gemv(1, 512, 3584, 16, 8, variant=2, depth=5)   # depth not an instance
    for variant in (1, 3, 4, 6):                        # no GEMV kernel of that number
        with pytest.raises(_native.AwqNativeError):
            _native.plan_gemv(1, 512, 3584, 16, 8, variant=variant)
    with pytest.raises(_native.AwqNativeError):
        _native.plan_gemv(1, 512, 3584, 16, 4, variant=2, split_k=2)   # k_waves must be 128 / rows
    with pytest.raises(_native.AwqNativeError):
        _native.plan_gemv(1, 512, 3584, 16, 8, variant=2, split_k=9)   # 28 groups: no split of 9 whole chunks
    p = _native.plan_gemv(1, 512, 3584, 16, 8, variant=2, split_k=7)
    assert (p.split_k, p.grid, p.block_threads) == (7, 7, 512)
    p = _native.plan_gemv(1, 3584, 3584, 0, 4, variant=5, split_k=36)
    # 7 strips of 64 packed columns x 36 splits; one 64-bit fixed-point slot per output
    assert (p.grid, p.block_threads, p.workspace_bytes) == (252, 256, _native.counter_bytes() + 3584 * 8)
    with pytest.raises(_native.AwqNativeError):
        _native.plan_skinny(65, 512, 3584, 256, 2)      # skinny serves M <= 64
    with pytest.raises(_native.AwqNativeError):
        _native.plan_skinny(8, 512, 3584, 256, 3)       # k_waves must be 1, 2 or 4
    for variant in (4, 5):                              # no tile kernel of that number
        with pytest.raises(_native.AwqNativeError):
            _native.plan_tile(512, 512, 3584, variant, 1)
    with pytest.raises(_native.AwqNativeError):
        _native.plan_tile(512, 512, 3584, 13, 1)


def test_planned_call_rejects_altered_plan(L):
    """gemm_planned re-derives the plan: a hand-edited field is refused before launch."""
    m, n, k = 512, 3584, 3584
    p = _native.plan_tile(m, n, k, 6, 1)
    p.grid += 1
    buf = np.zeros(1 << 12, dtype=np.uint8)
    ptr = ctypes.c_void_p((buf.ctypes.data + 255) & ~255)
    st = L.awq_w4a16_gemm_planned(ptr, ptr, ptr, ptr, ptr, m, n, k, 128, None, 0, ctypes.byref(p), None)
    assert st == _native.AWQ_ERR_PATH


# ---------------------------------------------------------------------------
# Argument checks of the C ABI (all fail before any device work)
# ---------------------------------------------------------------------------

def _aligned_ptr(buf, align=256, offset=0):
    return ctypes.c_void_p(((buf.ctypes.data + align - 1) & ~(align - 1)) + offset)


def test_c_abi_argument_errors(L):
    buf = np.zeros(1 << 16, dtype=np.uint8)
    a = _aligned_ptr(buf)
    mis = _aligned_ptr(buf, offset=2)
    ws = _aligned_ptr(buf)

    def gemm(x=a, qw=a, qz=a, s=a, out=a, M=4, N=512, K=3584, G=128, ws_=None, ws_bytes=0, path=0):
        return L.awq_w4a16_gemm_ex(x, qw, qz, s, out, M, N, K, G, ws_, ws_bytes, path, None)

    E = _native
    assert gemm(qw=None) == E.AWQ_ERR_NULL_POINTER
    assert gemm(x=None) == E.AWQ_ERR_NULL_POINTER
    assert gemm(N=12) == E.AWQ_ERR_BAD_DIMS
    assert gemm(K=200) == E.AWQ_ERR_BAD_DIMS
    assert gemm(N=0) == E.AWQ_ERR_BAD_DIMS
    assert gemm(M=-1) == E.AWQ_ERR_BAD_DIMS
    assert gemm(G=64, K=3584) == E.AWQ_ERR_GROUP_SIZE
    assert gemm(x=mis) == E.AWQ_ERR_MISALIGNED
    assert gemm(s=mis) == E.AWQ_ERR_MISALIGNED
    assert gemm(qw=ctypes.c_void_p(a.value + 2)) == E.AWQ_ERR_MISALIGNED
    assert gemm(K=1 << 23) == E.AWQ_ERR_TOO_LARGE
    assert gemm(M=(1 << 30) + 1) == E.AWQ_ERR_TOO_LARGE
    assert gemm(N=1 << 21) == E.AWQ_ERR_TOO_LARGE
    assert gemm(path=9) == E.AWQ_ERR_PATH
    assert gemm(path=E.PATH_GEMV, M=3) == E.AWQ_ERR_PATH
    # Split-K shapes need the workspace.
    need = _native.workspace_bytes(1, 37888, 3584)
    assert need > 0
    assert gemm(M=1, N=37888, ws_=None, ws_bytes=0) == E.AWQ_ERR_WORKSPACE
    assert gemm(M=1, N=37888, ws_=ws, ws_bytes=need - 1) == E.AWQ_ERR_WORKSPACE
    assert gemm(M=1, N=37888, ws_=_aligned_ptr(buf, offset=4), ws_bytes=need) == E.AWQ_ERR_MISALIGNED
    # M = 0 is a valid empty product: no launch, x and out may be NULL.
    assert gemm(M=0, x=None, out=None) == E.AWQ_OK
    # dequant checks
    assert L.awq_w4a16_dequant(None, a, a, a, 512, 3584, 128, None) == E.AWQ_ERR_NULL_POINTER
    assert L.awq_w4a16_dequant(a, a, a, mis, 512, 3584, 128, None) == E.AWQ_ERR_MISALIGNED
    assert L.awq_w4a16_dequant(a, a, a, a, 512, 3584, 96, None) == E.AWQ_ERR_GROUP_SIZE


# ---------------------------------------------------------------------------
# Python entry point: argument checks (raise before touching a device)
# ---------------------------------------------------------------------------

def _cpu_operands(m=2, k=256, n=64):
    x = torch.zeros((m, k), dtype=torch.float16)
    qw = torch.zeros((k, n // 8), dtype=torch.int32)
    qz = torch.zeros((k // 128, n // 8), dtype=torch.int32)
    s = torch.zeros((k // 128, n), dtype=torch.float16)
    return x, qw, qz, s


def test_python_entry_rejects_bad_operands():
    from kernels.awq_gemm import awq_gemm_forward

    x, qw, qz, s = _cpu_operands()
    with pytest.raises(ValueError, match="float16"):
        awq_gemm_forward(x.float(), qw, qz, s)
    with pytest.raises(ValueError, match="int32"):
        awq_gemm_forward(x, qw.long(), qz, s)
    with pytest.raises(ValueError, match="group_size"):
        awq_gemm_forward(x, qw, qz, s, group_size=64)
    with pytest.raises(ValueError, match="qweight shape"):
        awq_gemm_forward(x, qw[:128], qz, s)
    with pytest.raises(ValueError, match="K = "):
        awq_gemm_forward(x[:, :200], qw, qz, s)
    with pytest.raises(ValueError, match="scales shape"):
        awq_gemm_forward(x, qw, qz, torch.zeros((3, 64), dtype=torch.float16))
    # Valid operands on the CPU: refused (no CPU fallback exists).
    with pytest.raises(ValueError, match="ROCm device"):
        awq_gemm_forward(x, qw, qz, s)


def test_python_plan_helper():
    from kernels.awq_gemm import plan

    d = plan(1, 37888, 3584)
    assert d["path_name"] == "gemv"
    assert plan(2048, 37888, 3584)["path_name"] == "tile"


# ---------------------------------------------------------------------------
# Roofline arithmetic against the hand-computed table of the Qwen2-7B shapes
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("m,k,n,expect", [
    (1, 3584, 3584, 6_687_744),
    (1, 3584, 512, 961_536),
    (1, 3584, 4608, 8_596_480),
    (1, 3584, 18944, 35_318_784),
    (1, 3584, 37888, 70_630_400),
    (1, 18944, 3584, 35_318_784),
    (8, 18944, 3584, 35_634_176),
    (64, 18944, 3584, 38_157_312),
    (512, 18944, 3584, 58_342_400),
    (2048, 18944, 3584, 127_548_416),
    (2048, 3584, 37888, 240_416_768),
])
def test_algorithmic_bytes(m, k, n, expect):
    assert R.algorithmic_bytes(m, n, k) == expect


def test_bound_and_fraction():
    assert R.bound(1, 37888, 3584) == "hbm"
    assert R.bound(2048, 37888, 3584) == "mfma"
    b, achieved, peak, unit, frac = R.roofline_fraction(2048, 37888, 3584, 442e-6)
    assert (b, unit) == ("mfma", "TFLOP/s")
    assert frac == pytest.approx(0.5, rel=1e-3)
    b, achieved, peak, unit, frac = R.roofline_fraction(1, 37888, 3584, 70_630_400 / 4e12)
    assert (b, unit, peak) == ("hbm", "GB/s", 8000.0)
    assert frac == pytest.approx(0.5)


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in (r.stdout + r.stderr)


def test_fp16_linear_argument_checks(L):
    """awq_fp16_linear rejects bad calls before any launch (no GPU needed)."""
    f = L.awq_fp16_linear
    assert f(None, None, None, 0, 100, 3584, None) == _native.AWQ_OK            # M == 0: no-op
    assert f(None, None, None, 9, 100, 3584, None) == _native.AWQ_ERR_PATH      # decode sizes only
    assert f(None, None, None, 1, 100, 12, None) == _native.AWQ_ERR_BAD_DIMS    # K % 8
    assert f(None, None, None, 1, 0, 3584, None) == _native.AWQ_ERR_BAD_DIMS
    assert f(None, None, None, -1, 100, 3584, None) == _native.AWQ_ERR_BAD_DIMS
    assert f(None, None, None, 1, 100, 8192, None) == _native.AWQ_ERR_TOO_LARGE  # K > 4096
    assert f(None, None, None, 1, 152064, 3584, None) == _native.AWQ_ERR_NULL_POINTER


# ---------------------------------------------------------------------------
# Kernel sources
# ---------------------------------------------------------------------------

def test_no_valu_inline_asm_in_kernels():
    """No inline asm spells a vector ALU instruction.  The compiler inserts
    the wait states between a VALU write and an MFMA that reads the same
    registers (or between an MFMA and a VALU touching its operands) only
    around instructions it generated itself; an asm v_and_or_b32 feeding an
    MFMA has produced wrong output columns.  Scalar instructions and the
    LDS-direct buffer loads (with their own s_nop after the M0 write) stay."""
    csrc = os.path.join(ROOT, "qwen2-7b-triton_engine_amd", "csrc")
    offenders = []
    for name in sorted(os.listdir(csrc)):
        if not name.endswith((".hip", ".h")):
            continue
        text = open(os.path.join(csrc, name)).read()
        for m in re.finditer(r"\basm\s*(?:volatile\s*)?\((.*?)\)\s*;", text, re.S):
            body = "".join(re.findall(r'"((?:[^"\\]|\\.)*)"', m.group(1).split(":")[0]))
            if re.search(r"\bv_[a-z0-9_]+", body):
                offenders.append(f"{name}: {body.strip()[:60]}")
    assert offenders == [], offenders


def test_noalloc_refuses_shapes_beyond_its_scratch(L):
    """awq_w4a16_gemm_noalloc refuses a shape whose decode plan needs more
    workspace than its static scratch with AWQ_ERR_SCRATCH, before touching a
    pointer or the GPU; bad dimensions are refused first, and M = 0 is a
    no-op.  (Its GPU results are checked against awq_w4a16_gemm in the GPU
    tests.)"""
    m, n, k = 16, 262144, 8192
    p = _native.plan_for(m, n, k)
    assert p.path != _native.PATH_TILE and p.workspace_bytes > _native.NOALLOC_SCRATCH_BYTES
    buf = np.zeros(1 << 12, dtype=np.uint8)
    ptr = ctypes.c_void_p((buf.ctypes.data + 255) & ~255)
    assert L.awq_w4a16_gemm_noalloc(ptr, ptr, ptr, ptr, ptr, m, n, k, 128, None) == _native.AWQ_ERR_SCRATCH
    assert "scratch" in _native.error_string(_native.AWQ_ERR_SCRATCH)
    assert L.awq_w4a16_gemm_noalloc(ptr, ptr, ptr, ptr, ptr, 1, 12, 128, 128, None) == _native.AWQ_ERR_BAD_DIMS
    assert L.awq_w4a16_gemm_noalloc(ptr, ptr, ptr, ptr, ptr, 1, 64, 128, 64, None) == _native.AWQ_ERR_GROUP_SIZE
    assert L.awq_w4a16_gemm_noalloc(None, ptr, ptr, ptr, None, 0, 64, 128, 128, None) == _native.AWQ_OK
    # A tile plan past the scratch is lowered, not refused: down_proj at M = 2048 (56 MB of partials).
    big = _native.plan_for(2048, 3584, 18944)
    assert big.path == _native.PATH_TILE and big.workspace_bytes > _native.NOALLOC_SCRATCH_BYTES


def test_greedy_token_is_first_argmax():
    """The harness's graph-safe greedy pick (row maxima, then the best row)
    returns torch.argmax's index: the first largest logit, ties included."""
    sys.path.insert(0, os.path.join(ROOT, "qwen2-7b-triton_engine_amd"))
    from engine.qwen2_decode import _greedy_token

    g = torch.Generator().manual_seed(0)
    for n in (256, 257, 1000, 152064):
        for t in range(12):
            x = torch.randn(n, generator=g).half()
            if t % 3 == 0:
                x[torch.randint(0, n, (3,), generator=g)] = x.max()
            assert int(_greedy_token(x)) == int(torch.argmax(x)), (n, t)


def test_greedy_token_non_finite_logits():
    """NaN and +-inf logits: the pick is torch.argmax's (a NaN counts as the
    largest value, its first occurrence wins; +inf beats every finite logit;
    an all -inf row gives index 0), and it is always inside the vocabulary."""
    sys.path.insert(0, os.path.join(ROOT, "qwen2-7b-triton_engine_amd"))
    from engine.qwen2_decode import _greedy_token

    g = torch.Generator().manual_seed(1)
    for n in (256, 257, 1000, 152064):
        cases = []
        x = torch.randn(n, generator=g).half()
        x[n // 3] = float("nan")
        cases.append(x)
        x = torch.randn(n, generator=g).half()
        x[n - 1] = float("nan")
        x[n // 2] = float("nan")
        cases.append(x)
        x = torch.randn(n, generator=g).half()
        x[n // 5] = float("inf")
        x[n // 4] = float("inf")
        cases.append(x)
        x = torch.randn(n, generator=g).half()
        x[n // 7] = float("inf")
        x[n - 2] = float("nan")
        cases.append(x)
        cases.append(torch.full((n,), float("-inf")).half())
        x = torch.full((n,), float("-inf")).half()
        x[n - 1] = -1.0
        cases.append(x)
        cases.append(torch.full((n,), float("nan")).half())
        for i, x in enumerate(cases):
            got = int(_greedy_token(x))
            assert 0 <= got < n, (n, i, got)
            assert got == int(torch.argmax(x)), (n, i, got, int(torch.argmax(x)))


def test_checked_token_clamps_and_counts():
    """The decode step's token guard: tokens inside the vocabulary pass
    unchanged and leave the flag alone; a token below 0 or at / past the
    vocabulary size is clamped into range and counted in the flag."""
    sys.path.insert(0, os.path.join(ROOT, "qwen2-7b-triton_engine_amd"))
    from engine.qwen2_decode import _checked_token

    bad = torch.zeros(1, dtype=torch.int32)
    for t in (0, 1, 151999, 152063):
        out = _checked_token(torch.tensor([t]), 152064, bad)
        assert int(out) == t and int(bad) == 0
    expected = {-1: 0, -(2**40): 0, 152064: 152063, 152065: 152063, 2**62: 152063}
    for i, (t, want) in enumerate(expected.items()):
        out = _checked_token(torch.tensor([t]), 152064, bad)
        assert int(out) == want and int(bad) == i + 1, (t, int(out), int(bad))


def test_torch_binding_loads_and_checks_operands():
    """The torch binding of the eager entry point loads next to the library,
    was built against the same ABI, and refuses bad operands with the same
    ValueErrors as the Python checks before touching a GPU (here the operands
    are CPU tensors, so even good ones end at the device check)."""
    from kernels.awq_gemm import awq_gemm_forward

    b = _native.binding()
    assert b.abi_version() == _native.ABI_VERSION
    for name in ("awq_gemm_forward", "workspace", "workspace_buffers"):
        assert hasattr(b, name)
    k, n = 256, 64
    x = torch.zeros((2, k), dtype=torch.float16)
    qw = torch.zeros((k, n // 8), dtype=torch.int32)
    qz = torch.zeros((k // 128, n // 8), dtype=torch.int32)
    s = torch.zeros((k // 128, n), dtype=torch.float16)
    cases = [
        ((x.float(), qw, qz, s, 128), "x must be float16"),
        ((x, qw.float(), qz, s, 128), "qweight/qzeros must be int32"),
        ((x, qw, qz, s.float(), 128), "scales must be float16"),
        ((x, qw, qz, s, 64), "group_size 64 is not served"),
        ((x, qw[:, :4], qz, s, 128), "qweight shape"),
        ((x, qw, qz[:1], s, 128), "qzeros shape"),
        ((x[:, :200], qw, qz, s, 128), "must be a positive multiple of group_size"),
        ((x, qw, qz, s[:, :60], 128), "must be a positive multiple of 8"),
        ((x, qw, qz, s, 128), "operands must be on a ROCm device"),
    ]
    for args, msg in cases:
        with pytest.raises(ValueError, match=msg):
            awq_gemm_forward(*args)
