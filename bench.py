#!/usr/bin/env python3
"""Benchmark of the MI355X W4A16 AWQ GEMM (one GPU).

Headline workload (the decode sweep over Qwen2-7B linear shapes): one step is
every AWQ GEMM of one decode token of a 28-layer Qwen2-7B stack, called as
the reference engine calls them -- fused QKV (3584->4608), o_proj
(3584->3584), fused gate||up (3584->37888), down_proj (18944->3584)
(model/qwen2.py:104,156,183,196) -- at M = 1, 4 and 16 rows: 3 x 28 x 4 =
336 GEMMs over 28 distinct layers of random-init AWQ weights (3.4 GB, far
beyond the 256 MB MALL), captured once into a HIP graph and replayed.
``value`` = algorithmic bytes of the step / step time (GB/s).

Also reported (not part of ``value``): per-GEMM times of every per-layer
shape at M in {1, 4, 16}, the prefill gate||up GEMM at M = 2048 (TFLOP/s), the
down_proj M-sweep, the roofline of the dominant kernel, and the reference's
CPU dequant + matmul timed on a bounded sample of the same workload.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "qwen2-7b-triton_engine_amd")
for _p in (PKG, ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "W4A16 AWQ GEMM: decode HBM GB/s vs peak; prefill TFLOPS vs MFMA peak"
LAYERS = 28
HIDDEN, INTER = 3584, 18944
VOCAB = 152064
ENGINE_SHAPES = (("qkv_proj", HIDDEN, 4608), ("o_proj", HIDDEN, HIDDEN),
                 ("gate_up_proj", HIDDEN, 2 * INTER), ("down_proj", INTER, HIDDEN))
DECODE_M = (1, 4, 16)
# The down_proj M-sweep's HBM-bound points beyond the decode sweep, also in the decode counter pass.
SWEEP_PMC_M = (8, 64)
# Weight bytes every per-shape timing cycles through: 2.5x the 256 MB MALL,
# so that each launch reads its weights from HBM.
MIN_ROTATE_BYTES = 640e6


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_weights(torch, dev, k, n, seed):
    """Random AWQ operands: uniform int4 codes and zeros, scales U[0.002, 0.02]."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    qw = torch.randint(-2**31, 2**31 - 1, (k, n // 8), generator=g, device=dev, dtype=torch.int32)
    qz = torch.randint(-2**31, 2**31 - 1, (k // 128, n // 8), generator=g, device=dev, dtype=torch.int32)
    sc = (torch.rand((k // 128, n), generator=g, device=dev) * 0.018 + 0.002).half()
    return qw, qz, sc


def graph_of(torch, fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    return g


def time_graph(torch, g, reps):
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / reps


def kernel_family(_native, m, n, k):
    return _native.PATH_NAMES[_native.plan_for(m, n, k).path]


def kernel_family_kernel(_native, m, n, k, name):
    """`name` when it is a kernel AUTO's plan for (m, n, k) launches, else None
    (a stale counter profile of another kernel is not attached to a row)."""
    p = _native.plan_for(m, n, k)
    prefixes = FAMILY_KERNELS[_native.PATH_NAMES[p.path]]
    return name if name.startswith(prefixes) else None


# Kernels each path family launches (a GEMM whose split-K partials are added
# by a second launch runs a reduce kernel after the main kernel --
# awq_tile_reduce_kernel after the tile kernel, awq_splitk_reduce_kernel
# after the others; both count as that GEMM's launch).
FAMILY_KERNELS = {
    "gemv": ("awq_gemv",),
    "skinny": ("awq_skinny",),
    "stream": ("awq_stream", "awq_splitk_reduce"),
    "tile": ("awq_tile",),
}
FAMILY_NAMES = {
    "gemv": "awq_gemv_quad_kernel",
    "skinny": "awq_skinny_kernel",
    "stream": "awq_stream_row_kernel / awq_stream_kernel (+ awq_splitk_reduce_kernel)",
    "tile": "awq_tile_kernel (+ awq_tile_reduce_kernel)",
}


PREFILL_M = 2048
# Counters of the prefill pass (one rocprofv3 --pmc run: 6 SQ counters, 1 GRBM).
PREFILL_SQ_COUNTERS = ("SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CU_CYCLES SQ_LDS_IDX_ACTIVE SQ_LDS_BANK_CONFLICT "
                       "SQ_ACTIVE_INST_LDS SQ_INSTS_LDS GRBM_GUI_ACTIVE")
PREFILL_LAUNCHES = 3   # eager launches per shape in the prefill counter pass; the last one is summarised
COPY_BYTES = 64 << 20  # the calibration copy of the counter passes


def calibration_copy(torch, dev):
    """One device-to-device copy of COPY_BYTES (dispatched as the runtime's
    copyBuffer kernel): the byte counters' reading for it scales them."""
    src = torch.randint(-2**31, 2**31 - 1, (COPY_BYTES // 4,), device=dev, dtype=torch.int32)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()


def prefill_counter_pass(torch, dev):
    """The calibration copy, then PREFILL_LAUNCHES eager launches (synchronised
    one by one) of each engine shape at M = 2048 on random operands."""
    from kernels import _native
    from kernels.awq_gemm import awq_gemm_forward

    calibration_copy(torch, dev)
    for j, (name, k, n) in enumerate(ENGINE_SHAPES):
        w = make_weights(torch, dev, k, n, 1000 * 0 + j)
        x = torch.randn((PREFILL_M, k), device=dev).half()
        for _ in range(PREFILL_LAUNCHES):
            awq_gemm_forward(x, *w)
            torch.cuda.synchronize()
        del w, x
    log("prefill counter pass done: copy 67108864 B, then " + ", ".join(
        f"{name} x{PREFILL_LAUNCHES} {kernel_family(_native, PREFILL_M, n, k)}" for name, k, n in ENGINE_SHAPES))


# ---- profile summaries (host only: rocprofv3 CSV -> profiles/) -------------
# Second launches that add split-K partials.
REDUCE_KERNELS = ("awq_splitk_reduce_kernel", "awq_tile_reduce_kernel")


def _short_kernel(name):
    for key in (*REDUCE_KERNELS, "awq_zero_fill_kernel"):
        if key in name:
            return key
    name = name.replace("void awq::", "")
    return name.split("(")[0]


def _counter_csv(d):
    import glob
    hits = sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True))
    if not hits:
        raise SystemExit(f"no *counter_collection.csv under {d}")
    return hits[0]


def _dispatches(path):
    """[(dispatch id, kernel, {counter: value}, duration ns)] in dispatch order."""
    import csv
    per = {}
    for r in csv.DictReader(open(path)):
        d = int(r["Dispatch_Id"])
        e = per.setdefault(d, [r["Kernel_Name"], {}, int(r["End_Timestamp"]) - int(r["Start_Timestamp"])])
        e[1][r["Counter_Name"]] = e[1].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return [(d, per[d][0], per[d][1], per[d][2]) for d in sorted(per)]


def _copy_scale(rows, counter):
    for _, kname, c, _ in rows:
        if "copyBuffer" in kname and counter in c:
            return (COPY_BYTES / 1024) / c[counter], c[counter]
    raise SystemExit(f"no copyBuffer dispatch with {counter}")


def _gemm_groups(rows):
    """AWQ dispatches grouped per GEMM: a main kernel and, when its split-K
    partials are added by a second launch, the reduce kernel that follows
    it."""
    groups = []
    for row in rows:
        k = _short_kernel(row[1])
        if not k.startswith("awq_") or k == "awq_zero_fill_kernel":
            continue
        if k in REDUCE_KERNELS and groups:
            groups[-1].append(row)
        else:
            groups.append([row])
    return groups


def summarize(argv):
    kind, dirs = argv[0], argv[1:]
    from kernels.awq_roofline import HBM_PEAK_BPS, MFMA_F16_DENSE_PEAK_FLOPS, algorithmic_bytes, flops
    prof = os.path.join(ROOT, "profiles")
    cmd_head = 'cd /tmp && export TMPDIR=/tmp && cd "$GRAFT_REPO_ROOT"'
    if kind == "decode-pmc":
        fetch, write = (_dispatches(_counter_csv(d)) for d in dirs[:2])
        fs, fcopy = _copy_scale(fetch, "FETCH_SIZE")
        ws, wcopy = _copy_scale(write, "WRITE_SIZE")
        gf, gw = _gemm_groups(fetch), _gemm_groups(write)
        keys = [(m, name, k, n) for m in DECODE_M for name, k, n in ENGINE_SHAPES]
        keys += [(m, "down_proj", INTER, HIDDEN) for m in SWEEP_PMC_M]
        assert len(gf) == len(gw) == len(keys), (len(gf), len(gw), len(keys))
        launches = []
        for (m, name, k, n), a, b in zip(keys, gf, gw):
            assert [_short_kernel(r[1]) for r in a] == [_short_kernel(r[1]) for r in b]
            for j, (ra, rb) in enumerate(zip(a, b)):
                launches.append({"kernel": _short_kernel(ra[1]), "shape": name, "M": m, "K": k, "N": n,
                                 "fetch_bytes": round(ra[2]["FETCH_SIZE"] * fs * 1024),
                                 "write_bytes": round(rb[2]["WRITE_SIZE"] * ws * 1024),
                                 "algorithmic_bytes": algorithmic_bytes(m, n, k) if j == 0 else 0})
        cmds = [f"timeout -s KILL 120 rocprofv3 --pmc FETCH_SIZE -d {dirs[0]} -o fetch --output-format csv -- "
                "python3 bench.py --counter-pass",
                f"timeout -s KILL 120 rocprofv3 --pmc WRITE_SIZE -d {dirs[1]} -o write --output-format csv -- "
                "python3 bench.py --counter-pass",
                f"python3 bench.py --summarize decode-pmc {dirs[0]} {dirs[1]}"]
        json.dump({"source": "profiles/decode_sweep_pmc_traffic.md", "fetch_scale": fs, "write_scale": ws,
                   "launches": launches}, open(os.path.join(prof, "decode_sweep_pmc_traffic.json"), "w"), indent=1)
        md = ["# Decode sweep: HBM traffic per launch (rocprofv3 PMC FETCH_SIZE / WRITE_SIZE)", "",
              "Commands (two counter passes, then the summary; from the repository root on the MI355X box):", "",
              "```", cmd_head, *cmds, "```", "",
              "`bench.py --counter-pass` makes the operands, runs one 64 MiB device-to-device copy",
              "(`torch.Tensor.copy_`, dispatched as `__amd_rocclr_copyBuffer`), then one eager launch of each",
              "engine shape at M = 1, 4, 16 on layer 0's weights, then down_proj at M = 8 and 64 (the M-sweep's",
              "HBM-bound points) on the same weights (AUTO plans; a GEMM whose split-K partials are",
              "added by a second launch shows two dispatches, the main kernel and its reduce kernel,",
              "`awq_tile_reduce_kernel` after the tile kernel, `awq_splitk_reduce_kernel` after the others).", "",
              "## Calibration with the copy of known size (67,108,864 B read and written)", "",
              "| counter | reads for the copy (KiB) | expected (KiB) | scale factor |", "|---|---|---|---|",
              f"| FETCH_SIZE | {fcopy:.1f} | 65536 | {fs:.4f} |", f"| WRITE_SIZE | {wcopy:.1f} | 65536 | {ws:.4f} |",
              "", "Fetched and written bytes below are the counter times the factor above.", "",
              "## Per launch (scaled; MB = 1e6 bytes)", "",
              "| kernel | shape | M | fetch (MB) | write (MB) | traffic (MB) | algorithmic (MB) | traffic / algorithmic |",
              "|---|---|---|---|---|---|---|---|"]
        gemm_traffic = {}
        for e in launches:
            gemm_traffic[(e["M"], e["shape"])] = gemm_traffic.get((e["M"], e["shape"]), 0) + e["fetch_bytes"] + e["write_bytes"]
        for e in launches:
            t = e["fetch_bytes"] + e["write_bytes"]
            a = e["algorithmic_bytes"]
            shp = f"{e['shape']} {e['K']}->{e['N']}"
            if a:
                tot = gemm_traffic[(e["M"], e["shape"])]
                md.append(f"| `{e['kernel']}` | {shp} | {e['M']} | {e['fetch_bytes']/1e6:.2f} | {e['write_bytes']/1e6:.2f} "
                          f"| {t/1e6:.2f} | {a/1e6:.2f} | {t/a:.2f} (GEMM {tot/a:.2f}) |")
            else:
                md.append(f"| `{e['kernel']}` | {shp} | {e['M']} | {e['fetch_bytes']/1e6:.2f} | {e['write_bytes']/1e6:.2f} "
                          f"| {t/1e6:.2f} | (same GEMM) | |")
        open(os.path.join(prof, "decode_sweep_pmc_traffic.md"), "w").write("\n".join(md) + "\n")
        print(f"decode-pmc: {len(launches)} launches")
    elif kind == "prefill-pmc":
        sq, fetch, write = (_dispatches(_counter_csv(d)) for d in dirs[:3])
        fs, fcopy = _copy_scale(fetch, "FETCH_SIZE")
        ws, wcopy = _copy_scale(write, "WRITE_SIZE")
        gsq, gf, gw = _gemm_groups(sq), _gemm_groups(fetch), _gemm_groups(write)
        want = len(ENGINE_SHAPES) * PREFILL_LAUNCHES
        assert len(gsq) == len(gf) == len(gw) == want, (len(gsq), len(gf), len(gw), want)
        simds = 256 * 4
        rows = []
        for i, (name, k, n) in enumerate(ENGINE_SHAPES):
            last = (i + 1) * PREFILL_LAUNCHES - 1   # the warm launch
            a, b, c = gsq[last], gf[last], gw[last]
            main = a[0]
            cnt = main[2]
            dur_ns = main[3]
            xcds = 8
            clk_cycles = cnt["GRBM_GUI_ACTIVE"] / xcds
            busy = cnt["SQ_VALU_MFMA_BUSY_CYCLES"] / (simds * clk_cycles)
            fetch_b = sum(r[2]["FETCH_SIZE"] for r in b) * fs * 1024
            write_b = sum(r[2]["WRITE_SIZE"] for r in c) * ws * 1024
            f = flops(PREFILL_M, n, k)
            rows.append({
                "shape": name, "M": PREFILL_M, "K": k, "N": n, "kernel": _short_kernel(main[1]),
                "launches": [_short_kernel(r[1]) for r in a],
                "duration_us": round(dur_ns / 1e3, 2),
                "TFLOPs_in_pass": round(f / (dur_ns * 1e-9) / 1e12, 1),
                "mfma_busy": round(busy, 4),
                "clock_GHz": round(clk_cycles / (dur_ns * 1e-9) / 1e9, 3),
                "lds_bank_conflict_per_lds_active": round(cnt["SQ_LDS_BANK_CONFLICT"] / max(cnt["SQ_LDS_IDX_ACTIVE"], 1), 4),
                "counters": {key: cnt[key] for key in sorted(cnt)},
                "fetch_bytes": round(fetch_b), "write_bytes": round(write_b),
                "algorithmic_bytes": algorithmic_bytes(PREFILL_M, n, k),
            })
        cmds = [f"timeout -s KILL 120 rocprofv3 --pmc {PREFILL_SQ_COUNTERS} -d {dirs[0]} -o sq --output-format csv -- "
                "python3 bench.py --counter-pass prefill",
                f"timeout -s KILL 120 rocprofv3 --pmc FETCH_SIZE -d {dirs[1]} -o fetch --output-format csv -- "
                "python3 bench.py --counter-pass prefill",
                f"timeout -s KILL 120 rocprofv3 --pmc WRITE_SIZE -d {dirs[2]} -o write --output-format csv -- "
                "python3 bench.py --counter-pass prefill",
                f"python3 bench.py --summarize prefill-pmc {' '.join(dirs[:3])}"]
        json.dump({"source": "profiles/prefill_tile_pmc.md", "fetch_scale": fs, "write_scale": ws,
                   "simds": simds, "xcds": 8, "rows": rows},
                  open(os.path.join(prof, "prefill_tile_pmc.json"), "w"), indent=1)
        md = ["# Prefill (M = 2048) on the four Qwen2-7B engine shapes: rocprofv3 counters", "",
              "Commands (three counter passes, then the summary; from the repository root on the MI355X box):", "",
              "```", cmd_head, *cmds, "```", "",
              f"`bench.py --counter-pass prefill` runs one 64 MiB device-to-device copy (the byte counters' "
              f"calibration), then {PREFILL_LAUNCHES} eager launches of each engine shape at M = 2048 (AUTO plans, "
              "random operands), synchronised one by one; the last launch of each shape (warm clocks) is the one",
              "summarised.  Counters are summed over the device per dispatch.", "",
              "* MFMA busy = `SQ_VALU_MFMA_BUSY_CYCLES` / (1024 SIMDs x `GRBM_GUI_ACTIVE` / 8 XCDs): the share of",
              "  SIMD cycles with the matrix core busy while the kernel runs.",
              "* Effective clock = (`GRBM_GUI_ACTIVE` / 8) / kernel duration; the dense fp16 peak (2516.6 TFLOP/s)",
              "  assumes 2.4 GHz.",
              "* Durations are the counter run's (serialised dispatches, counters on): the bench's graph-timed",
              "  figures are the throughput numbers.",
              f"* Byte counters scaled by the copy: FETCH_SIZE x {fs:.4f} (read {fcopy:.1f} KiB for 65536), "
              f"WRITE_SIZE x {ws:.4f} (wrote {wcopy:.1f} KiB).", "",
              "| shape | kernels | duration (us) | TFLOP/s in the pass | MFMA busy | clock (GHz) | LDS bank conflicts / LDS active | "
              "fetch (MB) | write (MB) | algorithmic (MB) |", "|---|---|---|---|---|---|---|---|---|---|"]
        for r in rows:
            md.append(f"| {r['shape']} {r['K']}->{r['N']} | {' + '.join('`' + x + '`' for x in r['launches'])} | "
                      f"{r['duration_us']:.1f} | {r['TFLOPs_in_pass']:.0f} | {100 * r['mfma_busy']:.1f} % | "
                      f"{r['clock_GHz']:.2f} | {r['lds_bank_conflict_per_lds_active']:.3f} | {r['fetch_bytes']/1e6:.1f} | "
                      f"{r['write_bytes']/1e6:.1f} | {r['algorithmic_bytes']/1e6:.1f} |")
        md += ["", "## Raw counter values of the summarised dispatch (main kernel)", "",
               "| shape | " + " | ".join(f"`{c}`" for c in PREFILL_SQ_COUNTERS.split()) + " |",
               "|---|" + "---|" * len(PREFILL_SQ_COUNTERS.split())]
        for r in rows:
            md.append(f"| {r['shape']} | " + " | ".join(f"{r['counters'].get(c, float('nan')):.0f}"
                                                      for c in PREFILL_SQ_COUNTERS.split()) + " |")
        open(os.path.join(prof, "prefill_tile_pmc.md"), "w").write("\n".join(md) + "\n")
        print(f"prefill-pmc: {len(rows)} shapes")
    elif kind == "kernel-trace":
        import csv
        import glob
        import statistics
        d = dirs[0]
        stats_path = sorted(glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True))[0]
        trace_path = sorted(glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True))[0]
        out_name = dirs[1] if len(dirs) > 1 else "decode_sweep_kernel_trace.md"
        command = (f"rocprofv3 --kernel-trace --stats -d {d} -o bench --output-format csv -- "
                   "python3 bench.py --no-cpu-baseline --no-extras --steps 5 --warmup 1")
        all_stats = list(csv.DictReader(open(stats_path)))
        tot = sum(float(r["TotalDurationNs"]) for r in all_stats)
        md = [f"# rocprofv3 kernel trace: {out_name.replace('_kernel_trace.md', '').replace('_', ' ')}", "",
              "Commands (from the repository root on the MI355X box):", "", "```", cmd_head, command,
              f"python3 bench.py --summarize kernel-trace {d} {out_name}", "```", "",
              "## Per-kernel statistics (AWQ kernels only)", "",
              "| kernel | calls | average (us) | min (us) | max (us) | share of GPU time |", "|---|---|---|---|---|---|"]
        for r in all_stats:
            if "awq" not in r["Name"]:
                continue
            md.append(f"| `{_short_kernel(r['Name'])}` | {r['Calls']} | {float(r['AverageNs'])/1e3:.2f} | "
                      f"{float(r['MinNs'])/1e3:.2f} | {float(r['MaxNs'])/1e3:.2f} | {100*float(r['TotalDurationNs'])/tot:.1f} % |")
        groups = {}
        for r in csv.DictReader(open(trace_path)):
            if "awq" not in r["Kernel_Name"]:
                continue
            key = (_short_kernel(r["Kernel_Name"]), int(r["Grid_Size_X"]), int(r["Workgroup_Size_X"]))
            groups.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        md += ["", "## Per launch configuration (grid in threads)", "",
               "| kernel | grid | workgroup | launches | median (us) | mean (us) |", "|---|---|---|---|---|---|"]
        for (k, g, w), v in sorted(groups.items()):
            md.append(f"| `{k}` | {g} | {w} | {len(v)} | {statistics.median(v):.2f} | {statistics.mean(v):.2f} |")
        open(os.path.join(prof, out_name), "w").write("\n".join(md) + "\n")
        print(f"kernel-trace: {len(groups)} launch configurations -> profiles/{out_name}")
    elif kind == "prefill-issue":
        _summarize_prefill_issue(dirs[:2], prof, cmd_head)
    elif kind == "prefill-trace":
        _summarize_prefill_trace(dirs[0], prof, cmd_head)
    else:
        raise SystemExit(f"unknown summary kind {kind!r}")


PREFILL_ISSUE_COUNTERS = (
    "SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY SQ_ACTIVE_INST_ANY SQ_ACTIVE_INST_VALU "
    "SQ_ACTIVE_INST_LDS SQ_VALU_MFMA_COEXEC_CYCLES GRBM_GUI_ACTIVE",
    "SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_LDS SQ_WAIT_INST_LDS SQ_VALU_MFMA_BUSY_CYCLES SQ_ACTIVE_INST_SCA "
    "SQ_INSTS_SALU SQ_ACTIVE_INST_VALU2 GRBM_GUI_ACTIVE")


def _summarize_prefill_issue(dirs, prof, cmd_head):
    """profiles/prefill_tile_issue.md: where the SIMD cycles of the prefill tile kernels go, from
    two counter passes of `bench.py --counter-pass prefill` (the warm launch of each shape)."""
    a_runs, b_runs = (_gemm_groups(_dispatches(_counter_csv(d))) for d in dirs)
    want = len(ENGINE_SHAPES) * PREFILL_LAUNCHES
    assert len(a_runs) == len(b_runs) == want, (len(a_runs), len(b_runs), want)
    simds = 256 * 4
    cmds = [f"timeout -s KILL 120 rocprofv3 --pmc {c} -d {d} -o {t} --output-format csv -- "
            "python3 bench.py --counter-pass prefill" for c, d, t in zip(PREFILL_ISSUE_COUNTERS, dirs, "ab")]
    cmds.append(f"python3 bench.py --summarize prefill-issue {' '.join(dirs)}")
    md = ["# Prefill tile kernels (M = 2048): where the SIMD cycles go", "",
          "Commands (two counter passes, then the summary; from the repository root on the MI355X box):", "",
          "```", cmd_head, *cmds, "```", "",
          f"The warm (last of {PREFILL_LAUNCHES}) launch of each engine shape; counters summed over the device.",
          "SIMD cycles = 1024 SIMDs x `GRBM_GUI_ACTIVE` / 8 XCDs.  The SQ per-wave counters are in quad",
          "cycles (x 4 below) and are divided by the waves' own cycles (`SQ_WAVE_CYCLES` x 4).", "",
          "* MFMA busy: `SQ_VALU_MFMA_BUSY_CYCLES` / SIMD cycles (equal to MFMA count x 16 cycles /",
          "  SIMD cycles: the matrix core is busy exactly while its instructions run).",
          "* VALU issue: non-MFMA VALU instructions x 4 cycles / SIMD cycles (a wave64 VALU instruction",
          "  takes 4 cycles); co-executed: `SQ_VALU_MFMA_COEXEC_CYCLES` / SIMD cycles, the cycles in which",
          "  a VALU instruction issued while the matrix core was busy.",
          "* Waves per SIMD: `SQ_WAVE_CYCLES` x 4 / SIMD cycles.", "",
          "| shape | kernel | waves / SIMD | MFMA busy | VALU issue | VALU co-executed | VALU per MFMA | LDS per MFMA "
          "| SALU per MFMA | wave: active | wave: waiting to issue | wave: waiting (deps, barrier) |",
          "|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for i, (name, k, n) in enumerate(ENGINE_SHAPES):
        last = (i + 1) * PREFILL_LAUNCHES - 1
        a, b = a_runs[last][0][2], b_runs[last][0][2]
        cyc = simds * a["GRBM_GUI_ACTIVE"] / 8
        wave = a["SQ_WAVE_CYCLES"] * 4
        mf = b["SQ_INSTS_MFMA"]
        valu = b["SQ_INSTS_VALU"] - mf
        md.append(f"| {name} | `{_short_kernel(a_runs[last][0][1])}` | {wave / cyc:.2f} | "
                  f"{b['SQ_VALU_MFMA_BUSY_CYCLES'] / cyc:.3f} | {valu * 4 / cyc:.3f} | "
                  f"{a['SQ_VALU_MFMA_COEXEC_CYCLES'] / cyc:.3f} | {valu / mf:.2f} | {b['SQ_INSTS_LDS'] / mf:.2f} | "
                  f"{b['SQ_INSTS_SALU'] / mf:.2f} | {a['SQ_ACTIVE_INST_ANY'] * 4 / wave:.3f} | "
                  f"{a['SQ_WAIT_INST_ANY'] * 4 / wave:.3f} | {a['SQ_WAIT_ANY'] * 4 / wave:.3f} |")
    open(os.path.join(prof, "prefill_tile_issue.md"), "w").write("\n".join(md) + "\n")
    print("prefill-issue: 4 shapes -> profiles/prefill_tile_issue.md")


def _plan_kernel_key(_native, m, n, k):
    """(kernel name prefix, workgroups, threads) that AUTO's plan for (m, n, k) launches first."""
    p = _native.plan_for(m, n, k)
    path = _native.PATH_NAMES[p.path]
    if path == "tile":
        fin = 0 if p.variant in (6, 13, 14) else 1
        hy = "true" if p.variant in (13, 14) else "false"
        name = f"awq_tile_kernel<{p.tile_m // 16}, {fin}, {hy}, {p.block_threads // 64}>"
    else:
        name = FAMILY_KERNELS[path][0]
    return name, int(p.grid), int(p.block_threads), p


def _summarize_prefill_trace(d, prof, cmd_head):
    """profiles/prefill_tile_kernel_trace.md and lm_head_gemv_kernel_trace.md from one
    rocprofv3 --kernel-trace run of `bench.py --no-cpu-baseline --no-e2e --steps 1 --warmup 0`.
    Each measurement of the bench (an eager launch, then graph replays) is a run of AWQ launches
    of one kernel and grid; the runs are matched, in the bench's order, to the M = 2048
    engine shapes, the down_proj M-sweep and the lm_head GEMV at M = 1 and 4 by the kernel and
    grid of each one's AUTO plan."""
    import csv
    import glob
    import statistics

    from kernels import _native
    from kernels.awq_roofline import MFMA_F16_DENSE_PEAK_FLOPS, flops
    trace_path = sorted(glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True))[0]
    rows = sorted(csv.DictReader(open(trace_path)), key=lambda r: int(r["Start_Timestamp"]))
    # run: {"key": (name, wgs, threads), "main": [rows], "reduce": [rows]}; a measurement's
    # eager launch and its graph replays are parted by two or three small torch kernels (fills),
    # two measurements by more (operand set-up, or torch's own GEMM timed in between).
    runs, cur, gap = [], None, 0
    for r in rows:
        name = _short_kernel(r["Kernel_Name"])
        if "awq" not in name:
            gap += 1
            if gap > 3:
                cur = None
            continue
        gap = 0
        wgs = int(r["Grid_Size_X"]) // int(r["Workgroup_Size_X"])
        if name in REDUCE_KERNELS:
            if cur is not None:
                cur["reduce"].append(r)
            continue
        key = (name, wgs, int(r["Workgroup_Size_X"]))
        if cur is None or cur["key"] != key:
            cur = {"key": key, "main": [], "reduce": []}
            runs.append(cur)
        cur["main"].append(r)

    def us(r):
        return (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3

    items = [(name, 2048, k, n) for name, k, n in ENGINE_SHAPES]
    items += [("down_proj", m, INTER, HIDDEN) for m in (1, 8, 64, 512, 2048)]
    pos, found = 0, []
    for name, m, k, n in items:
        kname, wgs, threads, p = _plan_kernel_key(_native, m, n, k)
        while pos < len(runs) and not (runs[pos]["key"][0].startswith(kname) and runs[pos]["key"][1:] == (wgs, threads)):
            pos += 1
        if pos == len(runs):
            raise SystemExit(f"no run of {kname} x {wgs} for {name} M={m}")
        found.append((name, m, k, n, p, runs[pos]))
        pos += 1
    lm = []
    for m in (1, 4):
        while pos < len(runs) and "fp16_mfma_kernel" not in runs[pos]["key"][0]:
            pos += 1
        if pos == len(runs):
            raise SystemExit(f"no lm_head run for M={m}")
        lm.append((m, runs[pos]))
        pos += 1

    command = ("rocprofv3 --kernel-trace --stats -d " + d + " -o prefill --output-format csv -- "
               "python3 bench.py --no-cpu-baseline --no-e2e --steps 1 --warmup 0")
    head = ["Commands (from the repository root on the MI355X box):", "", "```", cmd_head, command,
            f"python3 bench.py --summarize prefill-trace {d}", "```", ""]
    md = ["# Prefill tile kernels and the down_proj M-sweep: rocprofv3 kernel trace", ""] + head + [
        "Each row is one measurement of `bench.py` (an eager launch, then HIP-graph replays over",
        ">= 640 MB of distinct random-init weight copies), found in the trace as a run of launches of",
        "the kernel and grid AUTO plans for the shape.  The first replays run while the clocks are",
        "still rising, so the median and the minimum are the figures to read.  Plans with the",
        "reduce-launch finish are followed by one `awq_tile_reduce_kernel` launch each (its median in",
        "the reduce column).  TFLOP/s = 2 M N K / (median launch + median reduce launch); the",
        f"percentage is of the dense fp16 MFMA peak ({MFMA_F16_DENSE_PEAK_FLOPS / 1e12:.1f} TFLOP/s).", "",
        "| GEMM | kernel | variant, split | workgroups x threads | LDS B | VGPR+AGPR / scratch | launches "
        "| avg us | median us | min us | reduce us | TFLOP/s |", "|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for name, m, k, n, p, run in found:
        t = [us(r) for r in run["main"]]
        red = statistics.median([us(r) for r in run["reduce"]]) if run["reduce"] else 0.0
        r0 = run["main"][0]
        med = statistics.median(t)
        tf = flops(m, n, k) / ((med + red) * 1e-6) / 1e12
        md.append(f"| {name} M={m} K={k} N={n} | `{run['key'][0]}` | {p.variant}, {p.split_k} | "
                  f"{run['key'][1]} x {run['key'][2]} | {r0['LDS_Block_Size']} | "
                  f"{r0['VGPR_Count']}+{r0['Accum_VGPR_Count']} / {r0['Scratch_Size']} | {len(t)} | "
                  f"{statistics.mean(t):.1f} | {med:.1f} | {min(t):.1f} | {red:.1f} | "
                  f"{tf:.0f} ({100 * tf * 1e12 / MFMA_F16_DENSE_PEAK_FLOPS:.1f} %) |")
    open(os.path.join(prof, "prefill_tile_kernel_trace.md"), "w").write("\n".join(md) + "\n")

    wbytes = VOCAB * HIDDEN * 2
    md = ["# lm_head fp16 GEMV: rocprofv3 kernel trace", ""] + head + [
        f"`bench.py` times the projection {VOCAB} x {HIDDEN} (fp16 weight, {wbytes / 1e9:.3f} GB) at M = 1 and 4",
        "over three weight copies in HIP graphs (torch's own `F.linear` on the same operands is timed",
        "beside it and does not appear here).  GB/s = weight bytes / median launch.", "",
        "| M | kernel | workgroups x threads | VGPR+AGPR / scratch | launches | avg us | median us | min us | GB/s |",
        "|---|---|---|---|---|---|---|---|---|"]
    for m, run in lm:
        t = [us(r) for r in run["main"]]
        r0 = run["main"][0]
        med = statistics.median(t)
        md.append(f"| {m} | `awq_fp16_mfma_kernel` | {run['key'][1]} x {run['key'][2]} | "
                  f"{r0['VGPR_Count']}+{r0['Accum_VGPR_Count']} / {r0['Scratch_Size']} | {len(t)} | "
                  f"{statistics.mean(t):.1f} | {med:.1f} | {min(t):.1f} | {wbytes / med / 1e3:.0f} |")
    open(os.path.join(prof, "lm_head_gemv_kernel_trace.md"), "w").write("\n".join(md) + "\n")
    print(f"prefill-trace: {len(found)} GEMMs, {len(lm)} lm_head points -> profiles/prefill_tile_kernel_trace.md, "
          "profiles/lm_head_gemv_kernel_trace.md")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=120.0,
                    help="seconds of CPU baseline work after which each remaining config gets one timed run")
    ap.add_argument("--no-extras", action="store_true", help="headline only (for profiling runs)")
    ap.add_argument("--no-e2e", action="store_true",
                    help="skip the end-to-end decode extra (its ~230k kernel launches swamp a kernel trace)")
    ap.add_argument("--counter-pass", nargs="?", const="decode", choices=("decode", "prefill"),
                    help="for rocprofv3 --pmc runs: a 64 MiB device copy (calibrates the byte counters), then "
                         "'decode' (default): one eager launch of every engine shape at M in {1,4,16}; "
                         "'prefill': three eager launches of every engine shape at M = 2048 (the third, on warm "
                         "clocks, is the one summarised); no timing output")
    ap.add_argument("--summarize", nargs="+", metavar=("KIND", "DIR"),
                    help="host only: turn rocprofv3 CSV output into the profiles/ summaries. "
                         "'decode-pmc FETCH_DIR WRITE_DIR', 'prefill-pmc SQ_DIR FETCH_DIR WRITE_DIR' "
                         "(directories of --counter-pass runs), 'kernel-trace DIR' (a --kernel-trace --stats run of the "
                         "headline), 'prefill-trace DIR' (one of --no-cpu-baseline --no-e2e --steps 1 --warmup 0) or "
                         "'prefill-issue A_DIR B_DIR' (the two issue-counter passes of --counter-pass prefill)")
    args = ap.parse_args()
    if args.summarize:
        summarize(args.summarize)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "this build has no multi-GPU path", file=sys.stderr)
        sys.exit(2)

    import torch

    from kernels import _native
    from kernels.awq_gemm import awq_gemm_forward
    from kernels.awq_roofline import (HBM_PEAK_BPS, MFMA_F16_DENSE_PEAK_FLOPS, QWEN2_7B_LINEARS,
                                      algorithmic_bytes, flops)

    dev = torch.device("cuda:0")
    props = torch.cuda.get_device_properties(0)
    log(f"device {props.name} CUs={props.multi_processor_count}")

    if args.counter_pass == "prefill":
        prefill_counter_pass(torch, dev)
        return

    # ---- synthetic operands: 28 layers x 4 fused projections ---------------
    t0 = time.time()
    layers = []
    for li in range(LAYERS):
        layers.append({name: make_weights(torch, dev, k, n, 1000 * li + j)
                       for j, (name, k, n) in enumerate(ENGINE_SHAPES)})
    gx = torch.Generator(device=dev)
    gx.manual_seed(7)
    xs = {(m, k): torch.randn((m, k), generator=gx, device=dev).half() for m in DECODE_M for k in (HIDDEN, INTER)}
    torch.cuda.synchronize()
    log(f"operands ready in {time.time() - t0:.1f}s")

    def step():
        outs = []
        for m in DECODE_M:
            for li in range(LAYERS):
                for name, k, n in ENGINE_SHAPES:
                    outs.append(awq_gemm_forward(xs[(m, k)], *layers[li][name]))
        return outs

    if args.counter_pass == "decode":
        src = torch.randint(-2**31, 2**31 - 1, (16 << 20,), device=dev, dtype=torch.int32)  # 64 MiB
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        for m in DECODE_M:
            for name, k, n in ENGINE_SHAPES:
                awq_gemm_forward(xs[(m, k)], *layers[0][name])
                torch.cuda.synchronize()
        for m in SWEEP_PMC_M:
            awq_gemm_forward(torch.randn((m, INTER), generator=gx, device=dev).half(), *layers[0]["down_proj"])
            torch.cuda.synchronize()
        log("counter pass done: copy 67108864 B, then " + ", ".join(
            [f"M={m} {name} {kernel_family(_native, m, n, k)}" for m in DECODE_M for name, k, n in ENGINE_SHAPES] +
            [f"M={m} down_proj {kernel_family(_native, m, HIDDEN, INTER)}" for m in SWEEP_PMC_M]))
        return

    step()  # eager: sizes the shared workspace before capture
    torch.cuda.synchronize()
    g = graph_of(torch, step)
    step_bytes = sum(algorithmic_bytes(m, n, k) for m in DECODE_M for _ in range(LAYERS)
                     for _, k, n in ENGINE_SHAPES)
    step_flops = sum(flops(m, n, k) for m in DECODE_M for _ in range(LAYERS) for _, k, n in ENGINE_SHAPES)

    # ---- timed region: exactly `steps` steps ------------------------------
    for _ in range(args.warmup):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    t_step = e0.elapsed_time(e1) / 1e3 / args.steps
    value = step_bytes / t_step / 1e9
    log(f"decode step: {t_step * 1e3:.3f} ms, {value:.1f} GB/s ({value / (HBM_PEAK_BPS / 1e9):.3f} of HBM peak)")
    del g

    # The same step as eager calls, the way the reference engine issues them (no graph):
    # wall time of `steps` steps after `warmup` eager ones, synchronised on both sides.
    for _ in range(max(1, args.warmup)):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t_eager = (time.perf_counter() - t0) / args.steps
    log(f"decode step, eager calls: {t_eager * 1e3:.3f} ms, {step_bytes / t_eager / 1e9:.1f} GB/s")

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_step * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 activations x int4 weights, fp32 accumulate",
        "data": "synthetic: random-init AWQ int4 weights (uniform codes/zeros, scales U[0.002,0.02]), x~N(0,1)",
        "config": {
            "workload": "Qwen2-7B decode sweep: 28 layers x {qkv 3584->4608, o 3584->3584, gate_up 3584->37888, "
                        "down 18944->3584} x M in {1,4,16}, one HIP graph per step",
            "layers": LAYERS, "M": list(DECODE_M), "group_size": 128,
            "gemms_per_step": len(DECODE_M) * LAYERS * len(ENGINE_SHAPES),
            "bytes_per_step": step_bytes, "flops_per_step": step_flops,
        },
        "roofline": None,
        "cpu_baseline": None,
        "eager_step": {"ms_per_step": round(t_eager * 1e3, 4), "GBps": round(step_bytes / t_eager / 1e9, 2),
                       "note": "the same 336 GEMMs as awq_gemm_forward calls issued eagerly (the reference "
                               "engine's usage), wall time per step"},
    }

    # ---- per-GEMM times: each (M, shape) over >= 640 MB of weights in one graph
    def rotation(k, n, base=(), seed=90000):
        need = max(len(base), 2, math.ceil(MIN_ROTATE_BYTES / (k * n // 2)))
        ws = list(base)
        while len(ws) < need:
            ws.append(make_weights(torch, dev, k, n, seed + len(ws)))
        return ws

    def per_launch(m, k, n, weights):
        x = xs[(m, k)] if (m, k) in xs else torch.randn((m, k), device=dev).half()
        awq_gemm_forward(x, *weights[0])
        torch.cuda.synchronize()
        gg = graph_of(torch, lambda: [awq_gemm_forward(x, *w) for w in weights])
        for _ in range(3):  # warm replays: clocks settle before the timed ones
            gg.replay()
        t = min(time_graph(torch, gg, 3) for _ in range(3)) / len(weights)
        del gg
        return t

    per_gemm = []
    family_time, family_bytes, family_launches = {}, {}, {}
    rot = {name: rotation(k, n, [layers[li][name] for li in range(LAYERS)], seed=90000 + 1000 * j)
           for j, (name, k, n) in enumerate(ENGINE_SHAPES)}
    for m in DECODE_M:
        for name, k, n in ENGINE_SHAPES:
            t = per_launch(m, k, n, rot[name])
            b = algorithmic_bytes(m, n, k)
            fam = kernel_family(_native, m, n, k)
            log(f"{name} M={m}: {t * 1e6:.2f} us ({fam}, {len(rot[name])} weight copies)")
            per_gemm.append({"shape": name, "M": m, "K": k, "N": n, "us": round(t * 1e6, 2), "kernel": fam,
                             "GBps": round(b / t / 1e9, 1), "hbm_frac": round(b / t / HBM_PEAK_BPS, 3)})
            family_time[fam] = family_time.get(fam, 0.0) + t * LAYERS
            family_bytes[fam] = family_bytes.get(fam, 0) + b * LAYERS
            family_launches[fam] = family_launches.get(fam, 0) + LAYERS
    # Eager calls, as the reference engine makes them (112 awq_gemm_forward calls per token,
    # model/qwen2.py:44,104,183, never graph-replayed, inference/engine.py:114-139): the wall time
    # per call of EAGER_CALLS back-to-back calls over the 28 layers' weights (host work and kernels
    # overlap; a loop bound by the host shows eager_us above the graph-timed us), and the host
    # time to issue one call (Python entry, checks, plan lookup, ctypes, launch).
    EAGER_CALLS = 3 * LAYERS
    for row in per_gemm:
        m, k, n, name = row["M"], row["K"], row["N"], row["shape"]
        x = xs[(m, k)]
        ws = [layers[li][name] for li in range(LAYERS)]
        for w in ws[:4]:
            awq_gemm_forward(x, *w)
        torch.cuda.synchronize()
        best_wall, best_host = float("inf"), float("inf")
        for _ in range(3):
            t0 = time.perf_counter()
            for i in range(EAGER_CALLS):
                awq_gemm_forward(x, *ws[i % LAYERS])
            t1 = time.perf_counter()
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            best_wall = min(best_wall, (t2 - t0) / EAGER_CALLS)
            best_host = min(best_host, (t1 - t0) / EAGER_CALLS)
        row["eager_us"] = round(best_wall * 1e6, 2)
        row["eager_host_us"] = round(best_host * 1e6, 2)
        log(f"{name} M={m}: eager {row['eager_us']} us per call (host {row['eager_host_us']} us), "
            f"graph {row['us']} us")

    dom = max(family_time, key=family_time.get)
    avg_t = family_time[dom] / family_launches[dom]
    avg_b = family_bytes[dom] / family_launches[dom]
    achieved = avg_b / avg_t / 1e9
    # HBM bytes per launch of the dominant kernel: rocprofv3 FETCH_SIZE + WRITE_SIZE of one launch
    # per (M, shape), each scaled by the counter's reading for a copy of known size (the committed
    # profile that bench.py --counter-pass feeds), averaged over the same launches as `achieved`.
    traffic = None
    traffic_path = os.path.join(ROOT, "profiles", "decode_sweep_pmc_traffic.json")
    if os.path.exists(traffic_path):
        with open(traffic_path) as f:
            pmc = json.load(f)
        prefixes = FAMILY_KERNELS[dom]
        keys = [(m, name) for m in DECODE_M for name, k, n in ENGINE_SHAPES if kernel_family(_native, m, n, k) == dom]
        hits = {}
        for e in pmc["launches"]:
            if e["kernel"].startswith(prefixes):
                key = (e["M"], e["shape"])
                hits[key] = hits.get(key, 0) + e["fetch_bytes"] + e["write_bytes"]
        if keys and all(key in hits for key in keys):
            traffic = round(sum(hits[key] for key in keys) / len(keys))
    result["roofline"] = {
        "bound": "hbm",
        "kernel": FAMILY_NAMES[dom],
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_BPS / 1e9,
        "unit": "GB/s",
        "frac": round(achieved / (HBM_PEAK_BPS / 1e9), 4),
        "traffic": traffic,
        "traffic_source": "profiles/decode_sweep_pmc_traffic.md" if traffic is not None else None,
        "bytes_per_launch": round(avg_b),
        "avg_launch_us": round(avg_t * 1e6, 3),
        "launches_per_step": family_launches[dom],
        "share_of_step_time": round(family_time[dom] / sum(family_time.values()), 3),
    }
    result["per_gemm_engine_shapes"] = per_gemm

    if not args.no_extras:
        # unfused per-layer shapes of the decode sweep (q/k/v/o, gate/up, down)
        sweep = []
        for name, k, n in QWEN2_7B_LINEARS:
            if name in ("v_proj", "up_proj", "o_proj"):
                continue  # same shape as k_proj / gate_proj / q_proj
            ws = rotation(k, n, seed=50000)
            for m in DECODE_M:
                t = per_launch(m, k, n, ws)
                log(f"unfused {name} M={m}: {t * 1e6:.2f} us ({len(ws)} weight copies)")
                b = algorithmic_bytes(m, n, k)
                sweep.append({"shape": name, "M": m, "K": k, "N": n, "us": round(t * 1e6, 2),
                              "kernel": kernel_family(_native, m, n, k),
                              "GBps": round(b / t / 1e9, 1), "hbm_frac": round(b / t / HBM_PEAK_BPS, 3)})
            del ws
        result["per_gemm_unfused_shapes"] = sweep

        # prefill at M = 2048 on the four engine shapes, and the down_proj M-sweep
        def mfma_point(m, k, n, weights, name=None):
            t = per_launch(m, k, n, weights)
            f = flops(m, n, k)
            b = algorithmic_bytes(m, n, k)
            log(f"{name or 'down_proj'} M={m}: {t * 1e6:.2f} us, {f / t / 1e12:.1f} TFLOP/s")
            row = {"shape": name} if name else {}
            row.update({"M": m, "K": k, "N": n, "us": round(t * 1e6, 2), "kernel": kernel_family(_native, m, n, k),
                        "TFLOPs": round(f / t / 1e12, 1), "mfma_frac": round(f / t / MFMA_F16_DENSE_PEAK_FLOPS, 4),
                        "GBps": round(b / t / 1e9, 1), "hbm_frac": round(b / t / HBM_PEAK_BPS, 3)})
            return row

        result["prefill_m2048"] = [mfma_point(2048, k, n, rot[name], name) for name, k, n in ENGINE_SHAPES]
        # MFMA utilisation and effective clock of each shape's kernel, from the committed counter
        # profile (bench.py --counter-pass prefill under rocprofv3 --pmc), the way the decode
        # roofline carries its traffic.
        pmc_path = os.path.join(ROOT, "profiles", "prefill_tile_pmc.json")
        if os.path.exists(pmc_path):
            with open(pmc_path) as f:
                pmc_rows = {r["shape"]: r for r in json.load(f)["rows"]}
            for row in result["prefill_m2048"]:
                r = pmc_rows.get(row["shape"])
                if r is not None and r["kernel"] == kernel_family_kernel(_native, 2048, row["N"], row["K"], r["kernel"]):
                    row["mfma_busy"] = r["mfma_busy"]
                    row["clock_GHz"] = r["clock_GHz"]
                    row["counters_source"] = "profiles/prefill_tile_pmc.md"
        result["prefill_gate_up"] = next(r for r in result["prefill_m2048"] if r["shape"] == "gate_up_proj")

        # The same shapes on torch's dense fp16 GEMM (hipBLASLt; F.linear with an [N, K] fp16
        # weight, no dequantisation at all), timed the same way over >= 640 MB of weights: the
        # library's own MFMA efficiency on this chip, next to the fused int4 kernels'.
        import torch.nn.functional as F

        for row in result["prefill_m2048"]:
            k, n = row["K"], row["N"]
            copies = max(2, math.ceil(MIN_ROTATE_BYTES / (k * n * 2)))
            dense = [(torch.randn((n, k), device=dev) * 0.02).half() for _ in range(copies)]
            xp = torch.randn((2048, k), device=dev).half()
            F.linear(xp, dense[0])
            torch.cuda.synchronize()
            gg = graph_of(torch, lambda: [F.linear(xp, w) for w in dense])
            for _ in range(3):
                gg.replay()
            t = min(time_graph(torch, gg, 3) for _ in range(3)) / copies
            del gg, dense
            torch.cuda.empty_cache()
            f = flops(2048, n, k)
            row["library_fp16_us"] = round(t * 1e6, 2)
            row["library_fp16_mfma_frac"] = round(f / t / MFMA_F16_DENSE_PEAK_FLOPS, 4)
            log(f"{row['shape']} M=2048 dense fp16 F.linear: {t * 1e6:.2f} us, {f / t / 1e12:.1f} TFLOP/s")
        result["down_m_sweep"] = [mfma_point(m, INTER, HIDDEN, rot["down_proj"])
                                  for m in (1, 8, 64, 512, 2048)]

        # fp16 lm_head GEMV (vocab x hidden, 1.09 GB per token), next to torch's own F.linear
        from kernels.lm_head import lm_head_forward
        import torch.nn.functional as F

        lm_ws = [(torch.randn((VOCAB, HIDDEN), device=dev) * 0.02).half() for _ in range(3)]
        lm_bytes = VOCAB * HIDDEN * 2
        lm = []
        for m in (1, 4):
            xl = torch.randn((m, HIDDEN), device=dev).half()
            row = {"M": m, "K": HIDDEN, "N": VOCAB}
            for key, fn in (("us", lambda w: lm_head_forward(xl, w)), ("torch_linear_us", lambda w: F.linear(xl, w))):
                fn(lm_ws[0])
                g = graph_of(torch, lambda: [fn(w) for w in lm_ws])
                g.replay()
                t = min(time_graph(torch, g, 5) for _ in range(3)) / len(lm_ws)
                row[key] = round(t * 1e6, 2)
                del g
            log(f"lm_head M={m}: {row['us']} us (torch F.linear {row['torch_linear_us']} us)")
            row["GBps"] = round(lm_bytes / (row["us"] * 1e-6) / 1e9, 1)
            row["hbm_frac"] = round(lm_bytes / (row["us"] * 1e-6) / HBM_PEAK_BPS, 3)
            lm.append(row)
        result["lm_head_fp16_gemv"] = lm
        del lm_ws

    if not args.no_extras and not args.no_e2e:
        # end-to-end Qwen2-7B-shaped greedy decoding (28 layers, random-init AWQ weights,
        # 1024-token random prompt, 128 new tokens; torch for the non-GEMM ops)
        from engine.qwen2_decode import QWEN2_7B, Qwen2AwqDecoder

        torch.cuda.empty_cache()
        e2e = Qwen2AwqDecoder(QWEN2_7B, max_seq_len=1024 + 128, seed=0, device=dev)
        prompt = torch.randint(0, QWEN2_7B.vocab_size, (1024,), generator=torch.Generator().manual_seed(1))
        log("e2e decode: capture + warm-up")
        e2e.generate(prompt, 128)                      # capture + warm-up
        r = e2e.generate(prompt, 128)
        log(f"e2e decode: {r['decode_tokens_per_s']:.1f} tokens/s")
        result["e2e_decode"] = {
            "layers": QWEN2_7B.num_layers, "prompt_tokens": 1024, "new_tokens": 128,
            "prefill_ms": round(r["prefill_s"] * 1e3, 2),
            "decode_ms_per_token": round(r["decode_s"] / 127 * 1e3, 3),
            "decode_tokens_per_s": round(r["decode_tokens_per_s"], 1),
            "note": "greedy, batch 1, one HIP graph replay per token; AWQ linears and lm_head on this "
                    "build's kernels, the other ops torch",
        }
        del e2e
        torch.cuda.empty_cache()

    # ---- CPU baseline: the reference's dequant + matmul on the host --------
    # Configs 0-3 on a bounded sample: torch-CPU fp16 matmul runs at about
    # 1-2 GFLOP/s on this host (no native fp16 GEMM), so a config whose full
    # size would take minutes is timed on its first `rows` rows of x (the
    # matmul, which dominates, is linear in the rows) and its full-size time
    # is projected from the sample's FLOP rate.  1 warm-up + median of 5 timed
    # runs (3 for samples of the M >= 512 configs), all host threads.
    if not args.no_cpu_baseline:
        from oracle.cpu_baseline import time_cpu_baseline  # reported baseline, not the product

        threads = min(16, os.cpu_count() or 1)
        gen = torch.Generator(device=dev)
        gen.manual_seed(11)
        # (config, shape, full M, sampled rows, K, N, weights)
        samples = [("0: q_proj GEMV (a 3584 x 3584 weight)", "q_proj", 1, 1, HIDDEN, HIDDEN, layers[0]["o_proj"])]
        samples += [("1: decode sweep, layer 0", name, m, m, k, n, layers[0][name])
                    for m in DECODE_M for name, k, n in ENGINE_SHAPES]
        samples += [("2: prefill gate_up", "gate_up_proj", 2048, 4, HIDDEN, 2 * INTER, layers[0]["gate_up_proj"])]
        samples += [("3: down_proj M-sweep", "down_proj", m, min(m, 8), INTER, HIDDEN, layers[0]["down_proj"])
                    for m in (1, 8, 64, 512, 2048)]
        rows, r, spent, cache = [], None, 0.0, {}
        for cfg, name, m, ms, k, n, w in samples:
            if (name, ms, k, n) in cache:            # the same sampled computation as an earlier row
                r = cache[(name, ms, k, n)]
            else:
                qw, qz, sc = (t.cpu() for t in w)
                x = torch.randn((ms, k), generator=gen, device=dev).half().cpu()
                t0 = time.perf_counter()
                r = time_cpu_baseline(x, qw, qz, sc, reps=3 if m >= 16 else 5, warmup=1, threads=threads,
                                      budget_s=max(1e-3, args.cpu_budget - spent))
                spent += time.perf_counter() - t0
                cache[(name, ms, k, n)] = r
            rate = flops(ms, n, k) / r["median_s"]
            full_s = r["median_s"] if ms == m else flops(m, n, k) / rate
            log(f"cpu baseline {cfg} {name} M={m} ({ms} rows timed): median {r['median_s']:.4f} s of {r['reps']}"
                f", full size {full_s:.3f} s")
            rows.append({"config": cfg, "shape": name, "M": m, "K": k, "N": n, "rows_timed": ms,
                         "median_s": round(r["median_s"], 5), "reps": r["reps"],
                         "full_size_s": round(full_s, 4) if ms == m else round(full_s, 2),
                         "projected": ms != m,
                         "GBps": round(algorithmic_bytes(m, n, k) / full_s / 1e9, 4),
                         "TFLOPs": round(flops(m, n, k) / full_s / 1e12, 6)})
        sweep = [row for row in rows if row["config"].startswith("1:")]
        sweep_b = sum(algorithmic_bytes(row["M"], row["N"], row["K"]) for row in sweep)
        sweep_t = sum(row["median_s"] for row in sweep)
        result["cpu_baseline"] = {
            "value": round(sweep_b / sweep_t / 1e9, 4),
            "unit": "GB/s",
            "cores": r["threads"],
            "kind": "port",
            "sample": "value: layer 0 of the decode sweep at M = 1, 4 and 16 (qkv, o, gate_up, down; 12 of the "
                      "336 GEMMs of a step, the same mix of shapes and M as the headline) through the torch-CPU "
                      "restatement of the reference's dequant+matmul (test/compare_benchmark.py:72-95), 1 warm-up "
                      "+ median of 5 (3 at M = 16); per_config: the q_proj GEMV, layer 0 of the decode sweep, the "
                      "M = 2048 gate_up and the down M-sweep, the M = 2048 gate_up and the down M >= 64 rows timed "
                      "on 4 / 8 rows of x and projected by FLOP rate",
            "cpu_model": r["cpu_model"],
            "os_cpu_count": r["os_cpu_count"],
            "per_config": rows,
        }

    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
