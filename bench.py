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


# Kernels each path family launches (a stream-path GEMM whose split-K partials
# are added by a second launch runs awq_splitk_reduce_kernel after the main
# kernel; both count as that GEMM's launch).
FAMILY_KERNELS = {
    "gemv": ("awq_gemv",),
    "skinny": ("awq_skinny",),
    "stream": ("awq_stream", "awq_splitk_reduce"),
    "tile": ("awq_tile", "awq_splitk_reduce"),
}
FAMILY_NAMES = {
    "gemv": "awq_gemv_quad_kernel",
    "skinny": "awq_skinny_kernel",
    "stream": "awq_stream_row_kernel / awq_stream_kernel (+ awq_splitk_reduce_kernel)",
    "tile": "awq_tile_kernel (+ awq_splitk_reduce_kernel)",
}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=90.0,
                    help="seconds of CPU baseline work after which each remaining config gets one timed run")
    ap.add_argument("--no-extras", action="store_true", help="headline only (for profiling runs)")
    ap.add_argument("--no-e2e", action="store_true",
                    help="skip the end-to-end decode extra (its ~230k kernel launches swamp a kernel trace)")
    ap.add_argument("--counter-pass", action="store_true",
                    help="for rocprofv3 --pmc runs: a 64 MiB device copy (calibrates the byte counters), "
                         "then one eager launch of every engine shape at M in {1,4,16}; no timing output")
    args = ap.parse_args()
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

    if args.counter_pass:
        src = torch.randint(-2**31, 2**31 - 1, (16 << 20,), device=dev, dtype=torch.int32)  # 64 MiB
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        for m in DECODE_M:
            for name, k, n in ENGINE_SHAPES:
                awq_gemm_forward(xs[(m, k)], *layers[0][name])
                torch.cuda.synchronize()
        log("counter pass done: copy 67108864 B, then " + ", ".join(
            f"M={m} {name} {kernel_family(_native, m, n, k)}" for m in DECODE_M for name, k, n in ENGINE_SHAPES))
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
                    for m in (1, 4) for name, k, n in ENGINE_SHAPES]
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
                r = time_cpu_baseline(x, qw, qz, sc, reps=3 if m >= 512 else 5, warmup=1, threads=threads,
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
            "sample": "value: layer 0 of the decode sweep at M = 1 and 4 (qkv, o, gate_up, down; 8 of the 336 "
                      "GEMMs of a step) through the torch-CPU restatement of the reference's dequant+matmul "
                      "(test/compare_benchmark.py:72-95), 1 warm-up + median of 5; per_config: the q_proj GEMV, layer 0 of "
                      "the decode sweep, the M = 2048 gate_up and the down M-sweep, the M = 2048 gate_up and the "
                      "down M >= 64 rows timed on 4 / 8 rows of x and projected by FLOP rate",
            "cpu_model": r["cpu_model"],
            "os_cpu_count": r["os_cpu_count"],
            "per_config": rows,
        }

    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
