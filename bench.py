#!/usr/bin/env python3
"""Benchmark of the quantized GEMV path on one MI355X.

Headline (BASELINE.json metric, config 1): GF4 decode GEMV, batch 1, W 12288x4096
(bf16 N(0,0.02) packed by the GF4 packer), x fp32 N(0,1).  One "step" is one
GEMV launch over one weight copy; the launches rotate over enough distinct
weight copies (> 600 MB) that every step streams its weights from HBM rather
than the 256 MB Infinity Cache.  Inputs are resident in HBM before timing.

Printed: one JSON line with the driver's contract fields plus
``roofline`` (dominant kernel, from per-launch HIP events on the launch stream)
and ``cpu_baseline`` (the numpy oracle dequant + matvec on the host cores).
Further configs are reported under ``extra``.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gf4_weight(rows: int, k: int, seed: int) -> np.ndarray:
    """Config-1 weights: bf16_RNE(0.02 N(0,1)) packed to GF4 words (uint8 view)."""
    from oracle import gf4 as ogf4
    from oracle import matvec as om

    rng = np.random.default_rng(seed)
    w = om.bf16_round(rng.standard_normal((rows, k), dtype=np.float32) * np.float32(0.02))
    return ogf4.gf4_pack(w).view(np.uint8).reshape(rows, -1)


def time_gemv(weights, x, y, steps: int, warmup: int, torch, runtime, awq=None, residual=False):
    """Time `steps` GEMV launches rotating over `weights` (list of HipWeight).

    The launches are captured once into a hipGraph (one launch per weight copy)
    and the graph is replayed, so the host launch rate does not limit the GPU.
    HIP events bracket the replays on the capture/replay stream.  Returns
    (ms_per_step, kernel_us) where kernel_us is the average per-launch time.
    """
    n = len(weights)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for i in range(n):  # warm-up outside capture (first-touch, code object load)
            runtime.decode_matvec(weights[i], x, y, residual=residual, awq=awq)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(n):
            runtime.decode_matvec(weights[i], x, y, residual=residual, awq=awq)
    reps_w = max(1, warmup // n)
    reps = max(1, steps // n)
    with torch.cuda.stream(stream):
        for _ in range(reps_w):
            graph.replay()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        ev0.record(stream)
        for _ in range(reps):
            graph.replay()
        ev1.record(stream)
    torch.cuda.synchronize()
    total_ms = ev0.elapsed_time(ev1)
    launches = reps * n
    return total_ms / launches, total_ms * 1e3 / launches, launches


def cpu_baseline_gf4(rows: int, k: int, seed: int, reps: int = 5):
    """numpy oracle: GF4 dequant (vectorised) + fp32 W @ x (OpenBLAS), median of reps."""
    from oracle import gf4 as ogf4

    words = gf4_weight(rows, k, seed).view("<u4")
    x = np.random.default_rng(seed + 1).standard_normal(k, dtype=np.float32)
    ogf4.gf4_dequant(words) @ x  # warm-up
    t_dq, t_mv = [], []
    for _ in range(reps):
        t0 = time.perf_counter()
        w = ogf4.gf4_dequant(words)
        t1 = time.perf_counter()
        _ = w @ x
        t2 = time.perf_counter()
        t_dq.append(t1 - t0)
        t_mv.append(t2 - t1)
    return float(np.median(t_dq)), float(np.median(t_mv))


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--copies", type=int, default=32, help="distinct weight copies rotated (>= 24)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; --gpus must be 1"}))
        return 2

    import torch

    from qwowl35_amd import runtime

    rows, k = 12288, 4096
    dev = torch.device("cuda:0")
    log(f"config1: GF4 {rows}x{k} b1, {args.copies} copies")
    raw = torch.from_numpy(gf4_weight(rows, k, seed=1))
    base = runtime.HipWeight.upload(raw, runtime.TYPE_GF4, rows, k, device=dev)
    weights = [base]
    for _ in range(args.copies - 1):
        st = base.storage.clone()
        weights.append(runtime.HipWeight.from_device(st, runtime.TYPE_GF4, rows, k))
    x = torch.from_numpy(np.random.default_rng(2).standard_normal(k, dtype=np.float32)).to(dev)
    y = torch.zeros(rows, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    ms_per_step, kernel_us, launches = time_gemv(weights, x, y, args.steps, args.warmup, torch, runtime)
    algo_bytes = rows * k // 2 + 4 * k + 4 * rows
    value = algo_bytes / (ms_per_step * 1e-3) / 1e9
    achieved = algo_bytes / (kernel_us * 1e-6) / 1e9
    log(f"ms/step {ms_per_step:.5f}  kernel {kernel_us:.3f} us  achieved {achieved:.0f} GB/s")

    cpu = None
    if not args.no_cpu:
        t_dq, t_mv = cpu_baseline_gf4(rows, k, seed=1)
        cores = os.cpu_count() or 1
        cpu = {
            "value": round(algo_bytes / (t_dq + t_mv) / 1e9, 3),
            "unit": "GB/s",
            "cores": cores,
            "kind": "port",
            "sample": f"numpy oracle GF4 dequant ({t_dq * 1e3:.1f} ms) + fp32 W@x ({t_mv * 1e3:.1f} ms), "
                      f"12288x4096 b1, median of 5",
        }
    out = {
        "metric": "GF4 b1 matvec HBM GB/s (12288x4096)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": launches,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "gf4-w/fp32-acc",
        "data": "synthetic",
        "config": {"workload": "gf4_matvec_b1_12288x4096", "rows": rows, "k": k, "batch": 1,
                   "weight_copies": args.copies},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
