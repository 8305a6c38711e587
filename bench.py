#!/usr/bin/env python3
"""Benchmark of the quantized GEMV path on one MI355X.

Headline (BASELINE.json metric, config 1): GF4 decode GEMV, batch 1, W 12288x4096
= GF4 pack of bf16(0.02 N(0,1)), x fp32 N(0,1).  One "step" is one GEMV launch
over one weight copy; the launches rotate over 32 distinct weight copies
(805 MB > the 256 MB Infinity Cache) so every step streams its weights from HBM.
Weights and activations are made on the GPU (torch's seeded generator, the
library's own GF4 / q8_0 / Q4_K encoders) and are resident before timing.

Launches are captured into a hipGraph and replayed; HIP events on the replay
stream bracket the timed replays.  Printed: one JSON line with the driver's
contract fields plus ``roofline`` (dominant kernel) and ``cpu_baseline`` (the
numpy oracle GF4 dequant + matvec on this host's cores), and under ``extra``
the other configs: GF4 batches 2..8 and the transposed shape, the q8_0 layer
set (config 2), the Q4_K down / LM-head GEMVs at batch 1 and 8 (config 3), the
GF4 prefill matmul with its MFMA utilisation (config 4) and the 32-layer 9B
decode-step projection stack replayed as one recorded plan (config 5).
``--gpus`` above 1 is refused: this build measures one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gf4_gemv_b1_12288x4096_traffic.md")


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Bench:
    def __init__(self, torch, runtime, seed: int = 1):
        self.torch = torch
        self.rt = runtime
        self.dev = torch.device("cuda:0")
        self.gen = torch.Generator(device=self.dev)
        self.gen.manual_seed(seed)
        self.stream = torch.cuda.Stream()

    def normal(self, shape, std=1.0, bf16=False):
        t = self.torch.randn(shape, generator=self.gen, device=self.dev, dtype=self.torch.float32)
        if std != 1.0:
            t.mul_(std)
        if bf16:
            t = t.to(self.torch.bfloat16).to(self.torch.float32)
        return t

    def weight(self, type_id, rows, k, std=0.02, tile_rows=None):
        """Encoded N(0, std) weight.  tile_rows: encode that many distinct rows and
        repeat them (the LM head, whose 1.0e9 fp32 source would not be worth making)."""
        if tile_rows is None or tile_rows >= rows:
            src = self.normal((rows, k), std, bf16=(type_id == self.rt.TYPE_GF4))
            hw = self.rt.quantize_weight(src, type_id)
            del src
            return hw
        src = self.normal((tile_rows, k), std)
        part = self.rt.quantize(src, type_id)
        rb = self.rt.row_bytes(type_id, k)
        full = self.torch.empty(rows * rb, dtype=self.torch.uint8, device=self.dev)
        for r0 in range(0, rows, tile_rows):
            n = min(tile_rows, rows - r0)
            full[r0 * rb:(r0 + n) * rb].copy_(part[:n * rb])
        return self.rt.HipWeight.from_device(full, type_id, rows, k)

    def time_calls(self, calls, steps: int, warmup: int):
        """Graph-capture ``calls`` (one launch each) and replay; returns
        (ms per launch, ms per graph, launches timed)."""
        torch = self.torch
        n = len(calls)
        with torch.cuda.stream(self.stream):
            for c in calls:  # first-touch and code-object load outside the capture
                c(self.stream)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=self.stream):
            for c in calls:
                c(self.stream)
        reps_w = max(1, warmup // n)
        reps = max(1, steps // n)
        with torch.cuda.stream(self.stream):
            for _ in range(reps_w):
                graph.replay()
        torch.cuda.synchronize()
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(self.stream):  # replays and events on the same stream
            ev0.record(self.stream)
            for _ in range(reps):
                graph.replay()
            ev1.record(self.stream)
        torch.cuda.synchronize()
        total = ev0.elapsed_time(ev1)
        return total / (reps * n), total / reps, reps * n


def gemv_calls(rt, weights, x, y):
    return [lambda s, w=w: rt.decode_matvec(w, x, y, stream=s) for w in weights]


def gemv_bytes(type_id, rows, k, nb, rt):
    return rows * rt.row_bytes(type_id, k) + 4 * nb * (k + rows)


def read_traffic(kernel_hint: str):
    """HBM bytes per launch from the committed PMC summary, if it names this kernel."""
    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None, None
    m = re.search(r"traffic_bytes_per_launch:\s*(\d+)", text)
    k = re.search(r"kernel:\s*`([^`]+)`", text)
    if not m or not k or kernel_hint not in k.group(1):
        return None, None
    return int(m.group(1)), k.group(1)


def stream_ceiling(b: Bench, rt, torch, bufs) -> dict:
    """Streaming-read ceiling on the same box: the library's read probe over the
    same rotated 25 MB buffers (launch and ramp included, like the GEMV) and
    over one 1 GiB buffer."""
    sinks = [torch.empty(rt.stream_read(bufs[0]).numel(), dtype=torch.int32, device=b.dev) for _ in bufs]
    calls = [lambda s, t=t, k=k: rt.stream_read(t, k, stream=s) for t, k in zip(bufs, sinks)]
    ms, _, _ = b.time_calls(calls, 2000, 200)
    big = torch.zeros(1 << 30, dtype=torch.uint8, device=b.dev)
    sink_big = rt.stream_read(big)
    ms_big, _, _ = b.time_calls([lambda s: rt.stream_read(big, sink_big, stream=s)], 40, 5)
    n = bufs[0].numel()
    tiny = torch.zeros(16, dtype=torch.uint8, device=b.dev)
    sink_tiny = rt.stream_read(tiny)
    ms_tiny, _, _ = b.time_calls([lambda s: rt.stream_read(tiny, sink_tiny, stream=s)] * 32, 2000, 200)
    return {"GB/s_25MB": round(n / (ms * 1e-3) / 1e9, 1), "us_25MB": round(ms * 1e3, 3),
            "GB/s_1GiB": round((1 << 30) / (ms_big * 1e-3) / 1e9, 1),
            "launch_floor_us": round(ms_tiny * 1e3, 3)}


BF16_DENSE_PEAK_TFLOPS = 2500.0


def mfma_ceiling(b: Bench, rt, torch) -> float:
    """Sustained fp16 MFMA rate on the same box (TFLOP/s): the library's MFMA
    probe, 4 workgroups (16 waves) per CU, no memory traffic."""
    wg = 4 * torch.cuda.get_device_properties(b.dev).multi_processor_count
    iters = 2000
    sink = torch.empty(wg * 256, dtype=torch.float32, device=b.dev)
    ms, _, _ = b.time_calls([lambda s: rt.mfma_probe(wg, iters, sink, stream=s)], 10, 2)
    return wg * iters * rt.MFMA_PROBE_FLOPS_PER_WG_ITER / (ms * 1e-3) / 1e12


def bench_prefill(b: Bench, rt, torch) -> dict:
    """Config 4: GF4 prefill dequant-matmul, W 12288x4096 and 4096x12288 (12
    rotated copies), A bf16 N(0,1) [M][k], AWQ U(0.5,2), bf16 out; the staged
    path (workspace, fp16 MFMA; the time includes the staging pass) and the
    direct path (bf16 MFMA).  Then the q8_0 projections through their fp16
    prefill image (6 rotated copies).  Utilisation is reported against the
    nominal 2.5 PFLOP/s and against the MFMA probe's sustained rate on this box."""
    ceiling = mfma_ceiling(b, rt, torch)
    out = {"mfma_probe_TFLOP/s": round(ceiling, 1)}
    for rows, k in ((12288, 4096), (4096, 12288)):
        ws = [b.weight(rt.TYPE_GF4, rows, k) for _ in range(12)]
        awq = torch.rand((k,), generator=b.gen, device=b.dev) * 1.5 + 0.5
        for m in (128, 512, 2048):
            a = b.normal((m, k)).to(torch.bfloat16)
            c = torch.empty((m, rows), dtype=torch.bfloat16, device=b.dev)
            wsp = rt.prefill_workspace(ws[0], m, device=b.dev)
            for path, work in (("", wsp), ("_direct", None)):
                calls = [lambda s, w=w, work=work: rt.matmul_prefill(w, a, awq=awq, dst=c, workspace=work, stream=s)
                         for w in ws]
                ms, _, _ = b.time_calls(calls, max(24, 4800 // m), 12)
                tflops = 2.0 * m * rows * k / (ms * 1e-3) / 1e12
                out[f"prefill_gf4_m{m}_{rows}x{k}{path}"] = {
                    "us": round(ms * 1e3, 2), "TFLOP/s": round(tflops, 1),
                    "mfma_util": round(tflops / BF16_DENSE_PEAK_TFLOPS, 4),
                    "frac_of_probe": round(tflops / ceiling, 4)}
        del ws
    # k-quant projections (q8_0 attention/SSM q, out): the F16 prefill image,
    # made once per weight at load time, contracted on fp16 MFMA.
    for rows, k in ((8192, 4096), (4096, 4096)):
        q8 = [b.weight(rt.TYPE_Q8_0, rows, k) for _ in range(6)]
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        imgs = [w.prefill for w in q8]
        ev1.record()
        torch.cuda.synchronize()
        out[f"prefill_image_q8_0_{rows}x{k}_us"] = round(ev0.elapsed_time(ev1) * 1e3 / len(q8), 2)
        for m in (128, 512, 2048):
            a = b.normal((m, k)).to(torch.bfloat16)
            c = torch.empty((m, rows), dtype=torch.bfloat16, device=b.dev)
            wsp = rt.prefill_workspace(imgs[0], m, device=b.dev)
            calls = [lambda s, w=w: rt.matmul_prefill(w, a, dst=c, workspace=wsp, stream=s) for w in imgs]
            ms, _, _ = b.time_calls(calls, max(24, 4800 // m), 12)
            tflops = 2.0 * m * rows * k / (ms * 1e-3) / 1e12
            out[f"prefill_q8_0_f16img_m{m}_{rows}x{k}"] = {
                "us": round(ms * 1e3, 2), "TFLOP/s": round(tflops, 1),
                "mfma_util": round(tflops / BF16_DENSE_PEAK_TFLOPS, 4),
                "frac_of_probe": round(tflops / ceiling, 4)}
        del q8, imgs
    return out


def bench_q6k_head(b: Bench, rt, torch) -> dict:
    """The 9B LM head as the reference requires it (Q6_K, 248320 x 4096,
    qw35-server/src/metal/bridge/Qw35MetalRuntime.m:202-208): the full-logits
    GEMV and the fused greedy head (qw35_hip_output_argmax: GEMV + per-workgroup
    argmax + reduction, no logits written) at batch 1 and 8."""
    vocab, hidden = 248320, 4096
    head = b.weight(rt.TYPE_Q6_K, vocab, hidden, tile_rows=16384)
    wbytes = head.storage.numel()
    out = {}
    for nb in (1, 8):
        x = b.normal((nb, hidden))
        y = torch.zeros((nb, vocab), dtype=torch.float32, device=b.dev)
        m, _, _ = b.time_calls(gemv_calls(rt, [head], x, y), 200, 20)
        out[f"q6_k_head_b{nb}_248320x4096"] = {"us": round(m * 1e3, 3),
                                                "GB/s": round(gemv_bytes(rt.TYPE_Q6_K, vocab, hidden, nb, rt) / m / 1e6, 1)}
        ws = rt.output_argmax_workspace(head, nb, device=b.dev)
        m, _, _ = b.time_calls([lambda s: rt.output_argmax(head, x, workspace=ws, stream=s)], 200, 20)
        out[f"q6_k_greedy_head_b{nb}"] = {"us_two_launches": round(m * 1e3, 3),
                                          "GB/s": round((wbytes + 4 * nb * hidden) / m / 1e6, 1)}
    return out


def bench_codecs(b: Bench, rt, torch, steps: int, warmup: int) -> dict:
    """Every decode-GEMV codec on one 12288x4096 projection at batch 1 and 8,
    rotating enough copies (>= 640 MB) that the 256 MB last-level cache holds none."""
    out = {}
    rows, k = 12288, 4096
    names = {"gf4": rt.TYPE_GF4, "gf2": rt.TYPE_GF2, "q8_0": rt.TYPE_Q8_0, "q4_k": rt.TYPE_Q4_K,
             "q5_k": rt.TYPE_Q5_K, "q6_k": rt.TYPE_Q6_K}
    for name, t in names.items():
        nbytes = rows * rt.row_bytes(t, k)
        copies = max(2, -(-(640 << 20) // nbytes))
        ws = [b.weight(t, rows, k) for _ in range(copies)]
        for nb in (1, 8):
            x = b.normal((nb, k))
            y = torch.zeros((nb, rows), dtype=torch.float32, device=b.dev)
            m, _, _ = b.time_calls(gemv_calls(rt, ws, x, y), steps, warmup)
            out[f"codec_{name}_b{nb}_12288x4096"] = {"us": round(m * 1e3, 3),
                                                     "GB/s": round(gemv_bytes(t, rows, k, nb, rt) / m / 1e6, 1)}
        del ws
    return out


def bench_decode_stack(b: Bench, rt, torch) -> dict:
    """Config 5: the 32-layer Qwen3.5-9B decode-step projection stack as one
    recorded plan (hipGraph): per layer the q8_0 mixer projections (full
    attention every 4th layer: q 8192, k 1024, v 1024, o 4096 rows; Gated
    DeltaNet otherwise: qkv 8192, z 4096, beta 32, alpha 32, out 4096 rows; all
    k = 4096), GF4 fused gate/up/SwiGLU (12288 x 4096) and GF4 down
    (4096 x 12288, residual), then the Q4_K LM head (248320 x 4096).  Every
    layer has its own weight buffers (5.2 GB per token)."""
    hidden, ffn, vocab, layers = 4096, 12288, 248320, 32
    src = {}

    def layer_weight(t, rows, k):
        key = (t, rows, k)
        if key not in src:
            src[key] = b.normal((rows, k), 0.02, bf16=(t == rt.TYPE_GF4))
        return rt.quantize_weight(src[key], t)

    stack = []
    for il in range(layers):
        if (il + 1) % 4 == 0:
            mixer = [layer_weight(rt.TYPE_Q8_0, r, hidden) for r in (8192, 1024, 1024)]
        else:
            mixer = [layer_weight(rt.TYPE_Q8_0, r, hidden) for r in (8192, 4096, 32, 32)]
        out_proj = layer_weight(rt.TYPE_Q8_0, hidden, hidden)
        ffn_w = [layer_weight(rt.TYPE_GF4, ffn, hidden), layer_weight(rt.TYPE_GF4, ffn, hidden),
                 layer_weight(rt.TYPE_GF4, hidden, ffn)]
        stack.append((mixer, out_proj, ffn_w))
    src.clear()
    head = b.weight(rt.TYPE_Q4_K, vocab, hidden, tile_rows=16384)
    total = sum(w.storage.numel() for mixer, o, f in stack for w in (*mixer, o, *f)) + head.storage.numel()
    out = {}
    for nb in (1, 8):
        x = b.normal((nb, hidden))
        att = b.normal((nb, hidden))
        awq = torch.rand((hidden,), generator=b.gen, device=b.dev) * 1.5 + 0.5
        h = torch.zeros((nb, hidden), dtype=torch.float32, device=b.dev)
        g = torch.zeros((nb, ffn), dtype=torch.float32, device=b.dev)
        att_out = [torch.zeros((nb, r), dtype=torch.float32, device=b.dev) for r in (8192, 1024, 1024)]
        delta_out = [torch.zeros((nb, r), dtype=torch.float32, device=b.dev) for r in (8192, 4096, 32, 32)]
        logits = torch.zeros((nb, vocab), dtype=torch.float32, device=b.dev)
        plan = rt.DecodePlan()
        for mixer, out_proj, (gate, up, down) in stack:
            outs = att_out if len(mixer) == 3 else delta_out  # q/k/v or qkv/z/beta/alpha
            for w, o in zip(mixer, outs):
                plan.matvec(w, x, o)
            plan.matvec(out_proj, att, h, residual=True)
            plan.swiglu(gate, up, x, g, awq=awq)
            plan.matvec(down, g, h, residual=True)
        plan.matvec(head, x, logits)
        plan.record()
        with torch.cuda.stream(b.stream):
            for _ in range(3):
                plan.launch(stream=b.stream)
        torch.cuda.synchronize()
        reps = 20
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(b.stream):
            ev0.record(b.stream)
            for _ in range(reps):
                plan.launch(stream=b.stream)
            ev1.record(b.stream)
        torch.cuda.synchronize()
        us = ev0.elapsed_time(ev1) * 1e3 / reps
        out[f"decode_stack_9b_b{nb}"] = {
            "gemvs": len(plan), "weight_bytes": int(total), "us_per_step": round(us, 1),
            "us_per_token": round(us / nb, 1), "GB/s": round(total / us / 1e3, 1)}
        plan.close()
    return out


def cpu_baseline_gf4(rows: int, k: int, seed: int, reps: int):
    """numpy oracle on the host: GF4 dequant (vectorised numpy) + fp32 W @ x (BLAS)."""
    from threadpoolctl import threadpool_info

    from oracle import gf4 as ogf4
    from oracle import matvec as om

    rng = np.random.default_rng(seed)
    w = om.bf16_round(rng.standard_normal((rows, k), dtype=np.float32) * np.float32(0.02))
    words = ogf4.gf4_pack(w)
    x = rng.standard_normal(k, dtype=np.float32)
    ogf4.gf4_dequant(words) @ x  # warm-up
    t_dq, t_mv = [], []
    for _ in range(reps):
        t0 = time.perf_counter()
        wd = ogf4.gf4_dequant(words)
        t1 = time.perf_counter()
        _ = wd @ x
        t2 = time.perf_counter()
        t_dq.append(t1 - t0)
        t_mv.append(t2 - t1)
    blas = max([int(p.get("num_threads", 1)) for p in threadpool_info()] or [1])
    return float(np.median(t_dq)), float(np.median(t_mv)), blas


def cpu_model() -> str:
    """The host CPU's model name (the first 'model name' of /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4000)
    ap.add_argument("--warmup", type=int, default=400)
    ap.add_argument("--copies", type=int, default=32, help="distinct GF4 weight copies rotated (>= 24)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--headline-only", action="store_true", help="skip the extra configs (= --extras none)")
    ap.add_argument("--extras", default="all",
                    help="comma list of extra configs: gf4,q8,q4k,q6k,codecs,prefill,stack (or all / none)")
    ap.add_argument("--cpu-reps", type=int, default=40)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures one GPU; multi-GPU runs are not part of it (--gpus 1)"}),
              flush=True)
        return 2

    import torch

    from qwowl35_amd import runtime as rt

    b = Bench(torch, rt)
    rows, k = 12288, 4096
    log(f"config 1: GF4 {rows}x{k} b1, {args.copies} copies")
    weights = [b.weight(rt.TYPE_GF4, rows, k) for _ in range(args.copies)]
    x = b.normal((1, k))
    y = torch.zeros((1, rows), dtype=torch.float32, device=b.dev)
    # plain device copy of a known size: the calibration kernel of the PMC traffic passes
    calib = weights[0].storage.clone()
    torch.cuda.synchronize()
    del calib

    ms, _, launches = b.time_calls(gemv_calls(rt, weights, x, y), args.steps, args.warmup)
    algo = gemv_bytes(rt.TYPE_GF4, rows, k, 1, rt)
    value = algo / (ms * 1e-3) / 1e9
    log(f"GF4 b1: {ms * 1e3:.3f} us/launch, {value:.0f} GB/s")
    traffic, traffic_kernel = read_traffic("gf4_mfma_gemv<1,")

    extra = {}
    ceil = stream_ceiling(b, rt, torch, [w.storage for w in weights])
    extra["stream_read_ceiling"] = ceil
    extra["gf4_b1_frac_of_stream_ceiling"] = round(value / ceil["GB/s_25MB"], 4)
    # Best frac of 8 TB/s one dependent launch of these bytes could reach here:
    # the measured per-launch floor plus the bytes at the 1 GiB read rate.
    best_us = ceil["launch_floor_us"] + algo / (ceil["GB/s_1GiB"] * 1e3)
    extra["single_launch_frac_bound"] = round(algo / (best_us * 1e3) / HBM_PEAK_GBS, 4)
    want = set() if args.headline_only or args.extras == "none" else (
        {"gf4", "q8", "q4k", "q6k", "codecs", "prefill", "stack"} if args.extras == "all"
        else set(args.extras.split(",")))
    if "gf4" in want:
        for nb in (2, 4, 8):
            xb = b.normal((nb, k))
            yb = torch.zeros((nb, rows), dtype=torch.float32, device=b.dev)
            m, _, _ = b.time_calls(gemv_calls(rt, weights, xb, yb), args.steps // 2, args.warmup)
            extra[f"gf4_b{nb}_12288x4096"] = {"us": round(m * 1e3, 3),
                                              "GB/s": round(gemv_bytes(rt.TYPE_GF4, rows, k, nb, rt) / m / 1e6, 1)}
    del weights
    if "gf4" in want:
        wt = [b.weight(rt.TYPE_GF4, 4096, 12288) for _ in range(args.copies)]
        xt = b.normal((1, 12288))
        yt = torch.zeros((1, 4096), dtype=torch.float32, device=b.dev)
        m, _, _ = b.time_calls(gemv_calls(rt, wt, xt, yt), args.steps // 2, args.warmup)
        extra["gf4_b1_4096x12288"] = {"us": round(m * 1e3, 3),
                                      "GB/s": round(gemv_bytes(rt.TYPE_GF4, 4096, 12288, 1, rt) / m / 1e6, 1)}
        del wt
    if "q8" in want:
        # config 2: q8_0 projections of one decoder layer, 3 distinct sets (670 MB)
        shapes = [(8192, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (12288, 4096), (12288, 4096),
                  (4096, 12288)]
        sets = [[b.weight(rt.TYPE_Q8_0, r, kk) for r, kk in shapes] for _ in range(3)]
        acts = {kk: b.normal((1, kk)) for kk in (4096, 12288)}
        outs = {r: torch.zeros((1, r), dtype=torch.float32, device=b.dev) for r, _ in shapes}
        calls = [lambda s, w=w: rt.decode_matvec(w, acts[w.k], outs[w.rows], stream=s) for st in sets for w in st]
        m, _, _ = b.time_calls(calls, args.steps // 2, args.warmup)
        per_set_ms = m * len(shapes)
        set_bytes = sum(gemv_bytes(rt.TYPE_Q8_0, r, kk, 1, rt) for r, kk in shapes)
        extra["q8_0_layer_set_b1"] = {"us_per_set": round(per_set_ms * 1e3, 3), "bytes": set_bytes,
                                      "GB/s": round(set_bytes / per_set_ms / 1e6, 1)}
        # The same sets as one recorded decode plan, each projection reading
        # the input it has in a layer: q/k/v share the attention input and
        # gate/up the FFN input, so each group is one launch (4 per set).
        xin = {name: b.normal((1, kk)) for name, kk in
               (("attn", 4096), ("o", 4096), ("ffn", 4096), ("down", 12288))}
        role = ["attn", "attn", "attn", "o", "ffn", "ffn", "down"]
        ys = [torch.zeros((1, r), dtype=torch.float32, device=b.dev) for r, _ in shapes]
        plan = rt.DecodePlan()
        for st in sets:
            for w, r, y in zip(st, role, ys):
                plan.matvec(w, xin[r], y)
        plan.record()
        with torch.cuda.stream(b.stream):
            for _ in range(3):
                plan.launch(stream=b.stream)
        torch.cuda.synchronize()
        reps = max(20, args.steps // 40)
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(b.stream):
            ev0.record(b.stream)
            for _ in range(reps):
                plan.launch(stream=b.stream)
            ev1.record(b.stream)
        torch.cuda.synchronize()
        plan_set_ms = ev0.elapsed_time(ev1) / reps / len(sets)
        extra["q8_0_layer_set_b1_plan"] = {"us_per_set": round(plan_set_ms * 1e3, 3), "merged": "q/k/v, o, gate/up, down",
                                           "GB/s": round(set_bytes / plan_set_ms / 1e6, 1)}
        plan.close()
        del sets
    if "q4k" in want:
        # config 3: Q4_K down 4096x12288 (24 copies) and LM head 248320x4096, batch 1 and 8
        down = [b.weight(rt.TYPE_Q4_K, 4096, 12288) for _ in range(24)]
        head = b.weight(rt.TYPE_Q4_K, 248320, 4096, tile_rows=16384)
        for nb in (1, 8):
            xd = b.normal((nb, 12288))
            yd = torch.zeros((nb, 4096), dtype=torch.float32, device=b.dev)
            m, _, _ = b.time_calls(gemv_calls(rt, down, xd, yd), args.steps // 4, args.warmup // 2)
            extra[f"q4_k_down_b{nb}_4096x12288"] = {
                "us": round(m * 1e3, 3), "GB/s": round(gemv_bytes(rt.TYPE_Q4_K, 4096, 12288, nb, rt) / m / 1e6, 1)}
            xh = b.normal((nb, 4096))
            yh = torch.zeros((nb, 248320), dtype=torch.float32, device=b.dev)
            m, _, _ = b.time_calls(gemv_calls(rt, [head], xh, yh), 200, 20)
            extra[f"q4_k_head_b{nb}_248320x4096"] = {
                "us": round(m * 1e3, 3), "GB/s": round(gemv_bytes(rt.TYPE_Q4_K, 248320, 4096, nb, rt) / m / 1e6, 1)}
        del down, head
    if "q6k" in want:
        extra.update(bench_q6k_head(b, rt, torch))
    if "codecs" in want:
        extra.update(bench_codecs(b, rt, torch, args.steps // 4, args.warmup // 2))
    if "prefill" in want:
        extra.update(bench_prefill(b, rt, torch))
    if "stack" in want:
        extra.update(bench_decode_stack(b, rt, torch))
    for key, v in extra.items():
        log(f"{key}: {v}")

    cpu = None
    if not args.no_cpu:
        t_dq, t_mv, blas = cpu_baseline_gf4(rows, k, seed=1, reps=args.cpu_reps)
        cpu = {
            "value": round(algo / (t_dq + t_mv) / 1e9, 3),
            "unit": "GB/s",
            "cores": blas,
            "kind": "port",
            "sample": f"numpy oracle on the host: GF4 dequant of the 12288x4096 b1 weight (1 thread, "
                      f"{t_dq * 1e3:.1f} ms) + fp32 W@x ({blas} BLAS threads, {t_mv * 1e3:.2f} ms), "
                      f"median of {args.cpu_reps}; {cpu_model()}, {os.cpu_count()} logical CPUs visible",
        }
    out = {
        "metric": "GF4 b1 matvec HBM GB/s (12288x4096)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": launches,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "gf4-weights/fp32-acc",
        "data": "synthetic",
        "config": {"workload": "gf4_matvec_b1_12288x4096", "rows": rows, "k": k, "batch": 1,
                   "weight_copies": args.copies},
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": traffic},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
