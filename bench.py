#!/usr/bin/env python3
"""Benchmark of the quantized GEMV / prefill path on one MI355X.

Headline (BASELINE.json metric, config 1): the GF4 decode GEMV, batch 1, W
12288x4096 = GF4 pack of bf16(0.02 N(0,1)), x fp32 N(0,1).  One "step" is one
GEMV launch over one weight copy; the launches rotate over 32 distinct weight
copies (805 MB > the 256 MB Infinity Cache) so every step streams its weights
from HBM.  Exactly ``--steps`` launches are timed.  Weights and activations are
made on the GPU (torch's seeded generator, the library's own encoders) and are
resident before timing; nothing crosses PCIe inside the timed region.

Launches are captured into hipGraphs and replayed; HIP events recorded on the
replay stream bracket the timed replays.  Printed: one JSON line with the
driver's contract fields plus ``roofline`` (the headline kernel) and
``cpu_baseline`` (the numpy oracle's dequantisation + BLAS matvec on this
host's cores), and under ``extra`` the other configs, each with its own
``roofline`` and ``cpu_baseline``: GF4 batches 2..8 and the down-projection
shape, the q8_0 layer set (config 2), the Q4_K down / LM-head GEMVs at batch 1
and 8 (config 3), the Q6_K head and greedy head, the GF4 prefill matmul with
its MFMA utilisation (config 4), and the 32-layer 9B decode-step projection
stack replayed as one recorded plan (config 5).  ``roofline.traffic`` is the
PMC-measured HBM bytes per launch from the committed ``profiles/*_traffic.md``
summary whose kernel line names exactly the instantiation this run launches
(``qw35_hip_gemv_kernel``), else null.  ``--gpus`` above 1 is refused: this
build measures one GPU.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import glob
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_DENSE_PEAK_TFLOPS = 2500.0
DTYPE = "gf4/q8_0/q4_k weights as exact f16, f32 activations as f16 hi+lo, f32 accumulate"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---------------------------------------------------------------- rooflines


def traffic_for(kernel: str | None) -> int | None:
    """HBM bytes per launch from the committed PMC summary that names exactly this kernel."""
    if not kernel:
        return None
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*_traffic.md"))):
        text = open(path).read()
        for m in re.finditer(r"kernel:\s*`([^`]+)`\s*\ntraffic_bytes_per_launch:\s*(\d+)", text):
            if re.search(re.escape(kernel) + r"\(", m.group(1)):
                return int(m.group(2))
    return None


def hbm_roofline(nbytes: float, us: float, kernel: str | None = None) -> dict:
    gbs = nbytes / (us * 1e3)
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic_for(kernel), "kernel": kernel}


def mfma_roofline(flops: float, us: float, kernel: str | None = None) -> dict:
    tf = flops / (us * 1e6)
    return {"bound": "mfma", "achieved": round(tf, 1), "peak": BF16_DENSE_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tf / BF16_DENSE_PEAK_TFLOPS, 4), "traffic": None, "kernel": kernel}


# ---------------------------------------------------------------- GPU timing


class Bench:
    def __init__(self, torch, rt, seed: int = 1):
        self.torch = torch
        self.rt = rt
        self.dev = torch.device("cuda:0")
        self.gen = torch.Generator(device=self.dev)
        self.gen.manual_seed(seed)
        self.stream = torch.cuda.Stream()  # default priority

    def normal(self, shape, std=1.0, bf16=False):
        t = self.torch.randn(shape, generator=self.gen, device=self.dev, dtype=self.torch.float32)
        if std != 1.0:
            t.mul_(std)
        if bf16:
            t = t.to(self.torch.bfloat16).to(self.torch.float32)
        return t

    def weight(self, type_id, rows, k, tile_rows=None):
        """Encoded N(0, 0.02) weight; tile_rows repeats that many distinct rows (the LM heads)."""
        from qwowl35_amd import qwen35

        if tile_rows is None or tile_rows >= rows:
            return qwen35.synthetic_weight(self.gen, type_id, rows, k)
        part = qwen35.synthetic_weight(self.gen, type_id, tile_rows, k)
        rb = self.rt.row_bytes(type_id, k)
        full = self.torch.empty(rows * rb, dtype=self.torch.uint8, device=self.dev)
        for r0 in range(0, rows, tile_rows):
            n = min(tile_rows, rows - r0)
            full[r0 * rb:(r0 + n) * rb].copy_(part.storage[:n * rb])
        return self.rt.HipWeight.from_device(full, type_id, rows, k)

    def _graph(self, calls):
        torch = self.torch
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=self.stream):
            for c in calls:
                c(self.stream)
        return g

    # Windows of up to this many launches issue them one by one behind the
    # warm-up work; longer ones replay one graph holding all of them.
    DIRECT_MAX = 64
    # GPU time the warm-up replays queue ahead of the window's start event.
    BACKLOG_MS = 20.0

    def time_launches(self, calls, launches: int, warmup: int):
        """Time exactly ``launches`` launches, rotating over ``calls`` (one launch
        each); returns (ms per launch, launches).

        The window's start event is queued behind at least BACKLOG_MS of
        warm-up replays still running on the GPU, so the window holds kernels
        back to back: not an idle GPU's first launch, and not the host's time
        to submit the timed work (a graph launch prepares its nodes before the
        first one runs; a 200-launch window behind 0.45 ms of warm-up measured
        7.41 us per headline launch against 6.85 behind 2.8 ms).  The first
        window of a process also ran slow behind 4 ms (20 headline launches:
        7.32-7.56 us) and not behind 20 ms (6.99-7.02, against 6.82 for 4000
        launches).  A graph replay boundary inside the window costs about
        5-20 us (about 0.14 us per launch when a 32-launch rotation graph is
        replayed 125 times, 0.2-1 us per launch of a 20-launch window), so the
        window holds none: up to DIRECT_MAX launches are issued one by one
        (the backlog also covers about 0.1 ms of host time per call), longer
        windows are one graph of exactly that many launches, whose one
        boundary is spread over all of them."""
        torch = self.torch
        n = len(calls)
        launches = max(1, int(launches))
        with torch.cuda.stream(self.stream):
            for c in calls:  # first touch and code-object load outside the capture
                c(self.stream)
        torch.cuda.synchronize()
        direct = launches <= self.DIRECT_MAX
        warm = self._graph([calls[i % n] for i in range(max(int(warmup), 2 * n))])
        timed = None if direct else self._graph([calls[i % n] for i in range(launches)])
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(self.stream):  # replays, launches and events on the same stream
            if timed is not None:
                timed.replay()
            ev0.record(self.stream)
            warm.replay()
            ev1.record(self.stream)
            torch.cuda.synchronize()
            warm_ms = max(ev0.elapsed_time(ev1), 1e-3)
            backlog_ms = self.BACKLOG_MS + (0.1 * launches if direct else 0.0)
            for _ in range(max(2, -(-int(backlog_ms * 1000) // int(warm_ms * 1000 + 1)))):
                warm.replay()  # still running while the window is queued
            ev0.record(self.stream)
            if timed is not None:
                timed.replay()
            else:
                for i in range(launches):
                    calls[i % n](self.stream)
            ev1.record(self.stream)
        torch.cuda.synchronize()
        return ev0.elapsed_time(ev1) / launches, launches

    def time_plan(self, plan, reps: int, warmup: int = 3):
        """ms per replay of a recorded DecodePlan."""
        torch = self.torch
        with torch.cuda.stream(self.stream):
            for _ in range(warmup):
                plan.launch(stream=self.stream)
        torch.cuda.synchronize()
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(self.stream):
            ev0.record(self.stream)
            for _ in range(reps):
                plan.launch(stream=self.stream)
            ev1.record(self.stream)
        torch.cuda.synchronize()
        return ev0.elapsed_time(ev1) / reps


def gemv_calls(rt, weights, x, y, awq=None, workspace=None):
    return [lambda s, w=w: rt.decode_matvec(w, x, y, awq=awq, stream=s, workspace=workspace) for w in weights]


def gemv_bytes(rt, type_id, rows, k, nb):
    return rows * rt.row_bytes(type_id, k) + 4 * nb * (k + rows)


def gemv_line(b: Bench, weights, nb, launches, warmup, awq=None) -> dict:
    """One GEMV configuration: µs per launch, algorithmic GB/s and its roofline.
    Shapes whose launch splits K get a workspace (qw35_hip_decode_matvec_ws),
    as the decode plans have."""
    rt, w0 = b.rt, weights[0]
    x = b.normal((nb, w0.k))
    y = b.torch.zeros((nb, w0.rows), dtype=b.torch.float32, device=b.dev)
    ws = rt.decode_matvec_workspace(w0, nb, device=b.dev)
    ms, _ = b.time_launches(gemv_calls(rt, weights, x, y, awq, ws), launches, warmup)
    kern = rt.gemv_kernel(w0, nb, awq=awq is not None, workspace=ws is not None)
    nbytes = gemv_bytes(rt, w0.type_id, w0.rows, w0.k, nb)
    return {"us": round(ms * 1e3, 3), "bytes": nbytes, "roofline": hbm_roofline(nbytes, ms * 1e3, kern["name"]),
            "launch": {"grid": kern["grid"], "block": kern["block"]}}


def stream_ceiling(b: Bench, bufs) -> dict:
    """Streaming-read ceiling on the same box: the library's read probe over the
    same rotated 25 MB buffers (launch and ramp included, like the GEMV), over
    one 1 GiB buffer, and over 16 bytes (one workgroup: the per-launch floor)."""
    rt, torch = b.rt, b.torch
    sinks = [torch.empty(rt.stream_read(bufs[0]).numel(), dtype=torch.int32, device=b.dev) for _ in bufs]
    calls = [lambda s, t=t, k=k: rt.stream_read(t, k, stream=s) for t, k in zip(bufs, sinks)]
    ms, _ = b.time_launches(calls, 2000, 200)
    big = torch.zeros(1 << 30, dtype=torch.uint8, device=b.dev)
    sink_big = rt.stream_read(big)
    ms_big, _ = b.time_launches([lambda s: rt.stream_read(big, sink_big, stream=s)], 40, 5)
    n = bufs[0].numel()
    tiny = torch.zeros(16, dtype=torch.uint8, device=b.dev)
    sink_tiny = rt.stream_read(tiny)
    ms_tiny, _ = b.time_launches([lambda s: rt.stream_read(tiny, sink_tiny, stream=s)] * 32, 2000, 200)
    return {"GB/s_25MB": round(n / (ms * 1e-3) / 1e9, 1), "us_25MB": round(ms * 1e3, 3),
            "GB/s_1GiB": round((1 << 30) / (ms_big * 1e-3) / 1e9, 1), "launch_floor_us": round(ms_tiny * 1e3, 3)}


def mfma_ceiling(b: Bench) -> float:
    """Sustained fp16 MFMA rate on the same box (TFLOP/s): the library's MFMA
    probe, 4 workgroups (16 waves) per CU, no memory traffic."""
    rt, torch = b.rt, b.torch
    wg = 4 * torch.cuda.get_device_properties(b.dev).multi_processor_count
    iters = 2000
    sink = torch.empty(wg * 256, dtype=torch.float32, device=b.dev)
    ms, _ = b.time_launches([lambda s: rt.mfma_probe(wg, iters, sink, stream=s)], 10, 2)
    return wg * iters * rt.MFMA_PROBE_FLOPS_PER_WG_ITER / (ms * 1e-3) / 1e12


# ---------------------------------------------------------------- CPU baseline (numpy oracle)


def cpu_threads() -> int:
    """Worker threads for the numpy baseline: the job's CPU share (OMP_NUM_THREADS), else the visible CPUs."""
    try:
        return max(1, int(os.environ.get("OMP_NUM_THREADS", "")))
    except ValueError:
        return max(1, min(16, os.cpu_count() or 1))


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


class CpuBaseline:
    """The repository's numpy CPU path: the oracle's vectorised dequantisation
    (rows split over ``threads`` workers; numpy releases the GIL) into an fp32
    matrix, then BLAS ``W @ x`` (float32).  Dequantisation and product are timed
    separately with perf_counter, median of ``reps`` after one warm-up."""

    def __init__(self, threads: int, reps: int):
        self.threads = threads
        self.reps = reps
        self.pool = cf.ThreadPoolExecutor(max_workers=threads)
        try:
            from threadpoolctl import threadpool_info

            self.blas = max([int(p.get("num_threads", 1)) for p in threadpool_info()] or [1])
        except Exception:  # noqa: BLE001
            self.blas = 1

    def dequant(self, type_id, raw: np.ndarray, rows: int, k: int, out: np.ndarray) -> None:
        from oracle import matvec as om

        rb = raw.size // rows
        raw2 = raw.reshape(rows, rb)
        step = -(-rows // self.threads)

        def job(r0):
            r1 = min(rows, r0 + step)
            out[r0:r1] = om.dequant(type_id, raw2[r0:r1], r1 - r0, k)

        list(self.pool.map(job, range(0, rows, step)))

    def gemv(self, type_id, raw: np.ndarray, rows: int, k: int, nb: int, seed: int = 0) -> tuple[float, float]:
        """(seconds of dequantisation, seconds of W @ X) per call, medians."""
        x = np.random.default_rng(seed).standard_normal((k, nb), dtype=np.float32)
        w = np.empty((rows, k), dtype=np.float32)
        self.dequant(type_id, raw, rows, k, w)
        _ = w @ x
        t_dq, t_mv = [], []
        for _ in range(self.reps):
            t0 = time.perf_counter()
            self.dequant(type_id, raw, rows, k, w)
            t1 = time.perf_counter()
            _ = w @ x
            t2 = time.perf_counter()
            t_dq.append(t1 - t0)
            t_mv.append(t2 - t1)
        self._quiesce()
        return float(np.median(t_dq)), float(np.median(t_mv))

    def matmul(self, type_id, raw: np.ndarray, rows: int, k: int, m: int, seed: int = 0) -> tuple[float, float]:
        """(dequantisation s, fp32 W @ A^T s) for an m-token chunk (the prefill baseline)."""
        a = np.random.default_rng(seed).standard_normal((k, m), dtype=np.float32)
        w = np.empty((rows, k), dtype=np.float32)
        self.dequant(type_id, raw, rows, k, w)
        _ = w @ a
        t_dq, t_mm = [], []
        for _ in range(self.reps):
            t0 = time.perf_counter()
            self.dequant(type_id, raw, rows, k, w)
            t1 = time.perf_counter()
            _ = w @ a
            t2 = time.perf_counter()
            t_dq.append(t1 - t0)
            t_mm.append(t2 - t1)
        self._quiesce()
        return float(np.median(t_dq)), float(np.median(t_mm))

    @staticmethod
    def _quiesce() -> None:
        """OpenBLAS worker threads spin for a while after a call before they
        sleep; the GPU line timed next must not share the job's CPUs with them
        (a timed window of few graph replays stalls when the submitting thread
        is descheduled: one such line measured 3x its time)."""
        time.sleep(0.3)

    def record(self, value, unit, sample: str) -> dict:
        return {"value": value, "unit": unit, "cores": self.threads, "kind": "port",
                "sample": f"{sample}; numpy oracle dequantisation on {self.threads} threads + BLAS ({self.blas} "
                          f"threads), median of {self.reps}; {cpu_model()}, {os.cpu_count()} logical CPUs visible"}


def host_bytes(w) -> np.ndarray:
    return w.storage.cpu().numpy()


# ---------------------------------------------------------------- configs


def bench_gf4_extra(b: Bench, weights, cpu: CpuBaseline | None, steps: int, warmup: int) -> dict:
    """GF4 12288x4096 at batch 2, 4, 8 (same rotated copies as the headline) and
    4096x12288 (the FFN down projection) at batch 1 and 8."""
    rt, out = b.rt, {}
    # The headline kernel with its weights cache-resident: every launch reads
    # one copy (25 MB, inside the 256 MB last-level cache), so HBM is not the limit.
    x1 = b.normal((1, weights[0].k))
    y1 = b.torch.zeros((1, weights[0].rows), dtype=b.torch.float32, device=b.dev)
    ms_hot, _ = b.time_launches(gemv_calls(rt, [weights[0]] * len(weights), x1, y1), 960, 96)
    out["gf4_b1_same_weights_us"] = round(ms_hot * 1e3, 3)
    for nb in (2, 4, 8):
        out[f"gf4_b{nb}_12288x4096"] = gemv_line(b, weights, nb, steps // 2, warmup)
    down = [b.weight(rt.TYPE_GF4, 4096, 12288) for _ in range(32)]
    for nb in (1, 8):
        line = gemv_line(b, down, nb, steps // 2, warmup)
        if cpu is not None:
            t_dq, t_mv = cpu.gemv(rt.TYPE_GF4, host_bytes(down[0]), 4096, 12288, nb)
            line["cpu_baseline"] = cpu.record(round(line["bytes"] / (t_dq + t_mv) / 1e9, 3), "GB/s",
                                              f"GF4 4096x12288 b{nb}: dequant {t_dq * 1e3:.1f} ms + matvec "
                                              f"{t_mv * 1e3:.2f} ms per call")
        out[f"gf4_b{nb}_4096x12288"] = line
    del down
    return out


Q8_LAYER = [(8192, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (12288, 4096), (12288, 4096), (4096, 12288)]


def bench_q8_layer(b: Bench, cpu: CpuBaseline | None, steps: int, warmup: int) -> dict:
    """Config 2: q8_0 projections of one decoder layer (q 8192, k / v 1024, o 4096,
    gate / up 12288 rows x 4096; down 4096 x 12288), batch 1, 3 distinct sets (670 MB)."""
    rt, torch = b.rt, b.torch
    sets = [[b.weight(rt.TYPE_Q8_0, r, k) for r, k in Q8_LAYER] for _ in range(3)]
    acts = {k: b.normal((1, k)) for k in (4096, 12288)}
    outs = {r: torch.zeros((1, r), dtype=torch.float32, device=b.dev) for r, _ in Q8_LAYER}
    calls = [lambda s, w=w: rt.decode_matvec(w, acts[w.k], outs[w.rows], stream=s) for st in sets for w in st]
    ms, _ = b.time_launches(calls, max(len(calls), steps // 2), warmup)
    set_bytes = sum(gemv_bytes(rt, rt.TYPE_Q8_0, r, k, 1) for r, k in Q8_LAYER)
    set_us = ms * 1e3 * len(Q8_LAYER)
    per_matrix = {f"{r}x{k}": rt.gemv_kernel(w, 1)["name"] for (r, k), w in zip(Q8_LAYER, sets[0])}
    out = {"q8_0_layer_set_b1": {"us_per_set": round(set_us, 3), "bytes": set_bytes, "kernels": per_matrix,
                                 "roofline": hbm_roofline(set_bytes, set_us)}}
    # The same sets as one recorded plan, each projection reading the input it
    # has in a layer: q/k/v share the attention input and gate/up the FFN input,
    # so each group is one merged launch (4 per set).
    xin = {name: b.normal((1, k)) for name, k in (("attn", 4096), ("o", 4096), ("ffn", 4096), ("down", 12288))}
    role = ["attn", "attn", "attn", "o", "ffn", "ffn", "down"]
    ys = [torch.zeros((1, r), dtype=torch.float32, device=b.dev) for r, _ in Q8_LAYER]
    plan = rt.DecodePlan()
    for st in sets:
        for w, r, y in zip(st, role, ys):
            plan.matvec(w, xin[r], y)
    plan.record()
    plan_us = b.time_plan(plan, max(20, steps // 40)) * 1e3 / len(sets)
    plan.close()
    line = {"us_per_set": round(plan_us, 3), "merged": "q/k/v, o, gate/up, down", "bytes": set_bytes,
            "roofline": hbm_roofline(set_bytes, plan_us)}
    if cpu is not None:
        t = 0.0
        parts = []
        for (r, k), w in zip(Q8_LAYER, sets[0]):
            t_dq, t_mv = cpu.gemv(rt.TYPE_Q8_0, host_bytes(w), r, k, 1)
            t += t_dq + t_mv
            parts.append(f"{r}x{k} {1e3 * (t_dq + t_mv):.1f} ms")
        line["cpu_baseline"] = cpu.record(round(set_bytes / t / 1e9, 3), "GB/s",
                                          f"the 7 q8_0 matrices at full size, b1 ({', '.join(parts)})")
        out["q8_0_layer_set_b1"]["cpu_baseline"] = line["cpu_baseline"]
    out["q8_0_layer_set_b1_plan"] = line
    del sets
    return out


def bench_q4k(b: Bench, cpu: CpuBaseline | None, steps: int, warmup: int) -> dict:
    """Config 3: Q4_K down 4096x12288 (24 copies) and LM head 248320x4096, batch 1 and 8."""
    rt = b.rt
    out = {}
    down = [b.weight(rt.TYPE_Q4_K, 4096, 12288) for _ in range(24)]
    head = b.weight(rt.TYPE_Q4_K, 248320, 4096, tile_rows=16384)
    for nb in (1, 8):
        out[f"q4_k_down_b{nb}_4096x12288"] = gemv_line(b, down, nb, steps // 4, warmup // 2)
        out[f"q4_k_head_b{nb}_248320x4096"] = gemv_line(b, [head], nb, 200, 20)
        if cpu is not None:
            t_dq, t_mv = cpu.gemv(rt.TYPE_Q4_K, host_bytes(down[0]), 4096, 12288, nb)
            line = out[f"q4_k_down_b{nb}_4096x12288"]
            line["cpu_baseline"] = cpu.record(round(line["bytes"] / (t_dq + t_mv) / 1e9, 3), "GB/s",
                                              f"Q4_K 4096x12288 b{nb}: dequant {t_dq * 1e3:.1f} ms + matvec "
                                              f"{t_mv * 1e3:.2f} ms per call")
            # head: a sample of 1/8 of the rows (31040 x 4096), time scaled by 8
            rows = 248320 // 8
            raw = host_bytes(head)[: rows * rt.row_bytes(rt.TYPE_Q4_K, 4096)]
            t_dq, t_mv = cpu.gemv(rt.TYPE_Q4_K, raw, rows, 4096, nb)
            line = out[f"q4_k_head_b{nb}_248320x4096"]
            line["cpu_baseline"] = cpu.record(round(line["bytes"] / (8 * (t_dq + t_mv)) / 1e9, 3), "GB/s",
                                              f"Q4_K head b{nb}: 31040 of the 248320 rows (dequant "
                                              f"{t_dq * 1e3:.1f} ms + matvec {t_mv * 1e3:.2f} ms), scaled by 8")
    del down, head
    return out


def bench_q6k_head(b: Bench, steps: int, cpu: CpuBaseline | None = None) -> dict:
    """The 9B LM head as the reference requires it (Q6_K, 248320 x 4096,
    Qw35MetalRuntime.m:202-208): the full-logits GEMV and the fused greedy
    head (GEMV + per-workgroup argmax + reduction, no logits written), b1 and b8."""
    rt, torch = b.rt, b.torch
    vocab, hidden = 248320, 4096
    head = b.weight(rt.TYPE_Q6_K, vocab, hidden, tile_rows=16384)
    wbytes = head.storage.numel()
    out = {}
    for nb in (1, 8):
        line = out[f"q6_k_head_b{nb}_248320x4096"] = gemv_line(b, [head], nb, 200, 20)
        if cpu is not None:
            # a sample of 1/64 of the rows (3880 x 4096; the numpy Q6_K unpacking
            # is ~10x slower per row than Q4_K's), time scaled by 64
            rows = vocab // 64
            raw = host_bytes(head)[: rows * rt.row_bytes(rt.TYPE_Q6_K, hidden)]
            t_dq, t_mv = cpu.gemv(rt.TYPE_Q6_K, raw, rows, hidden, nb)
            line["cpu_baseline"] = cpu.record(round(line["bytes"] / (64 * (t_dq + t_mv)) / 1e9, 3), "GB/s",
                                              f"Q6_K head b{nb}: 3880 of the 248320 rows (dequant "
                                              f"{t_dq * 1e3:.1f} ms + matvec {t_mv * 1e3:.2f} ms), scaled by 64")
        x = b.normal((nb, hidden))
        ws = rt.output_argmax_workspace(head, nb, device=b.dev)
        ms, _ = b.time_launches([lambda s: rt.output_argmax(head, x, workspace=ws, stream=s)], 200, 20)
        nbytes = wbytes + 4 * nb * hidden
        out[f"q6_k_greedy_head_b{nb}"] = {"us_two_launches": round(ms * 1e3, 3), "bytes": nbytes,
                                          "roofline": hbm_roofline(nbytes, ms * 1e3)}
    return out


def bench_codecs(b: Bench, steps: int, warmup: int) -> dict:
    """Every decode-GEMV codec on one 12288x4096 projection at batch 1 and 8,
    rotating enough copies (>= 640 MB) that the last-level cache holds none."""
    rt, out = b.rt, {}
    names = {"gf4": rt.TYPE_GF4, "gf2": rt.TYPE_GF2, "q8_0": rt.TYPE_Q8_0, "q4_k": rt.TYPE_Q4_K,
             "q5_k": rt.TYPE_Q5_K, "q6_k": rt.TYPE_Q6_K}
    for name, t in names.items():
        copies = max(2, -(-(640 << 20) // (12288 * rt.row_bytes(t, 4096))))
        ws = [b.weight(t, 12288, 4096) for _ in range(copies)]
        for nb in (1, 8):
            out[f"codec_{name}_b{nb}_12288x4096"] = gemv_line(b, ws, nb, steps, warmup)
        del ws
    return out


def bench_prefill(b: Bench, cpu: CpuBaseline | None) -> dict:
    """Config 4: GF4 prefill dequant-matmul, W 12288x4096 and 4096x12288 (12
    rotated copies), A bf16 N(0,1) [M][k], AWQ U(0.5,2), bf16 out, on the
    staged path (workspace, fp16 MFMA; the time includes the staging pass).
    Each shape also at M = 128 with fp32 activations and fp32 out (the
    runtime's multi-token chunks: an fp16 hi/lo pair per activation, twice the
    MFMA work).  Then q8_0 and Q4_K projections (6 rotated copies),
    dequantised inside the staged kernel and, for comparison, through their
    fp16 prefill image.  Utilisation is against the nominal 2.5 PFLOP/s and against the
    MFMA probe's sustained rate on this box.  Every line of this library's
    kernels carries the CPU baseline of the same shape and M (numpy
    dequantisation + fp32 BLAS)."""
    rt, torch = b.rt, b.torch
    ceiling = mfma_ceiling(b)
    out = {"mfma_probe_TFLOP/s": round(ceiling, 1)}

    def line(ms, m, rows, k, kern):
        flops = 2.0 * m * rows * k
        r = {"us": round(ms * 1e3, 2), "flops": flops, "roofline": mfma_roofline(flops, ms * 1e3, kern["name"]),
             "launch": {"grid": kern["grid"], "block": kern["block"], "splits": kern["splits"]}}
        r["frac_of_probe"] = round(flops / (ms * 1e-3) / 1e12 / ceiling, 4)
        return r

    def with_cpu(r, type_id, w, rows, k, m, what):
        if cpu is not None:
            t_dq, t_mm = cpu.matmul(type_id, host_bytes(w), rows, k, m)
            r["cpu_baseline"] = cpu.record(
                round(2.0 * m * rows * k / (t_dq + t_mm) / 1e12, 4), "TFLOP/s",
                f"{what} {rows}x{k}, M={m}: dequant {t_dq * 1e3:.1f} ms + fp32 W@A^T {t_mm * 1e3:.1f} ms")
        return r

    for rows, k in ((12288, 4096), (4096, 12288)):
        ws = [b.weight(rt.TYPE_GF4, rows, k) for _ in range(12)]
        awq = torch.rand((k,), generator=b.gen, device=b.dev) * 1.5 + 0.5
        for m, a_dt, c_dt, tag in ((128, torch.bfloat16, torch.bfloat16, ""), (512, torch.bfloat16, torch.bfloat16, ""),
                                   (2048, torch.bfloat16, torch.bfloat16, ""), (128, torch.float32, torch.float32, "_f32")):
            a = b.normal((m, k)).to(a_dt)
            c = torch.empty((m, rows), dtype=c_dt, device=b.dev)
            wsp = rt.prefill_workspace(ws[0], m, device=b.dev)
            calls = [lambda s, w=w: rt.matmul_prefill(w, a, awq=awq, out_dtype=c_dt, dst=c, workspace=wsp, stream=s)
                     for w in ws]
            ms, _ = b.time_launches(calls, max(24, 4800 // m), 12)
            kern = rt.prefill_kernel(ws[0], m, a_dt, awq=True, out_dtype=c_dt)
            out[f"prefill_gf4{tag}_m{m}_{rows}x{k}"] = with_cpu(line(ms, m, rows, k, kern), rt.TYPE_GF4, ws[0],
                                                                rows, k, m, "GF4")
        del ws
    for type_id, name, rows, k, ms_list in ((rt.TYPE_Q8_0, "q8_0", 8192, 4096, (128, 512, 2048)),
                                            (rt.TYPE_Q8_0, "q8_0", 4096, 4096, (128, 512, 2048)),
                                            (rt.TYPE_Q4_K, "q4_k", 12288, 4096, (128, 512)),
                                            (rt.TYPE_Q4_K, "q4_k", 4096, 12288, (128, 512))):
        wq = [b.weight(type_id, rows, k) for _ in range(6)]
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        imgs = [rt.prefill_image(w) for w in wq]
        ev1.record()
        torch.cuda.synchronize()
        out[f"prefill_image_{name}_{rows}x{k}_us"] = round(ev0.elapsed_time(ev1) * 1e3 / len(wq), 2)
        for m in ms_list:
            a = b.normal((m, k)).to(torch.bfloat16)
            c = torch.empty((m, rows), dtype=torch.bfloat16, device=b.dev)
            for tag, wl in (("", wq), ("_f16img", imgs)):
                wsp = rt.prefill_workspace(wl[0], m, device=b.dev)
                calls = [lambda s, w=w, wsp=wsp: rt.matmul_prefill(w, a, dst=c, workspace=wsp, stream=s) for w in wl]
                ms, _ = b.time_launches(calls, max(24, 4800 // m), 12)
                r = line(ms, m, rows, k, rt.prefill_kernel(wl[0], m))
                if not tag:
                    r = with_cpu(r, type_id, wq[0], rows, k, m, name)
                out[f"prefill_{name}{tag}_m{m}_{rows}x{k}"] = r
        del wq, imgs
    # Reference point, not this library: the vendor's dense fp16 GEMM (torch.mm,
    # served by hipBLASLt) on the same shapes with fp16 weights in HBM (4 rotated
    # copies), timed eagerly with events on the bench stream.
    for rows, k in ((12288, 4096), (8192, 4096)):
        wl = [b.normal((rows, k)).to(torch.float16) for _ in range(4)]
        for m in (128, 2048):
            a = b.normal((m, k)).to(torch.float16)
            reps = max(24, 4800 // m)
            with torch.cuda.stream(b.stream):
                for w in wl:
                    torch.mm(a, w.t())
                torch.cuda.synchronize()
                ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                ev0.record(b.stream)
                for i in range(reps):
                    torch.mm(a, wl[i % len(wl)].t())
                ev1.record(b.stream)
            torch.cuda.synchronize()
            us = ev0.elapsed_time(ev1) * 1e3 / reps
            out[f"library_fp16_gemm_m{m}_{rows}x{k}"] = {
                "us": round(us, 2), "TFLOP/s": round(2.0 * m * rows * k / us / 1e6, 1),
                "blas": str(torch.backends.cuda.preferred_blas_library()),
                "note": "torch.mm fp16 (hipBLASLt), fp16 weights: a reference rate on this box, not this library"}
        del wl
    return out


def cpu_stack_us(cpu: CpuBaseline, stack, m: int, head: bool) -> tuple[float, str]:
    """CPU time (us) of one step of the stack's projections over m tokens:
    every projection of one DeltaNet layer and one attention layer timed at
    full size (oracle dequantisation + fp32 BLAS, median of the CpuBaseline's
    runs) and scaled by the layer counts, plus the head on one token timed on
    1/8 of its rows and scaled by 8."""
    from qwowl35_amd import qwen35

    hp = stack.hp
    kinds = {}
    for il in range(hp.transformer_layers):
        kinds.setdefault(qwen35.is_attention_layer(hp, il), il)
    total, parts = 0.0, []
    for attn, il in kinds.items():
        n_layers = sum(1 for j in range(hp.transformer_layers) if qwen35.is_attention_layer(hp, j) == attn)
        t = 0.0
        for p in qwen35.mixer_projections(hp, il) + qwen35.ffn_projections(hp):
            w = stack.layers[il][p.name]
            t_dq, t_mm = (cpu.matmul if m > 1 else cpu.gemv)(w.type_id, host_bytes(w), w.rows, w.k, m)
            t += t_dq + t_mm
        total += n_layers * t
        parts.append(f"{'attention' if attn else 'DeltaNet'} layer {t * 1e3:.0f} ms x {n_layers}")
    if head:
        rows = hp.vocab // 8
        w = stack.head
        raw = host_bytes(w)[: rows * b_rt().row_bytes(w.type_id, w.k)]
        t_dq, t_mv = cpu.gemv(w.type_id, raw, rows, w.k, 1)
        total += 8 * (t_dq + t_mv)
        parts.append(f"head {8e3 * (t_dq + t_mv):.0f} ms (1/8 of the rows x 8)")
    return total * 1e6, ", ".join(parts)


def b_rt():
    from qwowl35_amd import runtime

    return runtime


def bench_stack(b: Bench, cpu: CpuBaseline | None) -> dict:
    """Config 5: the 32-layer Qwen3.5-9B decode-step projection stack as one
    recorded plan (hipGraph), in the reference's dispatch order: per layer the
    q8_0 mixer input projections (merged into one launch), the q8_0 output
    projection (+= residual), the GF4 fused gate/up/SwiGLU and the GF4 down
    projection (+= residual); then the Q4_K LM head.  The runtime's buffer
    sharing (one output buffer per role, no AWQ: the reference folds it into
    the norms) -- the same plan qw35_hip_runtime_eval_step records.  Every layer
    has its own weight buffers (5.2 GB per step).  Then one prefill chunk of
    128 tokens (the reference server's default chunk) over the same stack, as
    qw35_hip_runtime_eval_chunk records it: fp32 activations on the prefill
    matmul, the head on the last token."""
    from qwowl35_amd import qwen35

    hp = qwen35.QWEN35_9B
    stack = qwen35.ProjectionStack.synthetic(hp, distinct=False, head_tile_rows=16384, device=b.dev)
    total = stack.weight_bytes
    out = {}
    for nb in (1, 8):
        bufs = qwen35.StepBuffers.make(hp, nb, b.gen, awq=False, shared_outputs=True)
        bufs.ffn_norm = bufs.norm
        plan = qwen35.build_plan(stack, bufs)
        us = b.time_plan(plan, 20) * 1e3
        line = {"gemvs": len(plan), "weight_bytes": int(total), "us_per_step": round(us, 1),
                "us_per_token": round(us / nb, 1), "roofline": hbm_roofline(total, us)}
        if cpu is not None:
            cpu_us, how = cpu_stack_us(cpu, stack, nb, head=True)
            line["cpu_baseline"] = cpu.record(round(cpu_us / nb, 1), "us/token",
                                              f"9B projection stack at batch {nb}, timed per projection: {how}; "
                                              f"divided by the batch")
        out[f"decode_stack_9b_b{nb}"] = line
        plan.close()
        del bufs
    n = 128
    bufs = qwen35.StepBuffers.make(hp, n, b.gen, awq=False, shared_outputs=True)
    bufs.ffn_norm = bufs.norm
    ws = qwen35.chunk_workspace(stack, n)
    plan = qwen35.build_chunk_plan(stack, bufs, ws)
    us = b.time_plan(plan, 5) * 1e3
    flops = qwen35.chunk_flops(hp, n)
    line = {"n_tokens": n, "ops": len(plan), "us_per_chunk": round(us, 1), "us_per_token": round(us / n, 2),
            "tokens_per_s": round(n / us * 1e6, 1), "flops": flops,
            "roofline": mfma_roofline(flops, us, "gf4_prefill_f16_kernel (GF4 / q8_0 weights, fp32 activations)")}
    if cpu is not None:
        cpu_us, how = cpu_stack_us(cpu, stack, n, head=True)
        line["cpu_baseline"] = cpu.record(round(cpu_us / n, 1), "us/token",
                                          f"9B projection stack over a 128-token chunk, timed per projection: {how}; "
                                          f"divided by the tokens")
    out["prefill_chunk_9b_m128"] = line
    plan.close()
    del stack, bufs, ws
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4000)
    ap.add_argument("--warmup", type=int, default=400)
    ap.add_argument("--copies", type=int, default=32, help="distinct GF4 weight copies rotated (>= 24)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--headline-only", action="store_true", help="skip the extra configs (= --extras none)")
    ap.add_argument("--extras", default="all",
                    help="comma list of extra configs: gf4,q8,q4k,q6k,prefill,stack,codecs (all = every one "
                         "but codecs; none)")
    ap.add_argument("--cpu-reps", type=int, default=5)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures one GPU; multi-GPU runs are not part of it (--gpus 1)"}),
              flush=True)
        return 2

    import torch

    from qwowl35_amd import runtime as rt

    b = Bench(torch, rt)
    cpu = None if args.no_cpu else CpuBaseline(cpu_threads(), args.cpu_reps)
    rows, k = 12288, 4096
    log(f"config 1: GF4 {rows}x{k} b1, {args.copies} copies, {args.steps} timed launches")
    weights = [b.weight(rt.TYPE_GF4, rows, k) for _ in range(args.copies)]
    x = b.normal((1, k))
    y = torch.zeros((1, rows), dtype=torch.float32, device=b.dev)
    # plain device copy of a known size: the calibration kernel of the PMC traffic passes
    calib = weights[0].storage.clone()
    torch.cuda.synchronize()
    del calib

    ms, launches = b.time_launches(gemv_calls(rt, weights, x, y), args.steps, args.warmup)
    kern = rt.gemv_kernel(weights[0], 1)["name"]
    algo = gemv_bytes(rt, rt.TYPE_GF4, rows, k, 1)
    value = algo / (ms * 1e-3) / 1e9
    log(f"GF4 b1: {ms * 1e3:.3f} us/launch, {value:.0f} GB/s ({kern})")

    extra = {"headline_kernel": kern}
    ceil = stream_ceiling(b, [w.storage for w in weights])
    extra["stream_read_ceiling"] = ceil
    extra["gf4_b1_frac_of_stream_ceiling"] = round(value / ceil["GB/s_25MB"], 4)
    # Best frac of 8 TB/s one dependent launch of these bytes could reach here:
    # the measured per-launch floor plus the bytes at the 1 GiB read rate.
    best_us = ceil["launch_floor_us"] + algo / (ceil["GB/s_1GiB"] * 1e3)
    extra["single_launch_frac_bound"] = round(algo / (best_us * 1e3) / HBM_PEAK_GBS, 4)
    want = set() if args.headline_only or args.extras == "none" else (
        {"gf4", "q8", "q4k", "q6k", "prefill", "stack"} if args.extras == "all" else set(args.extras.split(",")))

    cpu_line = None
    if cpu is not None:
        t_dq, t_mv = cpu.gemv(rt.TYPE_GF4, host_bytes(weights[0]), rows, k, 1)
        cpu_line = cpu.record(round(algo / (t_dq + t_mv) / 1e9, 3), "GB/s",
                              f"GF4 12288x4096 b1 at full size: dequant {t_dq * 1e3:.1f} ms + matvec "
                              f"{t_mv * 1e3:.2f} ms per call")
    if "gf4" in want:
        extra.update(bench_gf4_extra(b, weights, cpu, args.steps, args.warmup))
    del weights
    if "q8" in want:
        extra.update(bench_q8_layer(b, cpu, args.steps, args.warmup))
    if "q4k" in want:
        extra.update(bench_q4k(b, cpu, args.steps, args.warmup))
    if "q6k" in want:
        extra.update(bench_q6k_head(b, args.steps, cpu))
    if "codecs" in want:
        extra.update(bench_codecs(b, args.steps // 4, args.warmup // 2))
    if "prefill" in want:
        extra.update(bench_prefill(b, cpu))
    if "stack" in want:
        extra.update(bench_stack(b, cpu))
    for key, v in extra.items():
        log(f"{key}: {v}")

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
        "dtype": DTYPE,
        "data": "synthetic",
        "config": {"workload": "gf4_matvec_b1_12288x4096", "rows": rows, "k": k, "batch": 1,
                   "weight_copies": args.copies},
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": traffic_for(kern)},
        "cpu_baseline": cpu_line,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
