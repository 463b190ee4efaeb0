#!/usr/bin/env python3
"""Benchmark of the MI355X W4A16 grouped-expert MoE layer.

Metric: weight-bandwidth GB/s = touched-expert packed weight +
scale bytes / time per call (the reference's definition,
bench/bench_moe.py:250-263, :742-744), as a fraction of the 8 TB/s HBM peak;
TFLOP/s = 2*M*topk*(2*N*K + K*N) / time at the prefill sizes.

One "step" is one fused_experts_w4a16 call (sort, w13+SiLU*up, w2, combine)
on one batch of synthetic input already resident in HBM.  The workload of the
headline value is BASELINE.json's configs[1]: E=256, top-10, K=3072, N=1024,
group 32, M=16 tokens, uniform routing.  The other configurations are reported
in "configs".

Timing (the reference's protocol, bench/bench_moe.py:475-512, on a graph of
K calls): W eager warm-up calls; the K calls captured as one HIP graph (chunks
of at most 2048 calls) that cycles through several routing/hidden sets, so
the touched weights exceed the 256 MB Infinity Cache several times over;
warm-up replays of that graph until at least 200 ms of device time has run
(a GPU that was idle runs its first ~15 ms of work up to 15 % slower while its
clocks ramp up); then R timed replays back to back, each bracketed by events
on the launch stream, the whole timed region bracketed by device
synchronisation.  The reported time per call is the p50 replay / K.

Per-kernel durations come from graphs of one stage at a time
(w4a16_moe_run_stage_ex, with the dispatch tuning the call itself uses) that
cycle over the same sets several times, timed with events on the stream the
kernels run on; the dominant kernel's algorithmic bytes / duration is the
roofline "achieved" figure.

Each configuration row also carries "router": the device time of the router
step in front of the layer (w4a16_moe_router_topk_softmax: fp32 logits
[M, 256] -> top-10 ids and softmax weights, bench/bench_moe.py:225-230) and its
logits+outputs bytes per second.

The CPU baseline is the oracle's PyTorch dequant reference
(oracle/moe_oracle.py, a restatement of bench/bench_moe.py:277-303) timed on
the host on a bounded sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 1]
                       [--no-sweep] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import ctypes
import importlib
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

METRIC = "weight-BW GB/s (% of HBM peak) at M=1..1024; bf16 TFLOP/s at M=4096 prefill"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
MALL_BYTES = 256 * 2**20       # Infinity Cache
# The reference's published number for this metric at configs[1] (M=16):
# 226.3 GB/s on NVIDIA GB10 (results/showdown2.json:1104; README.md:62-70).
REFERENCE_GBS_M16 = 226.3
STAGES = ("align", "w13", "w2", "combine")
WARM_MS = 200.0                # device time of warm-up replays before the timed ones
TIMED_MS = 250.0               # device time the timed replays aim for ...
MIN_REPLAYS, MAX_REPLAYS = 9, 50   # ... within these replay counts
CALIB_BYTES = 2**30            # plain device copy: PMC byte-counter scale and measured copy BW
# Kernel-name fragments of the dominant kernels in rocprofv3 counter files,
# per stage and path (dequant-GEMV for few pairs per expert, MFMA tiles else).
KERNEL_KEYS = {("w13", "gemv"): "gemv_kernel<0,", ("w2", "gemv"): "gemv_kernel<1,",
               ("w13", "mfma"): "mfma_kernel<0,", ("w2", "mfma"): "mfma_kernel<1,",
               ("w13", "mixed"): "mixed_kernel<0,", ("w2", "mixed"): "mixed_kernel<1,"}
KERNEL_LABELS = {"gemv": "dequant-GEMV (gemv_kernel)", "mfma": "dequant-MFMA tiles (mfma_kernel)",
                 "mixed": "GEMV and MFMA work items in one launch (mixed_kernel)"}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Workload:
    """One configuration: weights shared, n_sets routing/hidden sets."""

    def __init__(self, pkg, synth, shape, weights, cfg, dev, n_sets=None):
        import torch

        self.pkg, self.shape, self.cfg, self.dev = pkg, shape, cfg, dev
        self.w13, self.w2, self.s13, self.s2 = weights
        M, E = cfg.M, shape.E
        expect = min(E, M * shape.topk) * shape.bytes_per_expert
        if n_sets is None:
            n_sets = min(64, max(8, math.ceil(4 * MALL_BYTES / expect)))
        self.sets = []
        for i in range(n_sets):
            x = synth.make_hidden(M, shape.K, dev, seed=i)
            tw, ti = synth.make_routing(M, E, shape.topk, dev, seed=i, skewed=cfg.skewed,
                                        bias_seed=0)
            self.sets.append((x, tw, ti))
        self.touched = [synth.touched_experts(s[2], E) for s in self.sets]
        # the dispatch choices fused_experts_w4a16 makes for this M (tuned
        # table entry when one exists for the device, else built-in)
        self.tuning = pkg.tuning.select(M, E, shape.N, shape.K, shape.group, dev)
        self.bytes = [n * shape.bytes_per_expert for n in self.touched]
        self.w13_bytes = [n * shape.w13_bytes_per_expert for n in self.touched]
        self.w2_bytes = [n * shape.w2_bytes_per_expert for n in self.touched]
        torch.cuda.synchronize()

    def call(self, i):
        x, tw, ti = self.sets[i]
        return self.pkg.fused_experts_w4a16(x, self.w13, self.w2, self.s13, self.s2, tw, ti,
                                            self.shape.group)

    # ---- whole-call timing (the headline) ----------------------------------
    def time_calls(self, steps, warmup, replays=None, warm_ms=WARM_MS):
        """p50 over `replays` timed replays of one graph of `steps` calls."""
        import torch

        n = len(self.sets)
        for j in range(warmup):
            self.call(j % n)
        torch.cuda.synchronize()
        # The timed calls are captured as one graph of exactly `steps` calls
        # cycling through the sets (chunks of at most kMaxGraph calls), as a
        # serving loop captures a whole forward pass.
        kMaxGraph = 2048
        chunks = [min(kMaxGraph, steps - s0) for s0 in range(0, steps, kMaxGraph)]
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            for i in range(n):
                self.call(i)
        torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        graphs = {}
        for c in sorted(set(chunks)):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for i in range(c):
                    self.call(i % n)
            graphs[c] = g

        def replay():
            for c in chunks:
                graphs[c].replay()

        ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
        # Warm-up replays until warm_ms of device time has run.
        a, b = ev(), ev()
        a.record()
        replay()
        b.record()
        torch.cuda.synchronize()
        one_ms = a.elapsed_time(b)
        n_warm = max(2, math.ceil(warm_ms / max(one_ms, 1e-3)))
        for _ in range(n_warm - 1):
            replay()
        if replays is None:
            replays = min(MAX_REPLAYS, max(MIN_REPLAYS, math.ceil(TIMED_MS / max(one_ms, 1e-3))))
        evs = [ev() for _ in range(replays + 1)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        evs[0].record()
        for i in range(replays):
            replay()
            evs[i + 1].record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        per = [evs[i].elapsed_time(evs[i + 1]) for i in range(replays)]
        p50 = sorted(per)[len(per) // 2]
        nbytes = sum(self.bytes[i % n] for c in chunks for i in range(c))
        del graphs
        self.pkg.release_graph_workspaces()
        return {"elapsed_ms": p50, "wall_s": wall, "steps": steps, "bytes": nbytes,
                "replays": replays, "warmup_replays": n_warm,
                "replay_ms": {"p50": round(p50, 4), "min": round(min(per), 4),
                              "max": round(max(per), 4), "mean": round(sum(per) / len(per), 4)}}

    # ---- per-stage timing ---------------------------------------------------
    def stage_launches(self):
        """Kernel launches of each stage (sort, w13, w2, combine) of this M."""
        shape = self.shape
        ts = None if self.tuning is None else self.tuning.to_struct()
        return self.pkg._lib.stage_launches(self.cfg.M, shape.topk, shape.E, shape.N, shape.K,
                                            shape.group, ts)

    def time_stages(self, replays, timed=5):
        """Average device time per launch of each stage, over all sets (None
        for a stage that launches no kernel at this M)."""
        import torch

        lib = self.pkg._lib.lib()
        L = self.pkg._lib
        shape, M = self.shape, self.cfg.M
        ts = None if self.tuning is None else self.tuning.to_struct()
        tptr = None if ts is None else ctypes.byref(ts)
        ws_bytes = L.workspace_size_ex(M, shape.topk, shape.E, shape.N, shape.K, shape.group, ts)
        wss = [torch.empty(ws_bytes, dtype=torch.uint8, device=self.dev) for _ in self.sets]
        outs = [torch.empty(M, shape.K, dtype=torch.bfloat16, device=self.dev)
                for _ in self.sets]

        def args(i):
            x, tw, ti = self.sets[i]
            return (x.data_ptr(), x.stride(0), self.w13.data_ptr(), self.w2.data_ptr(),
                    self.s13.data_ptr(), self.s2.data_ptr(), tw.data_ptr(), ti.data_ptr(),
                    M, shape.topk, shape.E, shape.N, shape.K, shape.group,
                    outs[i].data_ptr(), outs[i].stride(0), wss[i].data_ptr(), ws_bytes,
                    torch.cuda.current_stream().cuda_stream)

        for i in range(len(self.sets)):
            L.check(lib.w4a16_moe_fused_experts_ex(*args(i), tptr))
        torch.cuda.synchronize()
        launches = self.stage_launches()
        result = {}
        for stage, name in enumerate(STAGES):
            if launches[stage] == 0:
                result[name] = None
                continue
            g = torch.cuda.CUDAGraph()
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                for i in range(len(self.sets)):
                    L.check(lib.w4a16_moe_run_stage_ex(stage, *args(i), tptr))
            torch.cuda.current_stream().wait_stream(s)
            # `replays` cycles over the sets in one graph: the replay overhead
            # is spread over all of its launches
            with torch.cuda.graph(g):
                for _ in range(replays):
                    for i in range(len(self.sets)):
                        L.check(lib.w4a16_moe_run_stage_ex(stage, *args(i), tptr))
            g.replay()
            evs = [torch.cuda.Event(enable_timing=True) for _ in range(timed + 1)]
            torch.cuda.synchronize()
            evs[0].record()
            for k in range(timed):
                g.replay()
                evs[k + 1].record()
            torch.cuda.synchronize()
            per = sorted(evs[k].elapsed_time(evs[k + 1]) for k in range(timed))
            result[name] = per[timed // 2] / (replays * len(self.sets))
            del g
        del wss, outs
        return result


def time_router(wl, replays):
    """Average device time of the router step (logits -> top-k ids and weights)
    at this configuration's M, graph-replayed over as many logits sets."""
    import torch

    shape, M = wl.shape, wl.cfg.M
    sets = []
    for i in range(len(wl.sets)):
        g = torch.Generator(device=wl.dev).manual_seed(17000 + M + i)
        sets.append(torch.randn((M, shape.E), generator=g, device=wl.dev))
    outs = [(torch.empty((M, shape.topk), device=wl.dev),
             torch.empty((M, shape.topk), dtype=torch.int32, device=wl.dev)) for _ in sets]
    for x, o in zip(sets, outs):
        wl.pkg.router_topk_softmax(x, shape.topk, out=o)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):  # `replays` cycles in one graph
        for _ in range(replays):
            for x, o in zip(sets, outs):
                wl.pkg.router_topk_softmax(x, shape.topk, out=o)
    g.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    g.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / (replays * len(sets))
    nbytes = M * shape.E * 4 + M * shape.topk * 8
    return {"us": round(ms * 1e3, 3), "GB_s": round(nbytes / (ms * 1e-3) / 1e9, 2)}


def summarize(wl, t, stages):
    shape, M = wl.shape, wl.cfg.M
    sec = t["elapsed_ms"] * 1e-3
    gbs = t["bytes"] / sec / 1e9
    tflops = shape.flops(M) * t["steps"] / sec / 1e12
    avg_touched = sum(wl.touched) / len(wl.touched)
    row = {
        "config": wl.cfg.index,
        "M": M,
        "routing": "skewed" if wl.cfg.skewed else "uniform",
        "sets": len(wl.sets),
        "touched_experts_avg": round(avg_touched, 2),
        "us_per_call": round(t["elapsed_ms"] * 1e3 / t["steps"], 3),
        "GB_s": round(gbs, 2),
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "TFLOP_s": round(tflops, 3),
        "pct_bf16_peak": round(100 * tflops / BF16_PEAK_TFLOPS, 3),
        "tuning": "built-in" if wl.tuning is None else wl.tuning.to_dict(),
        "timing": {"calls_per_replay": t["steps"], "timed_replays": t["replays"],
                   "warmup_replays": t["warmup_replays"], "replay_ms": t["replay_ms"]},
    }
    if stages is not None:
        row["stage_us"] = {k: (None if v is None else round(v * 1e3, 3))
                           for k, v in stages.items()}
        w13 = sum(wl.w13_bytes) / len(wl.w13_bytes)
        w2 = sum(wl.w2_bytes) / len(wl.w2_bytes)
        row["stage_GB_s"] = {"w13": round(w13 / (stages["w13"] * 1e-3) / 1e9, 2),
                             "w2": round(w2 / (stages["w2"] * 1e-3) / 1e9, 2)}
    return row


def parity_row(wl, cpu_budget_s, max_calls=9):
    """Set 0 of a workload against the oracle: the GPU output against the
    PyTorch CPU dequant reference (bench/bench_moe.py:271-303, errors as
    bench/bench_moe.py:520-527 computes them, plus max-abs over max|ref|),
    that reference's CPU time (p50 of as many calls as fit cpu_budget_s, at
    least one), and the expert sort against the oracle's
    moe_align_block_size (kernels/w4a16_moe.py:187-290), bit for bit."""
    import numpy as np
    import torch

    from oracle import moe_oracle as orc

    shape = wl.shape
    x, tw, ti = wl.sets[0]
    out = wl.call(0)
    torch.cuda.synchronize()
    out32 = out.float().cpu()
    xc, twc, tic = x.cpu(), tw.cpu(), ti.cpu()
    times, ref = [], None
    while not times or (sum(times) < cpu_budget_s and len(times) < max_calls):
        t0 = time.perf_counter()
        ref = orc.moe_reference(xc, *wl.wcpu, twc, tic, shape.group, out_dtype=None)
        times.append(time.perf_counter() - t0)
    cpu_s = sorted(times)[len(times) // 2]
    max_ref = float(ref.abs().max())
    mab = orc.max_abs(out32, ref)
    # The sort the fused call runs (block 16), standalone, and the one inside
    # the call's workspace when the call runs it (M above the GEMV-only bound).
    want = orc.moe_align_block_size(tic.numpy(), wl.pkg._lib.FUSED_BLOCK_M, shape.E)
    got = wl.pkg.moe_align_block_size_full(ti, wl.pkg._lib.FUSED_BLOCK_M, shape.E)
    torch.cuda.synchronize()
    routing_exact = all(np.array_equal(g.cpu().numpy(), w) for g, w in zip(got[:4], want[:4]))
    internal = None
    if wl.stage_launches()[0] > 0:
        ws, off = wl.pkg.workspace_tensor(x, ti, wl.w13, wl.w2, shape.group, tuning=wl.tuning)
        em, nb = want[0].size, want[1].size
        fields = (ws[off[0]: off[0] + 4 * em], ws[off[1]: off[1] + 4 * nb],
                  ws[off[2]: off[2] + 4], ws[off[3]: off[3] + 4 * (shape.E + 1)])
        internal = all(np.array_equal(f.view(torch.int32).cpu().numpy(), w)
                       for f, w in zip(fields, want[:4]))
    return {
        "parity": {"rel_l2": orc.rel_l2(out32, ref), "max_abs": mab, "max_ref": max_ref,
                   "max_abs_over_max_ref": mab / max_ref if max_ref else None,
                   "routing_bit_exact": routing_exact, "internal_sort_bit_exact": internal,
                   "oracle": "oracle.moe_reference (fp32, bf16-rounded dequantized weights), "
                             "routing set 0"},
        "cpu": {"us_per_call": round(cpu_s * 1e6, 1), "cores": torch.get_num_threads(),
                "calls": len(times), "kind": "port"},
    }


def cpu_model() -> str:
    """The host CPU's model name (Linux /proc/cpuinfo), else the architecture."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(wl, seconds_target=15.0, max_iters=10):
    """Time the oracle's CPU dequant reference on set 0 of the workload."""
    import torch

    from oracle import moe_oracle as orc

    threads = torch.get_num_threads()
    x, tw, ti = (t.cpu() for t in wl.sets[0])
    w = wl.wcpu
    gpu_out = wl.call(0).float().cpu()
    t0 = time.perf_counter()
    ref = orc.moe_reference(x, *w, tw, ti, wl.shape.group)  # warmup
    times = [time.perf_counter() - t0]
    while len(times) < max_iters and sum(times[1:]) < seconds_target:
        t0 = time.perf_counter()
        ref = orc.moe_reference(x, *w, tw, ti, wl.shape.group)
        times.append(time.perf_counter() - t0)
    timed = sorted(times[1:]) if len(times) > 1 else times
    p50 = timed[len(timed) // 2]
    nbytes = wl.bytes[0]
    ref32 = orc.moe_reference(x, *w, tw, ti, wl.shape.group, out_dtype=None)
    return {
        "value": round(nbytes / p50 / 1e9, 4),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle.moe_reference (PyTorch CPU dequant reference) on routing set 0 of "
                   f"config {wl.cfg.index} (M={wl.cfg.M}, {wl.touched[0]} touched experts), "
                   f"1 warmup + {len(timed)} timed calls, p50 {p50 * 1e3:.1f} ms; each "
                   f"config row's \"cpu\" field times the same reference on that config "
                   f"(config 0, M=1, is the one BASELINE.md names)"),
        "cpu": cpu_model(),
        "host_cpus": os.cpu_count(),
        "gpu_vs_cpu_rel_l2": orc.rel_l2(gpu_out, ref32),
        "gpu_vs_cpu_max_abs": orc.max_abs(gpu_out, ref32),
    }


def calibration_copy(dev):
    """One plain device-to-device copy of CALIB_BYTES, for PMC calibration."""
    import torch

    a = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    del a, b


def measured_copy_bw(dev, nbytes=CALIB_BYTES, reps=5):
    """A plain device-to-device copy of nbytes, best of reps: (read + written
    bytes) / time, the measured HBM figure reported beside the 8 TB/s peak."""
    import torch

    a = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    a.fill_(1)
    b.copy_(a)
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(reps):
        st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        st.record()
        b.copy_(a)
        en.record()
        torch.cuda.synchronize()
        best = min(best, st.elapsed_time(en) * 1e-3)
    del a, b
    torch.cuda.empty_cache()
    return {"GB_s": round(2 * nbytes / best / 1e9, 1), "bytes_copied": nbytes,
            "note": "torch device-to-device copy, (read + written bytes) / time, best of "
                    f"{reps}"}


def measured_dense_gemm(dev, m=40960, n=2048, k=3072, warm_ms=300.0, reps=20):
    """A plain bf16 GEMM (torch.matmul, hipBLASLt) with the w13 launch's FLOPs
    at configs[4] (M*topk rows, 2N columns, K deep), run back to back for
    warm_ms first so the board reaches the clock it sustains under MFMA load;
    p50 of reps timed calls.  The library's dense rate at that clock, reported
    beside the 2.5 PFLOP/s nominal peak."""
    import torch

    g = torch.Generator(device=dev).manual_seed(0)
    a = torch.randn(m, k, device=dev, dtype=torch.bfloat16, generator=g)
    b = torch.randn(k, n, device=dev, dtype=torch.bfloat16, generator=g)
    c = torch.empty(m, n, device=dev, dtype=torch.bfloat16)
    torch.matmul(a, b, out=c)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < warm_ms:
        for _ in range(10):
            torch.matmul(a, b, out=c)
        torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        st.record()
        torch.matmul(a, b, out=c)
        en.record()
        torch.cuda.synchronize()
        times.append(st.elapsed_time(en) * 1e-3)
    del a, b, c
    torch.cuda.empty_cache()
    p50 = sorted(times)[len(times) // 2]
    flop = 2.0 * m * n * k
    return {"TFLOP_s": round(flop / p50 / 1e12, 1), "us_per_gemm": round(p50 * 1e6, 2),
            "frac_of_peak": round(flop / p50 / 1e12 / BF16_PEAK_TFLOPS, 4),
            "shape": [m, n, k],
            "note": "torch.matmul bf16 (hipBLASLt), the w13 FLOPs of configs[4] as one dense "
                    f"GEMM, p50 of {reps} after {warm_ms:.0f} ms of back-to-back calls"}


# L2 -> memory request counters by size: bytes = size x requests, no
# calibration needed.  TCC_EA0_RDREQ_sum / TCC_EA0_WRREQ_sum count requests of
# every size (reads: 32, 64 or 128 bytes; writes: 32 or 64 bytes).
BYTE_COUNTERS = ("TCC_EA0_RDREQ_32B_sum", "TCC_EA0_RDREQ_64B_sum", "TCC_EA0_RDREQ_128B_sum",
                 "TCC_EA0_RDREQ_sum", "TCC_EA0_WRREQ_64B_sum", "TCC_EA0_WRREQ_sum")


def traffic_from_pmc(pmc_dirs, kernel_key):
    """HBM bytes per launch of a kernel from rocprofv3 --pmc CSV output.

    pmc_dirs: directories holding *_counter_collection.csv of runs of this
    command, either
      * the request counters by size (BYTE_COUNTERS): read bytes = 32 n32 +
        64 n64 + 128 n128, written bytes = 64 n64 + 32 (n - n64); or
      * a FETCH_SIZE run and a WRITE_SIZE run of a command that also ran
        calibration_copy(): each scaled by CALIB_BYTES / (its reading on the
        copy kernel).
    The request counters win when both are present; the calibrated figure is
    kept in the detail for comparison.  Returns (bytes, detail) or
    (None, reason).
    """
    import csv
    import glob

    sums, req = {}, {}
    for d in pmc_dirs:
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            rows = list(csv.DictReader(open(path)))
            for name in ("FETCH_SIZE", "WRITE_SIZE"):
                sel = [r for r in rows if r["Counter_Name"] == name]
                if not sel:
                    continue
                copies = [float(r["Counter_Value"]) for r in sel
                          if "copyBuffer" in r["Kernel_Name"]]
                mine = [float(r["Counter_Value"]) for r in sel if kernel_key in r["Kernel_Name"]]
                if not copies or not mine:
                    continue
                calib_kib = max(copies)
                factor = (CALIB_BYTES / 1024.0) / calib_kib
                sums[name] = (sum(mine) / len(mine) * 1024.0 * factor, factor, len(mine))
            for name in BYTE_COUNTERS:
                mine = [float(r["Counter_Value"]) for r in rows
                        if r["Counter_Name"] == name and kernel_key in r["Kernel_Name"]]
                if mine:
                    req[name] = (sum(mine) / len(mine), len(mine))
    detail = {}
    total = None
    if all(n in req for n in BYTE_COUNTERS):
        rd = (32 * req["TCC_EA0_RDREQ_32B_sum"][0] + 64 * req["TCC_EA0_RDREQ_64B_sum"][0] +
              128 * req["TCC_EA0_RDREQ_128B_sum"][0])
        n64 = req["TCC_EA0_WRREQ_64B_sum"][0]
        wr = 64 * n64 + 32 * (req["TCC_EA0_WRREQ_sum"][0] - n64)
        total = rd + wr
        detail["request_counters"] = {"read_bytes": int(rd), "written_bytes": int(wr),
                                      "dispatches": req["TCC_EA0_RDREQ_sum"][1]}
    if "FETCH_SIZE" in sums and "WRITE_SIZE" in sums:
        calibrated = sums["FETCH_SIZE"][0] + sums["WRITE_SIZE"][0]
        detail.update({k: {"bytes": int(v[0]), "scale": round(v[1], 4), "dispatches": v[2]}
                       for k, v in sums.items()})
        if total is None:
            total = calibrated
    if total is None:
        return None, ("no request-counter or FETCH_SIZE/WRITE_SIZE readings for the kernel "
                      "(and the copy)")
    return int(total), detail


def mfma_pair_share(wl):
    """Fraction of the (token, expert) pairs of set 0 that the call's dispatch
    sends to the MFMA kernels (the rest run on the dequant-GEMV kernels)."""
    import torch

    shape, M = wl.shape, wl.cfg.M
    if wl.tuning is not None:
        t = wl.tuning
        only_max_m, max_tokens = t.gemv_only_max_m, t.gemv_max_tokens
    else:
        t = wl.pkg._lib.default_tuning(M, shape.topk, shape.E, shape.N, shape.K, shape.group)
        only_max_m, max_tokens = t.gemv_only_max_m, t.gemv_max_tokens
    if M <= only_max_m:
        return 0.0
    ids = wl.sets[0][2].reshape(-1).long()
    counts = torch.bincount(ids[(ids >= 0) & (ids < shape.E)], minlength=shape.E)
    total = int(counts.sum())
    return float(counts[counts > max_tokens].sum()) / total if total else 0.0


def stage_roofline(wl, stage, us):
    """Roofline of one stage kernel at its average duration `us` (microseconds).

    The bound is the roof that gives the longer minimum time: HBM (8 TB/s)
    over the touched experts' packed weight + scale bytes, or dense bf16 MFMA
    (2.5 PFLOP/s) over 2 * pairs * (rows x reduction length) FLOPs.
    """
    shape, M = wl.shape, wl.cfg.M
    nbytes = sum(getattr(wl, f"{stage}_bytes")) / len(wl.sets)
    rows_k = 2 * shape.N * shape.K if stage == "w13" else shape.K * shape.N
    flops = 2 * M * shape.topk * rows_k
    share = mfma_pair_share(wl)
    if 0.0 < share < 1.0 and wl.stage_launches()[STAGES.index(stage)] == 1:
        path = "mixed"  # the split dispatch's two kinds of work items, one launch
    else:
        path = "mfma" if share >= 0.5 else "gemv"
    sec = us * 1e-6
    hbm_bound = nbytes / (HBM_PEAK_GBS * 1e9) >= flops / (BF16_PEAK_TFLOPS * 1e12)
    kernel = f"{stage} {KERNEL_LABELS[path]}"
    if hbm_bound:
        achieved, peak, unit = nbytes / sec / 1e9, HBM_PEAK_GBS, "GB/s"
    else:
        achieved, peak, unit = flops / sec / 1e12, BF16_PEAK_TFLOPS, "TFLOP/s"
    return {"bound": "hbm" if hbm_bound else "mfma", "kernel": kernel, "path": path,
            "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "algorithmic_bytes_per_launch": int(nbytes),
            "algorithmic_flops_per_launch": int(flops)}


def trace_from_profile(kernel, config_index):
    """The rocprofv3 kernel-trace average duration (us) recorded in profiles/
    for this kernel/config: every launch of a profiled bench run, cold graph
    launches included."""
    import re

    for path in sorted((ROOT / "profiles").glob("*.md")):
        for line in path.read_text().splitlines():
            m = re.match(r"\s*trace_avg_us\[(\w+), config (\d+)\]:\s*([0-9.]+)", line)
            if m and m.group(1) == kernel and int(m.group(2)) == config_index:
                return float(m.group(3)), str(path.relative_to(ROOT))
    return None, None


def traffic_from_profile(kernel, config_index):
    """The HBM bytes per launch recorded in profiles/ for this kernel/config."""
    import re

    for path in sorted((ROOT / "profiles").glob("*.md")):
        for line in path.read_text().splitlines():
            m = re.match(r"\s*traffic\[(\w+), config (\d+)\]:\s*(\d+)\s*bytes", line)
            if m and m.group(1) == kernel and int(m.group(2)) == config_index:
                return int(m.group(3)), str(path.relative_to(ROOT))
    return None, None


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=256)
    p.add_argument("--warmup", type=int, default=16)
    p.add_argument("--config", type=int, default=1, help="headline config index (0-4)")
    p.add_argument("--sets", type=int, default=None, help="routing sets to cycle through")
    p.add_argument("--no-sweep", action="store_true", help="skip the other configs")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--replays", type=int, default=None,
                   help=f"timed replays of the K-call graph (default: enough for "
                        f"{TIMED_MS:.0f} ms, {MIN_REPLAYS}..{MAX_REPLAYS})")
    p.add_argument("--no-parity", action="store_true",
                   help="skip the per-config oracle comparison and CPU timing")
    p.add_argument("--stage-replays", type=int, default=8)
    p.add_argument("--no-dense-gemm", action="store_true",
                   help="skip the hipBLASLt dense bf16 GEMM reported beside the MFMA peak")
    p.add_argument("--calibrate-copy", action="store_true",
                   help=f"run one {CALIB_BYTES >> 20} MiB device copy first (PMC calibration)")
    p.add_argument("--pmc-dir", action="append", default=[],
                   help="rocprofv3 --pmc output dirs of this command (request counters "
                        "TCC_EA0_RDREQ_*/WRREQ_*, or FETCH_SIZE and WRITE_SIZE with "
                        "--calibrate-copy) to derive roofline.traffic from")
    args = p.parse_args(argv)

    if args.gpus != 1:
        print(f"bench.py runs on one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        return 2
    if os.environ.get("WORLD_SIZE", "1") not in ("", "1"):
        print("bench.py is single-process, single-GPU", file=sys.stderr)
        return 2

    import torch

    pkg = __graft_entry__.load_package()
    synth = importlib.import_module(__graft_entry__.PKG_NAME + ".synth")
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    shape = synth.LayerShape()
    if args.calibrate_copy:
        calibration_copy(dev)
    log(f"device {torch.cuda.get_device_name(0)}; generating weights "
        f"({shape.E * shape.bytes_per_expert / 1e9:.2f} GB)")
    weights = synth.make_weights(shape, dev, seed=0)
    torch.cuda.synchronize()

    wcpu = None if args.no_parity and args.no_cpu_baseline else tuple(t.cpu() for t in weights)

    def parity(w, budget):
        if args.no_parity:
            return {}
        return parity_row(w, budget)

    head_cfg = synth.CONFIGS[args.config]
    wl = Workload(pkg, synth, shape, weights, head_cfg, dev, n_sets=args.sets)
    wl.wcpu = wcpu
    log(f"config {head_cfg.index} ({head_cfg.description}): {len(wl.sets)} sets, "
        f"avg touched experts {sum(wl.touched) / len(wl.touched):.1f}")
    t = wl.time_calls(args.steps, args.warmup, args.replays)
    log(f"timed {t['replays']} replays of {t['steps']} calls after {t['warmup_replays']} "
        f"warm-up replays: {json.dumps(t['replay_ms'])} ms per replay (wall {t['wall_s']:.3f} s)")
    stages = wl.time_stages(args.stage_replays)
    head = summarize(wl, t, stages)
    head["router"] = time_router(wl, 20)
    head.update(parity(wl, 5.0))
    log(f"headline: {json.dumps(head)}")

    dominant = "w13" if stages["w13"] >= stages["w2"] else "w2"
    roofline = stage_roofline(wl, dominant, stages[dominant] * 1e3)
    traffic, traffic_src = None, None
    if args.pmc_dir:
        key = KERNEL_KEYS[(dominant, roofline["path"])]
        traffic, detail = traffic_from_pmc(args.pmc_dir, key)
        traffic_src = {"pmc": detail}
    else:
        traffic, traffic_src = traffic_from_profile(dominant, head_cfg.index)
    roofline.update({"traffic": traffic, "traffic_source": traffic_src,
                     "avg_launch_us": round(stages[dominant] * 1e3, 3),
                     "timing": "stage graph: p50 replay of graphs of the dominant kernel "
                               "alone over the rotating sets / launches, HIP events on "
                               "the launch stream"})
    # The same roofline at the committed kernel trace's average duration (it
    # includes the first, cold launch of each graph), for comparison.
    trace_us, trace_src = trace_from_profile(dominant, head_cfg.index)
    if trace_us:
        rt = stage_roofline(wl, dominant, trace_us)
        roofline["trace"] = {"avg_launch_us": trace_us, "achieved": rt["achieved"],
                             "frac": rt["frac"], "source": trace_src}

    sweep = []
    if not args.no_sweep:
        for cfg in synth.CONFIGS:
            if cfg.index == head_cfg.index:
                sweep.append(head)
                continue
            w = Workload(pkg, synth, shape, weights, cfg, dev)
            w.wcpu = wcpu
            steps = len(w.sets) * (4 if cfg.M <= 64 else 2)
            tt = w.time_calls(steps, min(8, len(w.sets)))
            st = w.time_stages(2)
            row = summarize(w, tt, st)
            row["router"] = time_router(w, 20)
            row.update(parity(w, 5.0 if cfg.M <= 64 else 0.0))
            log(f"config {cfg.index}: {json.dumps(row)}")
            sweep.append(row)
            del w
            torch.cuda.empty_cache()
    for row in sweep:
        if "cpu" in row:
            row["cpu"]["speedup_gpu_vs_cpu"] = round(row["cpu"]["us_per_call"] /
                                                     row["us_per_call"], 1)

    copy_bw = measured_copy_bw(dev)
    log(f"measured device copy: {copy_bw['GB_s']} GB/s")
    dense = None if args.no_dense_gemm else measured_dense_gemm(dev)
    if dense:
        log(f"measured dense bf16 GEMM: {json.dumps(dense)}")
    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU baseline ...")
        cpu = cpu_baseline(wl)
        log(f"cpu baseline: {json.dumps(cpu)}")

    sec = t["elapsed_ms"] * 1e-3
    value = t["bytes"] / sec / 1e9
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": t["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(t["elapsed_ms"] / t["steps"], 6),
        "timing": {"protocol": ("p50 over timed replays of one HIP graph of `steps` calls, "
                                "after `warmup` eager calls and warm-up replays of that graph "
                                f"(>= {WARM_MS:.0f} ms of device time); replays back to back, "
                                "events on the launch stream, device synchronisation around "
                                "the timed region"),
                   "timed_replays": t["replays"], "warmup_replays": t["warmup_replays"],
                   "replay_ms": t["replay_ms"]},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(value / REFERENCE_GBS_M16, 3) if head_cfg.index == 1 else None,
        "baseline_ref": "reference kernel, GB10, M=16: 226.3 GB/s (results/showdown2.json:1104)",
        "dtype": "bf16",
        "data": ("synthetic: int4 codes uniform, bf16 scales U[0.005,0.02], x ~ N(0,1) bf16, "
                 "router logits N(0,1) fp32 -> top-10 softmax; routing/hidden sets rotated "
                 "to defeat the 256 MB Infinity Cache"),
        "config": {"workload": f"configs[{head_cfg.index}]: {head_cfg.description}; one MoE "
                               "layer E=256 top-10 K=3072 N=1024 group-32",
                   "M": head_cfg.M, "E": shape.E, "topk": shape.topk, "K": shape.K,
                   "N": shape.N, "group": shape.group, "sets": len(wl.sets),
                   "parallelism": "single GPU"},
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "roofline": roofline,
        "hbm_copy_measured": copy_bw,
        "mfma_dense_measured": dense,
        "cpu_baseline": cpu,
        "configs": sweep,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
