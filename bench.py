"""PairwiseLinear fwd+bwd benchmark on one MI355X (BASELINE.json metric).

Workload ("c2"): PairwiseLinear(128->128, tables=136,
comparisons=6), f32 LUT [136, 64, 128], batch 512, x ~ N(0,1), upstream grad
G ~ N(0,1); one step = forward + fast_sigmoid_odd min-margin STE backward
(y = layer(x); y.backward(G)) with x, thresholds and LUT gradients. Params are
the module's seeded init (seed 0); inputs are synthetic and already in HBM.

Timed regions (both full fwd+bwd of the module API, no work skipped):
  graph  -- the steps captured in HIP graphs (torch.cuda.CUDAGraph), four
            steps per graph, one on each of 4 distinct resident (x, G)
            batches: exactly K steps are timed (K // 4 four-step replays, then
            K % 4 one-step replays), after >= 0.3 s of replays (the GPU clocks
            ramp up under sustained load). This is `value`. A c2 step is a few
            kernels of ~22 us; one graph launch costs 14-19 us of host time
            and ~5 us on the device, so capturing the launch-bound loop four
            steps at a time keeps the GPU busy. The rate with one step per
            graph is reported beside it.
  eager  -- up to 200 plain autograd steps right after the graph phase; the
            three kernels of each step carry HIP events that their own
            dispatch stamps (library hook tropnn_hip_arm_kernel_events, via
            hipExtLaunchKernel), giving the per-kernel average durations used
            for `roofline`. c2's backward is the fused table kernel plus the
            input-gradient scatter kernel.
cpu_baseline: the oracle's torch restatement of the reference torch path, same
step on the host CPU for a bounded number of steps (rank 0, N=1 only).

Other BASELINE.json configs, each its own JSON line (--workload): c3, the f16
eval forward sweep at batch 1 / 64 / 8192; c4, the large f16-LUT layer fwd+bwd
at batch 8192; c5, the EMNIST classifier training step.

Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "PairwiseLinear samples/s fwd+bwd (T=136,C=6,B=512) + achieved HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0
B, I, O, T, C = 512, 128, 128, 136, 6
R = 1 << C
E = 4  # f32 LUT element bytes


def algorithmic_bytes(fused: bool, b: int = B, i: int = I, o: int = O, t: int = T, c: int = C, e: int = E,
                      streamed: bool = False) -> dict[str, int]:
    """Per-launch algorithmic bytes (gather / embedding-bag convention: every
    (item, table) pair moves its LUT row(s) once, streamed tensors and params
    once), split by the kernel that moves them; e = LUT element bytes. Sums to
    the FwdBwd figure of the plan: 148,548,672 B at c2 (the defaults),
    174,323,843,072 B at c4.
      forward: x, anchors + thresholds, one row per (item, table), y, codes;
        streamed (large training shapes, c4): forward_route takes x,
        anchors + thresholds and the codes, forward the rows and y;
    fused backward (narrow rows, c2's path):
      backward_fused: G, codes, current + neighbour rows per (item, table),
        one f32 grad-row contribution per (item, table), grad_lut once,
        grad_thr;
      backward_scatter: x re-read (margins), grad_x, anchors + thresholds;
    general backward (min-margin STE):
      backward_sort: nothing algorithmic (the code sort and G's chunk-major
        copy are implementation choices);
      backward_table: G, codes, current + neighbour rows per (item, table)
        (served from the table's LUT chunk in LDS), one f32 grad-row
        contribution per (item, table), grad_lut once;
      backward_reduce: grad_thr (the partial dots it sums are an
        implementation choice);
      backward_scatter: x re-read (margins), grad_x, anchors + thresholds."""
    r = 1 << c
    fwd = 4 * b * i + 20 * t * c + e * b * t * o + 4 * b * o + b * t
    g_codes_rows = 4 * b * o + b * t + 2 * e * b * t * o
    x_side = 4 * b * i + 4 * b * i + 20 * t * c
    lut_rows = 4 * b * t * o + 4 * t * r * o
    if fused:
        return {"forward": fwd, "backward_fused": g_codes_rows + lut_rows + 4 * t * c, "backward_scatter": x_side}
    head = {"forward": fwd}
    if streamed:
        route = 4 * b * i + 20 * t * c + b * t
        head = {"forward_route": route, "forward": fwd - route}
    return {**head, "backward_sort": 0, "backward_table": g_codes_rows + lut_rows,
            "backward_reduce": 4 * t * c, "backward_scatter": x_side}


def fused_backward() -> bool:
    """Whether the library runs c2's backward as the fused table kernel plus
    the scatter kernel (its workspace then holds 8-byte {gu, r} records)."""
    from tropnn_amd.backends.pairwise_hip import LUT_F32, STE_MIN_MARGIN, load_library

    lib = load_library()  # declares the C signatures
    return lib.tropnn_hip_pairwise_backward_workspace_size(B, I, O, T, C, LUT_F32, STE_MIN_MARGIN) == 8 * T * B


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


KERNEL_SOURCES = (
    "tropnn_amd/csrc/forward.hip",
    "tropnn_amd/csrc/backward.hip",
    "tropnn_amd/csrc/device.hpp",
    "tropnn_amd/csrc/launch.hpp",
    "include/tropnn_hip.h",
)


def source_digest() -> str:
    """sha256 of the kernel sources (kernels, launch planning, the shared
    header; not the C ABI's argument validation) with comments and
    whitespace removed, so that a comment edit does not invalidate a profile
    of the same code."""
    import hashlib
    import re

    h = hashlib.sha256()
    for src in KERNEL_SOURCES:
        text = (ROOT / src).read_text()
        text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
        text = re.sub(r"//[^\n]*", " ", text)
        h.update(" ".join(text.split()).encode())
    return h.hexdigest()


def measured_traffic(kernel: str, workload: str = "c2") -> int | None:
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC
    summary of the workload (profiles/traffic.json for c2,
    profiles/traffic_<workload>.json otherwise: FETCH_SIZE and WRITE_SIZE
    scaled by a calibration copy), used only while the kernel sources
    (comments aside) still hash to the profiled ones; otherwise None."""
    path = ROOT / "profiles" / ("traffic.json" if workload == "c2" else f"traffic_{workload}.json")
    if not path.exists():
        return None
    rec = json.loads(path.read_text())
    if rec.get("source_digest") != source_digest() or kernel not in rec.get("kernels", {}):
        return None
    k = rec["kernels"][kernel]
    return int(k["fetch_bytes"] + k["write_bytes"])


def cpu_baseline(budget_s: float) -> dict:
    """The oracle (torch restatement of the reference torch path) on the host
    cores: same c2 fwd+bwd step, full batch, as many steps as fit the budget."""
    import torch

    from oracle.pairwise_torch import OraclePairwiseLinear

    threads = torch.get_num_threads()
    layer = OraclePairwiseLinear(I, O, tables=T, comparisons=C, seed=0).train()
    x = torch.randn(B, I, generator=torch.Generator().manual_seed(0)).requires_grad_(True)
    g = torch.randn(B, 1, O, generator=torch.Generator().manual_seed(1))

    def step() -> None:
        layer.zero_grad(set_to_none=True)
        x.grad = None
        layer(x).backward(g)

    step()  # warmup
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {
        "value": B / med,
        "unit": "samples/s",
        "cores": threads,
        "kind": "port",
        "sample": f"c2 fwd+bwd, full batch {B}, {len(times)} steps (median {med * 1e3:.1f} ms/step), "
        f"oracle/pairwise_torch.py torch-CPU restatement, torch.set_num_threads={threads}",
    }


C5_LAYER_BYTES = 313_619_648  # the three layers' FwdBwd algorithmic bytes per c5 step (CE and Adam not counted)


def cpu_baseline_c5(budget_s: float) -> dict:
    """The oracle classifier (the three oracle layers, seeds 0, 1, 2) with
    torch Adam on the host cores: the same c5 training step, full batch."""
    import torch
    import torch.nn.functional as F

    from oracle.pairwise_torch import OraclePairwiseLinear
    from tropnn_amd.examples import make_c5_batch

    threads = torch.get_num_threads()
    dims = (784, 128, 128, 10)
    layers = torch.nn.ModuleList(
        [OraclePairwiseLinear(a, b, tables=T, comparisons=C, seed=k) for k, (a, b) in enumerate(zip(dims[:-1], dims[1:]))]
    )
    opt = torch.optim.Adam(layers.parameters(), lr=1e-3)
    x, y = make_c5_batch(512, seed=0)

    def step() -> None:
        opt.zero_grad(set_to_none=True)
        h = x.unsqueeze(1)
        for layer in layers:
            h = layer(h)
        F.cross_entropy(h.squeeze(1), y).backward()
        opt.step()

    step()
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {
        "value": 512 / med,
        "unit": "samples/s",
        "cores": threads,
        "kind": "port",
        "sample": f"c5 train step (3 oracle layers + CE + torch Adam), batch 512, {len(times)} steps "
        f"(median {med * 1e3:.1f} ms/step), torch.set_num_threads={threads}",
    }


def bench_c3(args, dev) -> dict:
    """c3: the c2 layer (128 -> 128, T = 136,
    C = 6) as eval forward only with f16 LUT reads, at batch 1, 64 and 8192:
    time per call (one HIP graph per call, replayed back to back over 4
    resident inputs; at small batches this is the host launch path), the
    forward kernel's own duration (events its dispatch stamps; the device
    latency), and the algorithmic-byte rate, F_eval = 4BI + 20TC + 2BTO + 4BO
    per call."""
    import torch

    from tropnn_amd import PairwiseLinear
    from tropnn_amd.backends.pairwise_hip import arm_kernel_events

    layer = PairwiseLinear(I, O, tables=T, comparisons=C, seed=0, device_lut_dtype="f16").to(dev).eval()
    layer.cache_route_debug = False
    results = {}
    for b in (1, 64, 8192):
        gen = torch.Generator().manual_seed(0)
        xs = [torch.randn(b, I, generator=gen).to(dev) for _ in range(4)]
        with torch.no_grad():
            for x in xs:  # warm the f16 read copy and the allocator
                layer(x)
            torch.cuda.synchronize()
            graphs = []
            for x in xs:
                gph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(gph):
                    layer(x)
                graphs.append(gph)
        torch.cuda.synchronize()
        t0, w = time.perf_counter(), 0
        while w < args.warmup or time.perf_counter() - t0 < 0.3:
            graphs[w % 4].replay()
            w += 1
        torch.cuda.synchronize()
        n = args.steps
        t0 = time.perf_counter()
        for k in range(n):
            graphs[k % 4].replay()
        torch.cuda.synchronize()
        us = (time.perf_counter() - t0) * 1e6 / n
        # the kernel's own duration over eager calls
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(100)]
        stream = torch.cuda.current_stream(dev)
        for e0, e1 in evs:
            e0.record(stream)
            e1.record(stream)
        with torch.no_grad():
            for k, (e0, e1) in enumerate(evs):
                arm_kernel_events("forward", e0, e1)
                layer(xs[k % 4])
        torch.cuda.synchronize()
        kus = sorted(1e3 * e0.elapsed_time(e1) for e0, e1 in evs)[len(evs) // 2]
        algo = 4 * b * I + 20 * T * C + 2 * b * T * O + 4 * b * O
        results[str(b)] = {
            "kernel_us": round(kus, 3),
            "us_per_call": round(us, 3),
            "samples_per_s": round(b / (us * 1e-6), 1),
            "algorithmic_bytes": algo,
            "algorithmic_GBs": round(algo / (us * 1e-6) / 1e9, 1),
        }
        log(f"c3 batch {b}: {us:.2f} us/call, kernel {kus:.2f} us")
    big = results["8192"]
    return {
        "metric": "PairwiseLinear c3 eval forward, f16 LUT reads (128->128, T=136, C=6): samples/s at batch 8192, latency at 1 and 64",
        "value": big["samples_per_s"],
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(big["us_per_call"] * 1e-3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 LUT reads, f32 accumulate",
        "data": "synthetic: x ~ N(0,1), 4 resident inputs per batch size; seeded module init (seed 0)",
        "config": {"workload": "c3: PairwiseLinear(128->128, tables=136, comparisons=6) eval forward, f16 LUT [136,64,128]", "batches": [1, 64, 8192]},
        "per_batch": results,
        "roofline_8192": {"bound": "hbm", "achieved": big["algorithmic_GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(big["algorithmic_GBs"] / HBM_PEAK_GBS, 4)},
    }


def bench_c5(args, dev) -> dict:
    """c5: the pairwise EMNIST classifier
    784 -> 128 -> 128 -> 10 (T = 136, C = 6, seeds 0, 1, 2), batch 512 of
    synthetic sparse inputs, one training step = zero_grad, forward, cross
    entropy (tropnn_amd.cross_entropy: the library's one-launch loss and
    gradient), backward, Adam (lr 1e-3) step (FusedAdam: the library's Adam
    kernel), captured in one HIP graph per resident batch (4, round-robin)
    and timed over replays like c2."""
    import torch

    from tropnn_amd import FusedAdam, cross_entropy
    from tropnn_amd.examples import EmnistPairwiseClassifier, make_c5_batch

    model = EmnistPairwiseClassifier().to(dev).train()
    for layer in model.layers:
        layer.cache_route_debug = False
    opt = FusedAdam(model.parameters(), lr=1e-3)  # the library's one-launch Adam, step counters on the device
    nb = 4
    batches = [tuple(t.to(dev) for t in make_c5_batch(512, seed=k)) for k in range(nb)]

    def step(k: int) -> None:
        x, y = batches[k]
        cross_entropy(model(x), y).backward()
        opt.step()

    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for w in range(max(3, args.warmup)):
            opt.zero_grad(set_to_none=True)
            step(w % nb)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    graphs = []
    for k in range(nb):
        opt.zero_grad(set_to_none=True)
        gph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gph):
            step(k)
        graphs.append(gph)
    torch.cuda.synchronize()
    t0, w = time.perf_counter(), 0
    while w < args.warmup or time.perf_counter() - t0 < 0.3:
        graphs[w % nb].replay()
        w += 1
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        graphs[k % nb].replay()
    torch.cuda.synchronize()
    us = (time.perf_counter() - t0) * 1e6 / args.steps
    log(f"c5 graph {us:.1f} us/step")
    cpu = cpu_baseline_c5(args.cpu_budget) if args.cpu_budget > 0 else None
    value = 512 / (us * 1e-6)
    out = {
        "metric": "EmnistPairwiseClassifier c5 training samples/s (3 PairwiseLinear layers + CE + Adam)",
        "value": round(value, 1),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us * 1e-3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: x = rand * (rand >= 0.8), labels randint(0, 10), 4 resident batches round-robin; "
        "seeded layer init (seeds 0, 1, 2)",
        "config": {
            "workload": "c5: EmnistPairwiseClassifier 784->128->128->10, tables 136, comparisons 6, batch 512, "
            "cross entropy (tropnn_hip_cross_entropy) + Adam lr 1e-3 (tropnn_hip_adam_step), "
            "one HIP graph per training step",
            "batch": 512,
        },
        "layer_algorithmic_bytes_per_step": C5_LAYER_BYTES,
        "layer_algorithmic_GBs": round(C5_LAYER_BYTES / (us * 1e-6) / 1e9, 1),
        "cpu_baseline": cpu,
    }
    if cpu:
        out["speedup_vs_cpu"] = round(value / cpu["value"], 1)
    return out


C4 = {"b": 8192, "i": 1024, "o": 4096, "t": 512, "c": 8}
C4_CPU_BATCH = 8


def cpu_baseline_c4(budget_s: float) -> dict:
    """The oracle's torch restatement of the reference torch path at c4's
    layer (f32 LUT, as that path reads it) on the host cores, fwd + min-margin
    STE bwd, at a reduced batch of 8 items: the full batch of 8192 would hold
    ~64 GiB of saved STE rows (one [B, tables, 4096] f32 neighbour difference
    per route chunk). Reported per sample."""
    import torch

    from oracle.pairwise_torch import OraclePairwiseLinear

    threads = torch.get_num_threads()
    layer = OraclePairwiseLinear(C4["i"], C4["o"], tables=C4["t"], comparisons=C4["c"], seed=0).train()
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(C4_CPU_BATCH, C4["i"], generator=gen).requires_grad_(True)
    g = torch.randn(C4_CPU_BATCH, 1, C4["o"], generator=gen)

    def step() -> None:
        layer.zero_grad(set_to_none=True)
        x.grad = None
        layer(x).backward(g)

    step()
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {
        "value": C4_CPU_BATCH / med,
        "unit": "samples/s",
        "cores": threads,
        "kind": "port",
        "sample": f"c4 layer fwd+bwd at batch {C4_CPU_BATCH} (the full 8192 needs ~64 GiB of saved STE rows), "
        f"f32 LUT, {len(times)} steps (median {med * 1e3:.0f} ms/step), oracle/pairwise_torch.py "
        f"torch-CPU restatement, torch.set_num_threads={threads}",
    }


def bench_c4(args, dev) -> dict:
    """c4: PairwiseLinear(1024 -> 4096, T = 512,
    C = 8) reading an f16 LUT (the RNE copy of the f32 master; 1 GiB), batch
    8192, one step = forward + min-margin STE backward with x, thresholds and
    f32 LUT (2 GiB) gradients. A step takes tens of milliseconds, so plain
    eager module steps are timed (K steps after the warmup); each kernel's
    duration comes from events its own dispatch stamps, over the same steps.
    The forward takes the streamed path (route-record kernel, then the
    streamed gather) and the backward the general path (sort, row, reduce and
    scatter kernels)."""
    import torch

    from tropnn_amd import PairwiseLinear
    from tropnn_amd.backends.pairwise_hip import arm_kernel_events

    b = C4["b"]
    layer = PairwiseLinear(C4["i"], C4["o"], tables=C4["t"], comparisons=C4["c"], seed=0, device_lut_dtype="f16")
    layer = layer.to(dev).train()
    layer.cache_route_debug = False
    nb = 2
    gen = torch.Generator().manual_seed(0)
    xs = [torch.randn(b, C4["i"], generator=gen).to(dev).requires_grad_(True) for _ in range(nb)]
    gs = [torch.randn(b, 1, C4["o"], generator=gen).to(dev) for _ in range(nb)]

    def step(k: int) -> None:
        layer.zero_grad(set_to_none=True)
        xs[k].grad = None
        layer(xs[k]).backward(gs[k])

    for w in range(args.warmup):
        step(w % nb)
    torch.cuda.synchronize()
    algo = algorithmic_bytes(False, e=2, streamed=True, **C4)
    names = tuple(algo)
    stream = torch.cuda.current_stream(dev)
    evs = {n: [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)] for n in names}
    for n in names:
        for e0, e1 in evs[n]:
            e0.record(stream)
            e1.record(stream)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        for n in names:
            arm_kernel_events(n, *evs[n][k])
        step(k % nb)
    torch.cuda.synchronize()
    step_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    kern_us = {n: 1e3 * sum(e0.elapsed_time(e1) for e0, e1 in evs[n]) / args.steps for n in names}
    log(f"c4 {step_ms:.2f} ms/step; kernels (ms): " + ", ".join(f"{n}={v * 1e-3:.3f}" for n, v in kern_us.items()))
    dom = max(names, key=lambda n: kern_us[n])
    achieved = algo[dom] / (kern_us[dom] * 1e-6) / 1e9
    if args.calibrate_copy_bytes > 0:
        calibration_copy(args.calibrate_copy_bytes, dev)
    cpu = None
    if args.cpu_budget > 0:
        log("timing the CPU baseline")
        cpu = cpu_baseline_c4(args.cpu_budget)
        log(f"cpu baseline {cpu['value']:.1f} samples/s on {cpu['cores']} threads")
    value = b / (step_ms * 1e-3)
    total_algo = sum(algo.values())
    out = {
        "metric": "PairwiseLinear c4 samples/s fwd+bwd (1024->4096, T=512, C=8, f16 LUT, B=8192) + achieved HBM GB/s vs peak",
        "value": round(value, 1),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: x, G ~ N(0,1), 2 resident batches alternating; seeded module init (seed 0)",
        "config": {
            "workload": "c4: PairwiseLinear(1024->4096, tables=512, comparisons=8), f16 LUT reads [512,256,4096] "
            "(RNE copy of the f32 master), batch 8192, fwd + fast_sigmoid_odd min-margin STE bwd "
            "(x, thresholds, f32 LUT grads)",
            "batch": b,
            "in_features": C4["i"],
            "out_features": C4["o"],
            "tables": C4["t"],
            "comparisons": C4["c"],
            "lut_dtype": "f16",
            "mode": "eager module fwd+bwd",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dom,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(dom, "c4"),
        },
        "cpu_baseline": cpu,
        "step_algorithmic_GBs": round(total_algo / (step_ms * 1e-3) / 1e9, 1),
        "step_roofline_frac": round(total_algo / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "kernels": {
            n: {"avg_us": round(kern_us[n], 1), "algorithmic_bytes": algo[n],
                "achieved_GBs": round(algo[n] / (kern_us[n] * 1e-6) / 1e9, 1) if kern_us[n] > 0 else None}
            for n in names
        },
    }
    if cpu:
        out["speedup_vs_cpu"] = round(value / cpu["value"], 1)
    return out


def calibration_copy(nbytes: int, dev) -> None:
    """One plain device copy of `nbytes`: the reference dispatch whose
    rocprofv3 FETCH_SIZE / WRITE_SIZE readings scale the kernels' to bytes."""
    import torch

    n = nbytes // 4
    src = torch.ones(n, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    log(f"calibration copy of {n * 4} bytes done")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument(
        "--workload",
        choices=("c2", "c3", "c4", "c5"),
        default="c2",
        help="c2: the BASELINE metric (default); c3: f16 eval forward at batch 1 / 64 / 8192; "
        "c4: the large f16-LUT layer fwd+bwd at batch 8192; c5: the EMNIST classifier training step",
    )
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default 500; 20 for c4)")
    ap.add_argument("--warmup", type=int, default=None, help="warmup steps (default 50; 3 for c4)")
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU baseline work (0 = skip)")
    ap.add_argument(
        "--calibrate-copy-bytes",
        type=int,
        default=0,
        help="also run one plain device copy of this many bytes (the reference dispatch that scales "
        "rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes)",
    )
    args = ap.parse_args()
    if args.steps is None:
        args.steps = 20 if args.workload == "c4" else 500
    if args.warmup is None:
        args.warmup = 3 if args.workload == "c4" else 50
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py measures one GPU only: the PairwiseLinear path is built and measured on a single MI355X "
            "(multi-GPU sharding is a design note, not part of this build). Run with --gpus 1.",
            file=sys.stderr,
        )
        return 2

    import torch

    from tropnn_amd import PairwiseLinear
    from tropnn_amd.backends.pairwise_hip import arm_kernel_events, library_path

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log(f"device {torch.cuda.get_device_name(dev)}, library {library_path()}")
    if args.workload != "c2":
        runner = {"c3": bench_c3, "c4": bench_c4, "c5": bench_c5}[args.workload]
        print(json.dumps(runner(args, dev)))
        return 0

    layer = PairwiseLinear(I, O, tables=T, comparisons=C, seed=0).to(dev).train()
    layer.cache_route_debug = False  # route debug tensors are not part of the step
    nb = 4
    gen = torch.Generator().manual_seed(0)
    xs = [torch.randn(B, I, generator=gen).to(dev).requires_grad_(True) for _ in range(nb)]
    gs = [torch.randn(B, 1, O, generator=gen).to(dev) for _ in range(nb)]

    def step(k: int) -> None:
        layer.zero_grad(set_to_none=True)
        xs[k].grad = None
        layer(xs[k]).backward(gs[k])

    stream = torch.cuda.current_stream(dev)
    for w in range(args.warmup):  # eager warmup (allocator, library, anchor index)
        step(w % nb)
    torch.cuda.synchronize()

    # ---- graph capture: one graph per resident batch, one step per graph
    side = torch.cuda.Stream(dev)
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        for w in range(3):
            step(w % nb)
    stream.wait_stream(side)
    torch.cuda.synchronize()

    def capture(ks: list[int]) -> torch.cuda.CUDAGraph:
        layer.zero_grad(set_to_none=True)
        for k in ks:
            xs[k].grad = None
        gph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gph):
            for k in ks:
                layer.zero_grad(set_to_none=True)
                layer(xs[k]).backward(gs[k])
        return gph

    def replay_rate(graphs: list, steps_per_graph: int, steps: int, tail: list | None = None) -> float:
        """us per step over exactly `steps` steps (steps // steps_per_graph
        replays of `graphs`, then steps % steps_per_graph one-step replays of
        `tail`), after >= 0.3 s (and >= --warmup replays) of warmup: the GPU
        clocks ramp up under sustained load."""
        torch.cuda.synchronize()
        t0, w = time.perf_counter(), 0
        while w < args.warmup or time.perf_counter() - t0 < 0.3:
            graphs[w % len(graphs)].replay()
            w += 1
        torch.cuda.synchronize()
        n, rest = divmod(steps, steps_per_graph)
        t0 = time.perf_counter()
        for k in range(n):
            graphs[k % len(graphs)].replay()
        for k in range(rest):
            tail[k % len(tail)].replay()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e6 / steps

    graphs = [capture([k]) for k in range(nb)]
    graph1_us = replay_rate(graphs, 1, args.steps)
    log(f"graph {graph1_us:.1f} us/step (one step per graph)")
    graphs4 = [capture([(j + i) % nb for i in range(4)]) for j in range(nb)]
    graph_us = replay_rate(graphs4, 4, args.steps, tail=graphs)
    graph_ms = graph_us * 1e-3
    log(f"graph {graph_us:.1f} us/step (four steps per graph)")

    # ---- per-kernel durations: eager steps right after the graph phase (GPU
    # clocks still up); each kernel's own dispatch stamps the armed events
    algo = algorithmic_bytes(fused_backward())
    names = tuple(algo)
    ksteps = min(args.steps, 200)
    evs = {n: [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(ksteps)] for n in names}
    for n in names:  # create the event handles
        for e0, e1 in evs[n]:
            e0.record(stream)
            e1.record(stream)
    for w in range(nb):
        step(w)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(ksteps):
        for n in names:
            arm_kernel_events(n, *evs[n][k])
        step(k % nb)
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / ksteps
    kern_us = {n: 1e3 * sum(e0.elapsed_time(e1) for e0, e1 in evs[n]) / ksteps for n in names}
    log(f"eager {eager_ms * 1e3:.1f} us/step; kernels (us): " + ", ".join(f"{n}={v:.2f}" for n, v in kern_us.items()))

    # ---- roofline of the dominant kernel
    dom = max(names, key=lambda n: kern_us[n])
    achieved = algo[dom] / (kern_us[dom] * 1e-6) / 1e9
    kernels = {
        n: {"avg_us": round(kern_us[n], 3), "algorithmic_bytes": algo[n], "achieved_GBs": round(algo[n] / (kern_us[n] * 1e-6) / 1e9, 1)}
        for n in names
    }

    if args.calibrate_copy_bytes > 0:
        calibration_copy(args.calibrate_copy_bytes, dev)

    cpu = None
    if args.cpu_budget > 0:
        log("timing the CPU baseline")
        cpu = cpu_baseline(args.cpu_budget)
        log(f"cpu baseline {cpu['value']:.0f} samples/s on {cpu['cores']} threads")

    value = B / (graph_ms * 1e-3)
    total_algo = sum(algo.values())
    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(graph_ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: x, G ~ N(0,1), 4 resident batches round-robin; seeded module init (seed 0)",
        "config": {
            "workload": "c2: PairwiseLinear(128->128, tables=136, comparisons=6), f32 LUT [136,64,128], batch 512, "
            "fwd + fast_sigmoid_odd min-margin STE bwd (x, thresholds, LUT grads)",
            "batch": B,
            "in_features": I,
            "out_features": O,
            "tables": T,
            "comparisons": C,
            "lut_dtype": "f32",
            "mode": "hip-graph replay of the module fwd+bwd, four steps (one per resident batch) per graph",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dom,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(dom),
        },
        "cpu_baseline": cpu,
        "step_algorithmic_GBs": round(total_algo / (graph_ms * 1e-3) / 1e9, 1),
        "us_per_step_one_step_per_graph": round(graph1_us, 3),
        "eager_ms_per_step": round(eager_ms, 6),
        "kernels": kernels,
    }
    if cpu:
        out["speedup_vs_cpu"] = round(value / cpu["value"], 1)
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
