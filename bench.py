"""PairwiseLinear fwd+bwd benchmark on one MI355X (BASELINE.json metric).

Workload ("c2"): PairwiseLinear(128->128, tables=136,
comparisons=6), f32 LUT [136, 64, 128], batch 512, x ~ N(0,1), upstream grad
G ~ N(0,1); one step = forward + fast_sigmoid_odd min-margin STE backward
(y = layer(x); y.backward(G)) with x, thresholds and LUT gradients. Params are
the module's seeded init (seed 0); inputs are synthetic and already in HBM.

Timed regions (both full fwd+bwd of the module API, no work skipped), each
measured by time_windows(): windows of exactly K = --steps steps are issued
back to back with a HIP event between consecutive windows, after >= 0.3 s of
warmup (the GPU clocks ramp up under sustained load); at least 25 windows,
100 steps and 0.2 s are timed and the MEDIAN window per step is reported,
with the fastest and slowest windows and the wall-clock mean beside it:
  graph  -- the steps captured in HIP graphs (torch.cuda.CUDAGraph), four
            steps per graph, one on each of 4 distinct resident (x, G)
            batches (a window is K // 4 four-step replays, then K % 4
            one-step replays). This is `value` / `ms_per_step`. One graph
            launch costs 14-19 us of host time and ~5 us on the device, so
            capturing the launch-bound loop four steps at a time keeps the GPU
            busy. The rate with one step per graph, and with the reference
            shell's route debug tensors written (cache_route_debug=True), are
            reported beside it.
  eager  -- plain autograd steps back to back (as the reference harness
            times its train step, tools/benchmarking/benchmark.py:105-118),
            and again under torch.autograd.set_multithreading_enabled(False),
            torch's switch that runs the backward on the calling thread
            instead of handing it to the device's autograd thread and back
            (`eager_us_per_step_calling_thread_engine`); in a further 200
            steps the kernels of each step carry HIP events that their own
            dispatch stamps (library hook tropnn_hip_arm_kernel_events, via
            hipExtLaunchKernel), giving the per-kernel durations (mean,
            median, min, max) that `roofline` uses.
peak_bytes: device bytes allocated above the resident state by one eval
forward and by one fwd+bwd step, measured as the reference harness measures
them (tools/benchmarking/benchmark.py:57-88), and the backward's workspace.

roofline (the dominant kernel, the longest average duration):
  achieved / frac -- HBM bytes per launch as rocprofv3 counts them
            (FETCH_SIZE + WRITE_SIZE, scaled by a calibration copy; committed
            in profiles/traffic*.json for the kernel sources they were taken
            from) / the launch duration measured here / 8 TB/s;
  algorithmic_* -- the gather convention (every (item, table) moves its LUT
            rows once): how fast the algorithm's work is done, which exceeds
            the HBM peak where rows come from LDS and L2;
  compulsory_*  -- each tensor the kernel must touch, once;
  l2_hit_rate   -- TCC_HIT / (TCC_HIT + TCC_MISS) from the same profile.

cpu_baseline: the oracle's torch restatement of the reference torch path
(kind "port"), the same step on every host core this process may use
(os.sched_getaffinity), rank 0 at N = 1 only; cpu_baselines adds the
Zig-equivalent C forward (oracle/lut_cpu.c, the reference backend="zig" path,
inference only) on the same cores.

Other BASELINE.json configs, each its own JSON line (--workload): c1, the
small f32 eval forward at batch 8 (latency); c3, the f16 eval forward sweep
at batch 1 / 64 / 8192; c4, the large f16-LUT layer fwd+bwd at batch 8192;
c5, the EMNIST classifier training step and its 100-step loss curve. The
default run also measures all four after the headline and adds compact
records of them under `other_configs` (--other-configs off skips them).

Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import json
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
C1 = {"b": 8, "i": 256, "o": 512, "t": 16, "c": 6}
C4 = {"b": 8192, "i": 1024, "o": 4096, "t": 512, "c": 8}
C4_CPU_BATCH = 8


def algorithmic_bytes(fused: bool, b: int = B, i: int = I, o: int = O, t: int = T, c: int = C, e: int = E,
                      streamed: bool = False, scatter: bool = False) -> dict[str, int]:
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
        grad_thr, and (its item role forming the input gradient in the same
        launch) x re-read (margins), grad_x, anchors + thresholds;
      with `scatter` (more tables than the item role takes) the last three
        go to backward_scatter, the kernel that then forms grad_x;
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
        if scatter:
            return {"forward": fwd, "backward_fused": g_codes_rows + lut_rows + 4 * t * c, "backward_scatter": x_side}
        return {"forward": fwd, "backward_fused": g_codes_rows + lut_rows + 4 * t * c + x_side}
    head = {"forward": fwd}
    if streamed:
        route = 4 * b * i + 20 * t * c + b * t
        head = {"forward_route": route, "forward": fwd - route}
    return {**head, "backward_sort": 0, "backward_table": g_codes_rows + lut_rows,
            "backward_reduce": 4 * t * c, "backward_scatter": x_side}


def compulsory_bytes(fused: bool, b: int = B, i: int = I, o: int = O, t: int = T, c: int = C, e: int = E,
                     streamed: bool = False, scatter: bool = False) -> dict[str, int]:
    """Per-launch compulsory bytes: each tensor a kernel must read or write,
    once, with the LUT capped at the min(B, 2^C) rows per table that items
    can touch. Each kernel counts what it must move by itself, so the LUT,
    which the forward and the backward each read, counts in both:
      forward: x, anchors + thresholds, the LUT, y, one code byte per
        (item, table) kept for the backward (streamed: the route kernel
        takes x, anchors + thresholds and the codes, the gather the LUT and y);
      backward_fused / backward_table: G, the codes, the LUT (for the STE
        dots), grad_lut (every row, untouched rows as zeros), and for the
        fused kernel grad_thr and (without `scatter`) grad_x and the anchors;
      backward_reduce: grad_thr;
      backward_scatter: grad_x and the anchors;
      backward_sort: nothing.
    The step total at c2 is 14,589,824 B: 9,981,056 B for every tensor of the
    step once, plus the code bytes and the backward's second LUT read."""
    r = 1 << c
    lut = e * t * min(b, r) * o
    grad_lut = 4 * t * r * o
    fwd = 4 * b * i + 20 * t * c + lut + 4 * b * o + b * t
    bwd_rows = 4 * b * o + b * t + lut + grad_lut
    x_side = 4 * b * i + 16 * t * c
    if fused:
        if scatter:
            return {"forward": fwd, "backward_fused": bwd_rows + 4 * t * c, "backward_scatter": x_side}
        return {"forward": fwd, "backward_fused": bwd_rows + 4 * t * c + x_side}
    head = {"forward": fwd}
    if streamed:
        route = 4 * b * i + 20 * t * c + b * t
        head = {"forward_route": route, "forward": fwd - route}
    return {**head, "backward_sort": 0, "backward_table": bwd_rows, "backward_reduce": 4 * t * c,
            "backward_scatter": x_side}


def backward_path() -> tuple[bool, bool]:
    """(fused, scatter): whether the library runs c2's backward as the fused
    table kernel, and whether a scatter kernel follows it. The workspace
    tells: none when the fused launch's item role forms the input gradient,
    the 8-byte {gu, r} records when the scatter kernel does; the general
    path's also holds the sorted slots, a copy of G and the partial dots."""
    from tropnn_amd.backends.pairwise_hip import LUT_F32, STE_MIN_MARGIN, load_library

    lib = load_library()  # declares the C signatures
    ws = lib.tropnn_hip_pairwise_backward_workspace_size(B, I, O, T, C, LUT_F32, STE_MIN_MARGIN)
    return ws <= 8 * T * B + 16 * T * C + 16, ws > 0


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


def profile_record(kernel: str, workload: str = "c2") -> dict | None:
    """The committed rocprofv3 counter summary of one kernel of a workload
    (profiles/traffic.json for c2, profiles/traffic_<workload>.json
    otherwise): fetch_bytes and write_bytes (FETCH_SIZE and WRITE_SIZE
    scaled by a calibration copy) and, where the profile has them, TCC_HIT /
    TCC_MISS per launch. Used only while the kernel sources (comments aside)
    still hash to the profiled ones; otherwise None."""
    path = ROOT / "profiles" / ("traffic.json" if workload == "c2" else f"traffic_{workload}.json")
    if not path.exists():
        return None
    rec = json.loads(path.read_text())
    if rec.get("source_digest") != source_digest() or kernel not in rec.get("kernels", {}):
        return None
    return rec["kernels"][kernel]


def measured_traffic(kernel: str, workload: str = "c2") -> int | None:
    """HBM bytes per launch of `kernel` (FETCH_SIZE + WRITE_SIZE) from the
    committed profile, or None (see profile_record)."""
    k = profile_record(kernel, workload)
    return None if k is None else int(k["fetch_bytes"] + k["write_bytes"])


def l2_hit_rate(kernel: str, workload: str = "c2") -> float | None:
    k = profile_record(kernel, workload)
    if k is None or "tcc_hit" not in k:
        return None
    total = k["tcc_hit"] + k["tcc_miss"]
    return round(k["tcc_hit"] / total, 4) if total > 0 else None


def roofline(kernel: str, avg_us: float, algo: int, comp: int, workload: str) -> dict:
    """The roofline object of one kernel: HBM bytes per launch from the
    committed counter profile / the live launch duration / 8 TB/s, beside the
    algorithmic (gather convention) and compulsory figures. Without a
    profile of the current sources, `achieved` falls back to the compulsory
    bytes and `basis` says so."""
    t = avg_us * 1e-6
    traffic = measured_traffic(kernel, workload)
    hbm_bytes = traffic if traffic is not None else comp
    achieved = hbm_bytes / t / 1e9
    return {
        "bound": "hbm",
        "kernel": kernel,
        "basis": ("rocprofv3 FETCH_SIZE + WRITE_SIZE bytes per launch (calibrated; profiles/"
                  + ("traffic.json" if workload == "c2" else f"traffic_{workload}.json") + ") / live launch duration")
        if traffic is not None else "compulsory bytes / live launch duration (no counter profile of these sources)",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": traffic,
        "avg_us": round(avg_us, 3),
        "l2_hit_rate": l2_hit_rate(kernel, workload),
        "mall_hit_rate": None,  # gfx950's rocprofv3 exposes no MALL (Infinity Cache) counter
        "algorithmic_bytes": algo,
        "algorithmic_GBs": round(algo / t / 1e9, 1),
        "algorithmic_frac": round(algo / t / 1e9 / HBM_PEAK_GBS, 4),
        "compulsory_bytes": comp,
        "compulsory_frac": round(comp / t / 1e9 / HBM_PEAK_GBS, 4),
    }


# ---------------------------------------------------------------- CPU legs
def host_threads() -> int:
    """Host cores this process may run on (os.sched_getaffinity): every CPU
    leg uses all of them, torch through torch.set_num_threads and the
    Zig-equivalent through tropnn_set_num_threads."""
    return len(os.sched_getaffinity(0))


def _median_time(fn, budget_s: float, min_iters: int = 3) -> tuple[float, int]:
    """Median wall time of fn() over as many calls as fit `budget_s` (at
    least min_iters), after one warmup call."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < min_iters:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def _oracle_layer(i: int, o: int, t: int, c: int, seed: int = 0):
    from oracle.pairwise_torch import OraclePairwiseLinear

    return OraclePairwiseLinear(i, o, tables=t, comparisons=c, seed=seed)


def cpu_torch_train(i: int, o: int, t: int, c: int, b: int, budget_s: float, label: str) -> dict:
    """The oracle (torch restatement of the reference torch path) fwd + STE
    bwd on the host cores: y = layer(x); y.backward(G), x needing grad."""
    import torch

    n = host_threads()
    torch.set_num_threads(n)
    layer = _oracle_layer(i, o, t, c).train()
    x = torch.randn(b, i, generator=torch.Generator().manual_seed(0)).requires_grad_(True)
    g = torch.randn(b, 1, o, generator=torch.Generator().manual_seed(1))

    def step() -> None:
        layer.zero_grad(set_to_none=True)
        x.grad = None
        layer(x).backward(g)

    med, n_it = _median_time(step, budget_s)
    return {
        "value": b / med,
        "unit": "samples/s",
        "cores": n,
        "kind": "port",
        "path": "torch-CPU (reference backend='torch')",
        "ms_per_call": round(med * 1e3, 4),
        "sample": f"{label} fwd+bwd at batch {b}, {n_it} steps (median {med * 1e3:.2f} ms/step), "
        f"oracle/pairwise_torch.py torch-CPU restatement, torch.set_num_threads={n} "
        f"(all cores in os.sched_getaffinity)",
    }


def cpu_torch_eval(i: int, o: int, t: int, c: int, b: int, budget_s: float, label: str) -> dict:
    """The oracle's eval forward (torch.no_grad, f32 LUT: the reference torch
    path reads the f32 parameter) on the host cores, calls back to back like
    tools/benchmarking/benchmark.py:91-102."""
    import torch

    n = host_threads()
    torch.set_num_threads(n)
    layer = _oracle_layer(i, o, t, c).eval()
    x = torch.randn(b, i, generator=torch.Generator().manual_seed(0))

    def call() -> None:
        with torch.no_grad():
            layer(x)

    med, n_it = _median_time(call, budget_s)
    return {
        "value": b / med,
        "unit": "samples/s",
        "cores": n,
        "kind": "port",
        "path": "torch-CPU (reference backend='torch')",
        "ms_per_call": round(med * 1e3, 4),
        "sample": f"{label} eval forward at batch {b}, f32 LUT, {n_it} calls (median {med * 1e3:.3f} ms/call), "
        f"oracle/pairwise_torch.py, torch.set_num_threads={n}",
    }


def cpu_zig_eval(i: int, o: int, t: int, c: int, b: int, lut_dtype: str, budget_s: float, label: str) -> dict:
    """The Zig-equivalent CPU forward (oracle/lut_cpu.c, the C restatement of
    kernels/src/lut.zig:248-318) on the host cores, called as
    pairwise_zig_forward calls the Zig library (backends/pairwise_zig.py:
    35-103): the LUT in the read dtype prepared once (the reference caches
    its f16 copy by version, layers/pairwise.py:82-92), per call an output
    allocation and the C call, which zeroes and fills it."""
    import torch

    from oracle import lut_cpu

    n = host_threads()
    torch.set_num_threads(n)
    lib = lut_cpu.load()
    lib.tropnn_set_num_threads(n)
    layer = _oracle_layer(i, o, t, c)
    x = torch.randn(b, i, generator=torch.Generator().manual_seed(0)).contiguous()
    anchors = layer.anchors.contiguous()
    thr = layer.thresholds.detach().contiguous()
    w = layer.lut.detach().to(torch.float16 if lut_dtype == "f16" else torch.float32).contiguous()
    fn = lib.lut_forward_batch_f16_no_cache if lut_dtype == "f16" else lib.lut_forward_batch_with_offsets_no_cache

    def call() -> None:
        out = torch.empty(b, o, dtype=torch.float32)
        fn(b, t, c, i, o, w.data_ptr(), anchors.data_ptr(), thr.data_ptr(), x.data_ptr(), out.data_ptr())

    med, n_it = _median_time(call, budget_s)
    return {
        "value": b / med,
        "unit": "samples/s",
        "cores": n,
        "kind": "port",
        "path": f"Zig-equivalent CPU (reference backend='zig', {lut_dtype} LUT)",
        "ms_per_call": round(med * 1e3, 4),
        "sample": f"{label} eval forward at batch {b}, {lut_dtype} LUT, {n_it} calls (median {med * 1e3:.3f} ms/call), "
        f"oracle/lut_cpu.c (-O3 -march=x86-64-v3), tropnn_set_num_threads={n}",
    }


# ---------------------------------------------------------------- GPU helpers
def _kernel_events(names, n):
    import torch

    evs = {k: [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
           for k in names}
    stream = torch.cuda.current_stream()
    for k in names:  # create the event handles
        for e0, e1 in evs[k]:
            e0.record(stream)
            e1.record(stream)
    return evs


def _spread(values) -> dict:
    """mean, median, min and max of a list of per-launch (or per-step) times."""
    v = sorted(values)
    return {"mean": sum(v) / len(v), "median": v[len(v) // 2], "min": v[0], "max": v[-1], "n": len(v)}


# (min windows, min steps, min seconds, warmup seconds) of time_windows();
# --quick (rocprofv3 counter passes, where every dispatch is serialised)
# lowers them to a few dispatches of each kernel
WINDOW_FLOORS = {"windows": 25, "steps": 100, "seconds": 0.2, "warmup_s": 0.3}


def time_windows(window, steps: int, warmup: int, min_windows: int | None = None, min_steps: int | None = None,
                 min_seconds: float | None = None) -> dict:
    """Device time per step as the median over >= 100 steps (the benchmark
    plan for c2). window() issues one window of `steps` steps without
    waiting for them. After >= `warmup` warmup windows and >= 0.3 s of them
    (the GPU clocks ramp up under sustained load), n windows are issued back
    to back with no host synchronisation between them and a HIP event
    recorded on the current stream between consecutive windows, n =
    max(min_windows, ceil(min_steps / steps), the windows that fill
    min_seconds). Each window's time is the interval between its two events;
    the figure is the median window per step, with the fastest and slowest
    windows and the wall-clock mean over the whole timed region beside it, so
    one host stall moves one window, not the figure."""
    import math

    import torch

    min_windows = WINDOW_FLOORS["windows"] if min_windows is None else min(min_windows, WINDOW_FLOORS["windows"])
    min_steps = WINDOW_FLOORS["steps"] if min_steps is None else min(min_steps, WINDOW_FLOORS["steps"])
    min_seconds = WINDOW_FLOORS["seconds"] if min_seconds is None else min(min_seconds, WINDOW_FLOORS["seconds"])
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    t0, w = time.perf_counter(), 0
    while w < max(warmup, 2) or time.perf_counter() - t0 < WINDOW_FLOORS["warmup_s"]:
        window()
        w += 1
    torch.cuda.synchronize()
    est_s = (time.perf_counter() - t0) / w
    n = max(min_windows, math.ceil(min_steps / steps), math.ceil(min_seconds / max(est_s, 1e-9)))
    n = min(n, 20000)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    window()  # queue work ahead of the first event so it marks a busy device
    t0 = time.perf_counter()
    evs[0].record(stream)
    for k in range(n):
        window()
        evs[k + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per_step = sorted(1e3 * evs[k].elapsed_time(evs[k + 1]) / steps for k in range(n))
    return {
        "us_per_step": per_step[n // 2],
        "min": per_step[0],
        "max": per_step[-1],
        "windows": n,
        "steps_per_window": steps,
        "wall_mean": wall * 1e6 / (n * steps),
    }


def window_fields(t: dict, prefix: str = "") -> dict:
    """The spread of a time_windows() result as JSON fields (us per step)."""
    return {
        f"{prefix}windows": t["windows"],
        f"{prefix}window_min_us": round(t["min"], 3),
        f"{prefix}window_max_us": round(t["max"], 3),
        f"{prefix}wall_mean_us": round(t["wall_mean"], 3),
    }


def peak_bytes(fn, dev) -> int:
    """Peak device bytes allocated by one fn() call above what was allocated
    before it, measured as the reference harness measures its forward and
    train peaks (tools/benchmarking/benchmark.py:57-88): memory_allocated
    before, reset_peak_memory_stats, the call and a synchronize,
    max_memory_allocated after."""
    import torch

    torch.cuda.synchronize(dev)
    base = torch.cuda.memory_allocated(dev)
    torch.cuda.reset_peak_memory_stats(dev)
    out = fn()
    torch.cuda.synchronize(dev)
    peak = torch.cuda.max_memory_allocated(dev)
    del out
    torch.cuda.synchronize(dev)
    return max(0, int(peak - base))


def eval_peak_bytes(layer, x, dev) -> int:
    """Peak bytes of one eval forward under torch.no_grad (benchmark.py:57-70)."""
    import torch

    def fn():
        with torch.no_grad():
            return layer(x)

    layer.eval()
    return peak_bytes(fn, dev)


def train_peak_bytes(layer, x, g, dev) -> int:
    """Peak bytes of one fwd+bwd step (y = layer(x); y.backward(G)) with the
    gradients set to None before the baseline is read, as benchmark.py:73-88
    measures its train step; the gradients the step leaves are part of the
    peak."""
    def fn():
        layer(x).backward(g)

    layer.train()
    layer.zero_grad(set_to_none=True)
    x.grad = None
    out = peak_bytes(fn, dev)
    layer.zero_grad(set_to_none=True)
    x.grad = None
    return out


def backward_workspace_bytes(b: int, i: int, o: int, t: int, c: int, lut_f16: bool) -> int:
    """The device workspace one min-margin STE backward allocates
    (tropnn_hip_pairwise_backward_workspace_size)."""
    from tropnn_amd.backends.pairwise_hip import LUT_F16, LUT_F32, STE_MIN_MARGIN, load_library

    return int(load_library().tropnn_hip_pairwise_backward_workspace_size(
        b, i, o, t, c, LUT_F16 if lut_f16 else LUT_F32, STE_MIN_MARGIN))


def _eval_forward_gpu(layer, xs, steps: int, warmup: int) -> dict:
    """GPU times of the module's eval forward on resident inputs: back to back
    eager calls (benchmark.py:91-102's loop), the median latency of one call
    to its result (call, then synchronize), one HIP graph per call replayed
    back to back, and the forward kernel's own duration (events stamped by
    its dispatch). Back-to-back figures are time_windows() medians of windows
    of `steps` calls."""
    import torch

    from tropnn_amd.backends.pairwise_hip import arm_kernel_events

    nb = len(xs)
    ctr = [0]

    def eager_window() -> None:
        with torch.no_grad():
            for _ in range(steps):
                layer(xs[ctr[0] % nb])
                ctr[0] += 1

    with torch.no_grad():
        for x in xs:
            layer(x)
    eager = time_windows(eager_window, steps, warmup)
    with torch.no_grad():
        lat = []
        for k in range(min(steps * 10, 200)):
            t0 = time.perf_counter()
            layer(xs[k % nb])
            torch.cuda.synchronize()
            lat.append(time.perf_counter() - t0)
        lat.sort()
        sync_us = lat[len(lat) // 2] * 1e6
        graphs = []
        for x in xs:
            gph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gph):
                layer(x)
            graphs.append(gph)

    def graph_window() -> None:
        for _ in range(steps):
            graphs[ctr[0] % nb].replay()
            ctr[0] += 1

    graph = time_windows(graph_window, steps, warmup)
    abi = _abi_eval_windows(layer, xs, steps, warmup)
    evs = _kernel_events(("forward",), 100)["forward"]
    with torch.no_grad():
        for k, (e0, e1) in enumerate(evs):
            arm_kernel_events("forward", e0, e1)
            layer(xs[k % nb])
    torch.cuda.synchronize()
    kern = _spread([1e3 * e0.elapsed_time(e1) for e0, e1 in evs])
    return {"eager_us_per_call": eager["us_per_step"], "sync_latency_us": sync_us,
            "graph_us_per_call": graph["us_per_step"], "abi_us_per_call": abi["us_per_step"],
            "kernel_us": kern["median"], "kernel_us_mean": kern["mean"],
            "kernel_spread": kern, "eager_windows": eager, "graph_windows": graph, "abi_windows": abi}


def _abi_eval_windows(layer, xs, steps: int, warmup: int) -> dict:
    """The eval entry point of the C ABI (tropnn_hip_lut_forward_batch_f32 /
    _f16, the Zig exports' counterpart) called the way cpu_zig_eval calls the
    Zig-equivalent CPU forward: the LUT in the read dtype prepared once, per
    call an output allocation and the call (through ctypes, on torch's
    current stream), calls back to back on resident inputs. Both CPU and GPU
    figures then leave out the module's Python (shared by every backend of
    the reference's module)."""
    import torch

    from tropnn_amd.backends.pairwise_hip import load_library

    lib = load_library()
    w = layer._lut_for_reading().detach().contiguous()
    f16 = w.dtype == torch.float16
    fn = lib.tropnn_hip_lut_forward_batch_f16 if f16 else lib.tropnn_hip_lut_forward_batch_f32
    anc = layer.anchors.contiguous()
    thr = layer.thresholds.detach().contiguous()
    b, i = xs[0].shape
    t, c, o = layer.tables, layer.comparisons, layer.out_features
    dev = xs[0].device
    stream = torch.cuda.current_stream(dev).cuda_stream
    scale = float(layer.output_scale)
    args = (t, c, i, o, w.data_ptr(), anc.data_ptr(), thr.data_ptr())
    ptrs = [x.contiguous().data_ptr() for x in xs]
    nb = len(xs)
    ctr = [0]

    def window() -> None:
        for _ in range(steps):
            out = torch.empty(b, o, dtype=torch.float32, device=dev)
            rc = fn(b, *args, ptrs[ctr[0] % nb], out.data_ptr(), scale, stream)
            if rc != 0:
                raise RuntimeError(lib.tropnn_hip_last_error().decode())
            ctr[0] += 1

    # the ABI call gives the module's output (checked once)
    out = torch.empty(b, o, dtype=torch.float32, device=dev)
    fn(b, *args, ptrs[0], out.data_ptr(), scale, stream)
    with torch.no_grad():
        ref = layer(xs[0]).reshape(b, o)
    if not torch.equal(out, ref):
        raise AssertionError("the C ABI's eval forward differs from the module's")
    return time_windows(window, steps, warmup)


# ---------------------------------------------------------------- workloads
def bench_c1(args, dev) -> dict:
    """c1: PairwiseLinear(256 -> 512, T = 16,
    C = 6), f32 eval forward at batch 8, seeded init (seed 0), x ~ N(0,1)
    from seed 0: a latency configuration. `value` is the module's eval
    forward time per call with calls back to back, as the reference harness
    times it (benchmark.py:91-102); beside it the latency of one call to its
    result, the per-call time of graph replays, the kernel's own duration,
    and both reference CPU paths on the same host cores."""
    import torch

    from tropnn_amd import PairwiseLinear

    b = C1["b"]
    layer = PairwiseLinear(C1["i"], C1["o"], tables=C1["t"], comparisons=C1["c"], seed=0).to(dev).eval()
    gen = torch.Generator().manual_seed(0)
    xs = [torch.randn(b, C1["i"], generator=gen).to(dev) for _ in range(4)]
    gpu = _eval_forward_gpu(layer, xs, args.steps, args.warmup)
    log("c1: " + ", ".join(f"{k}={v:.2f}" for k, v in gpu.items() if isinstance(v, float)))
    fwd_peak = eval_peak_bytes(layer, xs[0], dev)
    algo = 4 * b * C1["i"] + 20 * C1["t"] * C1["c"] + 4 * b * C1["t"] * C1["o"] + 4 * b * C1["o"]
    cpus = []
    if args.cpu_budget > 0:
        budget = min(args.cpu_budget, 5.0)
        cpus.append(cpu_zig_eval(C1["i"], C1["o"], C1["t"], C1["c"], b, "f32", budget, "c1"))
        cpus.append(cpu_torch_eval(C1["i"], C1["o"], C1["t"], C1["c"], b, budget, "c1"))
        for c in cpus:
            log(f"c1 cpu {c['path']}: {c['ms_per_call'] * 1e3:.1f} us/call on {c['cores']} cores")
    us = gpu["eager_us_per_call"]
    out = {
        "metric": "PairwiseLinear c1 eval forward time per call (256->512, T=16, C=6, f32 LUT, B=8), calls back to back",
        "value": round(us, 3),
        "unit": "us/call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us * 1e-3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: x ~ N(0,1) from seed 0, 4 resident inputs; seeded module init (seed 0)",
        "config": {"workload": "c1: PairwiseLinear(256->512, tables=16, comparisons=6) eval forward, f32 LUT "
                   "[16,64,512], batch 8", "batch": b, "mode": "eager module calls under torch.no_grad"},
        "sync_latency_us": round(gpu["sync_latency_us"], 3),
        "graph_us_per_call": round(gpu["graph_us_per_call"], 3),
        "abi_us_per_call": round(gpu["abi_us_per_call"], 3),
        "kernel_us": round(gpu["kernel_us"], 3),
        **window_fields(gpu["eager_windows"]),
        "roofline": roofline("forward", gpu["kernel_us_mean"], algo,
                             compulsory_bytes(True, b=b, i=C1["i"], o=C1["o"], t=C1["t"], c=C1["c"])["forward"] - b * C1["t"],
                             "c1"),
        "peak_bytes": {"forward": fwd_peak},
        "cpu_baseline": cpus[0] if cpus else None,
        "cpu_baselines": cpus,
    }
    if cpus:
        out["speedup_vs_cpu"] = {c["path"]: round(c["ms_per_call"] * 1e3 / us, 2) for c in cpus}
    return out


def bench_c3(args, dev) -> dict:
    """c3: the c2 layer (128 -> 128, T = 136,
    C = 6) as eval forward only with f16 LUT reads, at batch 1, 64 and 8192:
    per call with calls back to back (eager or graph replays, the faster of
    the two), one call's latency to its result, the kernel's own duration,
    and the algorithmic-byte rate,
    F_eval = 4BI + 20TC + 2BTO + 4BO per call; beside each, the Zig-
    equivalent CPU forward (f16 LUT, as the reference's zig path reads it)
    and the torch-CPU forward (f32 LUT) on the same host cores."""
    import torch

    from tropnn_amd import PairwiseLinear

    layer = PairwiseLinear(I, O, tables=T, comparisons=C, seed=0, device_lut_dtype="f16").to(dev).eval()
    layer.cache_route_debug = False
    results = {}
    for b in (1, 64, 8192):
        gen = torch.Generator().manual_seed(0)
        xs = [torch.randn(b, I, generator=gen).to(dev) for _ in range(4)]
        gpu = _eval_forward_gpu(layer, xs, args.steps, args.warmup)
        algo = 4 * b * I + 20 * T * C + 2 * b * T * O + 4 * b * O
        # calls back to back, eager (the reference harness's loop) or as graph
        # replays, whichever the box runs faster: at small batches the graph
        # skips the Python path, at large ones eager calls pipeline behind the
        # kernels while each graph launch adds its own host and device cost
        us = min(gpu["eager_us_per_call"], gpu["graph_us_per_call"])
        mode = "eager" if us == gpu["eager_us_per_call"] else "graph"
        res = {
            "kernel_us": round(gpu["kernel_us"], 3),
            "kernel_us_mean": round(gpu["kernel_us_mean"], 3),
            "us_per_call": round(us, 3),
            "mode": mode,
            "eager_us_per_call": round(gpu["eager_us_per_call"], 3),
            "graph_us_per_call": round(gpu["graph_us_per_call"], 3),
            "abi_us_per_call": round(gpu["abi_us_per_call"], 3),
            "sync_latency_us": round(gpu["sync_latency_us"], 3),
            **window_fields(gpu[f"{mode}_windows"]),
            "samples_per_s": round(b / (us * 1e-6), 1),
            "algorithmic_bytes": algo,
            "algorithmic_GBs": round(algo / (us * 1e-6) / 1e9, 1),
            "forward_peak_bytes": eval_peak_bytes(layer, xs[0], dev),
        }
        log(f"c3 batch {b}: graph {gpu['graph_us_per_call']:.2f} us/call, eager {gpu['eager_us_per_call']:.2f}, "
            f"C ABI {gpu['abi_us_per_call']:.2f}, kernel {gpu['kernel_us']:.2f} us")
        if args.cpu_budget > 0:
            budget = min(args.cpu_budget, 4.0)
            cpus = [cpu_zig_eval(I, O, T, C, b, "f16", budget, "c3"), cpu_torch_eval(I, O, T, C, b, budget, "c3")]
            res["cpu_baselines"] = cpus
            res["speedup_vs_cpu"] = {c["path"]: round(c["ms_per_call"] * 1e3 / us, 1) for c in cpus}
            for c in cpus:
                log(f"c3 batch {b} cpu {c['path']}: {c['ms_per_call']:.3f} ms/call")
        results[str(b)] = res
    big = results["8192"]
    comp = compulsory_bytes(True, b=8192, e=2)["forward"] - 8192 * T
    out = {
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
        "config": {"workload": "c3: PairwiseLinear(128->128, tables=136, comparisons=6) eval forward, f16 LUT [136,64,128]",
                   "batches": [1, 64, 8192],
                   "mode": "module eval calls back to back under torch.no_grad: eager or one HIP graph per call, "
                   "the faster (per_batch.mode)"},
        "per_batch": results,
        "roofline": roofline("forward", big["kernel_us_mean"], big["algorithmic_bytes"], comp, "c3"),
        "cpu_baseline": results["8192"].get("cpu_baselines", [None])[0],
    }
    return out


def bench_c5(args, dev) -> dict:
    """c5: the pairwise EMNIST classifier
    784 -> 128 -> 128 -> 10 (T = 136, C = 6, seeds 0, 1, 2), batch 512 of
    synthetic sparse inputs, one training step = zero_grad, forward, cross
    entropy (tropnn_amd.cross_entropy: the library's one-launch loss and
    gradient), backward, Adam (lr 1e-3) step (FusedAdam: the library's Adam
    kernel), captured in one HIP graph per resident batch (4, round-robin)
    and timed over replays like c2. Then the 100-step loss curve
    (examples/emnist.py:203-228's loop on fresh seeded batches) of the HIP
    stack and of the oracle stack with torch Adam, from the same init."""
    import torch

    from tropnn_amd import FusedAdam, cross_entropy, unit_gradient
    from tropnn_amd.examples import EmnistPairwiseClassifier, make_c5_batch

    model = EmnistPairwiseClassifier().to(dev).train()
    for layer in model.layers:
        layer.cache_route_debug = False
    opt = FusedAdam(model.parameters(), lr=1e-3)  # the library's one-launch Adam, step counters on the device
    nb = 4
    batches = [tuple(t.to(dev) for t in make_c5_batch(512, seed=k)) for k in range(nb)]

    def step(k: int) -> None:
        x, y = batches[k]
        loss = cross_entropy(model(x), y)
        loss.backward(unit_gradient(loss))  # as loss.backward(), without its fill and scaling launches
        opt.step()

    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        for w in range(max(3, args.warmup)):
            opt.zero_grad(set_to_none=True)
            step(w % nb)
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    # peak bytes of one eager training step (forward, loss, backward,
    # optimizer step) after the optimizer state exists, the gradients set to
    # None before the baseline is read (benchmark.py:73-88)
    opt.zero_grad(set_to_none=True)
    train_peak = peak_bytes(lambda: step(0), dev)
    graphs = []
    for k in range(nb):
        opt.zero_grad(set_to_none=True)
        gph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gph):
            step(k)
        graphs.append(gph)
    torch.cuda.synchronize()
    ctr = [0]

    def window() -> None:
        for _ in range(args.steps):
            graphs[ctr[0] % nb].replay()
            ctr[0] += 1

    tw = time_windows(window, args.steps, args.warmup)
    us = tw["us_per_step"]
    log(f"c5 graph {us:.1f} us/step (median of {tw['windows']} windows, {tw['min']:.1f}-{tw['max']:.1f})")
    curve = c5_loss_curve(dev, args.curve_steps) if args.curve_steps > 0 else None
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
        **window_fields(tw),
        "layer_algorithmic_bytes_per_step": C5_LAYER_BYTES,
        "layer_algorithmic_GBs": round(C5_LAYER_BYTES / (us * 1e-6) / 1e9, 1),
        "peak_bytes": {"train_step": train_peak},
        "cpu_baseline": cpu,
        "loss_curve": curve,
    }
    if cpu:
        out["speedup_vs_cpu"] = round(value / cpu["value"], 1)
    return out


C5_LAYER_BYTES = 313_619_648  # the three layers' FwdBwd algorithmic bytes per c5 step (CE and Adam not counted)


def c5_loss_curve(dev, steps: int) -> dict:
    """`steps` training steps of the HIP classifier (tropnn_amd.cross_entropy,
    FusedAdam) and of the oracle classifier on the CPU (F.cross_entropy,
    torch.optim.Adam), from the same seeded init, on the same fresh batch per
    step (make_c5_batch with seed 1000 + step), eager. Per step: both losses,
    and whether every layer's route codes agree bit for bit. Route flips
    (a margin within rounding of zero) make the two trajectories part; the
    first step with differing codes is reported."""
    import torch
    import torch.nn.functional as F

    from tropnn_amd import FusedAdam, cross_entropy
    from tropnn_amd.examples import EmnistPairwiseClassifier, make_c5_batch

    n = host_threads()
    torch.set_num_threads(n)
    model = EmnistPairwiseClassifier().to(dev).train()
    dims = (784, 128, 128, 10)
    ref_layers = torch.nn.ModuleList(
        [_oracle_layer(a, b, T, C, seed=k) for k, (a, b) in enumerate(zip(dims[:-1], dims[1:]))]
    ).train()
    opt = FusedAdam(model.parameters(), lr=1e-3)
    opt_ref = torch.optim.Adam(ref_layers.parameters(), lr=1e-3, foreach=False)
    hip_loss, ref_loss, same_codes = [], [], []
    t0 = time.perf_counter()
    for k in range(steps):
        x, y = make_c5_batch(512, seed=1000 + k)
        opt.zero_grad(set_to_none=True)
        loss = cross_entropy(model(x.to(dev)), y.to(dev))
        loss.backward()
        opt.step()
        opt_ref.zero_grad(set_to_none=True)
        h = x.unsqueeze(1)
        for layer in ref_layers:
            h = layer(h)
        loss_r = F.cross_entropy(h.squeeze(1), y)
        loss_r.backward()
        opt_ref.step()
        hip_loss.append(loss.detach().item())
        ref_loss.append(loss_r.item())
        same_codes.append(all(torch.equal(a._last_indices.cpu(), b._last_indices) for a, b in zip(model.layers, ref_layers)))
    first_diff = next((k for k, s in enumerate(same_codes) if not s), None)
    rel = [abs(a - b) / abs(b) for a, b in zip(hip_loss, ref_loss)]
    upto = first_diff if first_diff is not None else steps
    log(f"c5 loss curve: {steps} steps in {time.perf_counter() - t0:.1f} s, codes first differ at step {first_diff}, "
        f"loss {hip_loss[0]:.4f} -> {hip_loss[-1]:.4f} (oracle {ref_loss[0]:.4f} -> {ref_loss[-1]:.4f})")
    return {
        "steps": steps,
        "batches": "make_c5_batch(512, seed=1000 + step), a fresh batch per step",
        "hip": [round(v, 6) for v in hip_loss],
        "oracle": [round(v, 6) for v in ref_loss],
        "codes_equal": same_codes,
        "first_step_codes_differ": first_diff,
        "max_rel_loss_diff_while_codes_equal": max(rel[:upto]) if upto > 0 else None,
        "max_rel_loss_diff": max(rel),
        "oracle_threads": n,
    }


def cpu_baseline_c5(budget_s: float) -> dict:
    """The oracle classifier (the three oracle layers, seeds 0, 1, 2) with
    torch Adam on the host cores: the same c5 training step, full batch."""
    import torch
    import torch.nn.functional as F

    from tropnn_amd.examples import make_c5_batch

    n = host_threads()
    torch.set_num_threads(n)
    dims = (784, 128, 128, 10)
    layers = torch.nn.ModuleList([_oracle_layer(a, b, T, C, seed=k) for k, (a, b) in enumerate(zip(dims[:-1], dims[1:]))])
    opt = torch.optim.Adam(layers.parameters(), lr=1e-3)
    x, y = make_c5_batch(512, seed=0)

    def step() -> None:
        opt.zero_grad(set_to_none=True)
        h = x.unsqueeze(1)
        for layer in layers:
            h = layer(h)
        F.cross_entropy(h.squeeze(1), y).backward()
        opt.step()

    med, n_it = _median_time(step, budget_s)
    return {
        "value": 512 / med,
        "unit": "samples/s",
        "cores": n,
        "kind": "port",
        "sample": f"c5 train step (3 oracle layers + CE + torch Adam), batch 512, {n_it} steps "
        f"(median {med * 1e3:.1f} ms/step), torch.set_num_threads={n}",
    }


def cpu_baseline_c4(budget_s: float) -> dict:
    """The oracle's torch restatement of the reference torch path at c4's
    layer (f32 LUT, as that path reads it) on the host cores, fwd + min-margin
    STE bwd, at a reduced batch of 8 items: the full batch of 8192 would hold
    ~64 GiB of saved STE rows (one [B, tables, 4096] f32 neighbour difference
    per route chunk). Reported per sample."""
    return cpu_torch_train(C4["i"], C4["o"], C4["t"], C4["c"], C4_CPU_BATCH, budget_s,
                           f"c4 layer (the full batch 8192 needs ~64 GiB of saved STE rows; f32 LUT)")


def bench_c4(args, dev) -> dict:
    """c4: PairwiseLinear(1024 -> 4096, T = 512,
    C = 8) reading an f16 LUT (the RNE copy of the f32 master; 1 GiB), batch
    8192, one step = forward + min-margin STE backward with x, thresholds and
    f32 LUT (2 GiB) gradients. A step takes milliseconds, so plain eager
    module steps are timed (K steps after the warmup); each kernel's
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
    train_peak = train_peak_bytes(layer, xs[0], gs[0], dev)
    workspace = backward_workspace_bytes(b, C4["i"], C4["o"], C4["t"], C4["c"], True)
    algo = algorithmic_bytes(False, e=2, streamed=True, **C4)
    comp = compulsory_bytes(False, e=2, streamed=True, **C4)
    names = tuple(algo)
    ctr = [0]

    def window() -> None:
        for _ in range(args.steps):
            step(ctr[0] % nb)
            ctr[0] += 1

    # steps take milliseconds: at least 5 windows and 10 steps (the benchmark
    # plan's >= 10 for c4), no time floor
    tw = time_windows(window, args.steps, 0, min_windows=5, min_steps=10, min_seconds=0.0)
    step_ms = tw["us_per_step"] * 1e-3
    # per-kernel durations over further steps, from events each kernel's own
    # dispatch stamps (kept out of the timed windows above)
    evs = _kernel_events(names, args.steps)
    torch.cuda.synchronize()
    for k in range(args.steps):
        for n in names:
            arm_kernel_events(n, *evs[n][k])
        step(k % nb)
    torch.cuda.synchronize()
    spread = {n: _spread([1e3 * e0.elapsed_time(e1) for e0, e1 in evs[n]]) for n in names}
    kern_us = {n: spread[n]["mean"] for n in names}
    log(f"c4 {step_ms:.2f} ms/step (median of {tw['windows']} windows of {args.steps}); kernels (ms): "
        + ", ".join(f"{n}={v * 1e-3:.3f}" for n, v in kern_us.items()))
    dom = max(names, key=lambda n: kern_us[n])
    cpu = None
    if args.cpu_budget > 0:
        log("timing the CPU baseline")
        cpu = cpu_baseline_c4(args.cpu_budget)
        log(f"cpu baseline {cpu['value']:.1f} samples/s on {cpu['cores']} threads")
    value = b / (step_ms * 1e-3)
    total_algo = sum(algo.values())
    traffic = {n: measured_traffic(n, "c4") for n in names}
    step_traffic = sum(traffic.values()) if all(v is not None for v in traffic.values()) else None
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
        **window_fields(tw),
        "roofline": roofline(dom, kern_us[dom], algo[dom], comp[dom], "c4"),
        "cpu_baseline": cpu,
        "peak_bytes": {"train_step": train_peak, "backward_workspace": workspace},
        "step": {
            "hbm_traffic_bytes": step_traffic,
            "hbm_frac": round(step_traffic / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4) if step_traffic else None,
            "compulsory_bytes": sum(comp.values()),
            "compulsory_frac": round(sum(comp.values()) / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "algorithmic_bytes": total_algo,
            "algorithmic_frac": round(total_algo / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        },
        "kernels": {
            n: {"avg_us": round(kern_us[n], 1), "min_us": round(spread[n]["min"], 1),
                "max_us": round(spread[n]["max"], 1), "algorithmic_bytes": algo[n], "compulsory_bytes": comp[n],
                "hbm_traffic_bytes": traffic[n], "l2_hit_rate": l2_hit_rate(n, "c4"),
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


def bench_c2(args, dev) -> dict:
    import torch

    from tropnn_amd import PairwiseLinear
    from tropnn_amd.backends.pairwise_hip import arm_kernel_events

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
    for w in range(max(args.warmup, nb)):  # eager warmup (allocator, library, anchor index)
        step(w % nb)
    torch.cuda.synchronize()
    train_peak = train_peak_bytes(layer, xs[0], gs[0], dev)
    fwd_peak = eval_peak_bytes(layer, xs[0].detach(), dev)
    layer.train()

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

    def replay_window(graphs: list, steps_per_graph: int, tail: list | None = None):
        """One window of exactly --steps steps: steps // steps_per_graph
        replays of `graphs` round robin, then steps % steps_per_graph
        one-step replays of `tail`."""
        n, rest = divmod(args.steps, steps_per_graph)
        ctr = [0]

        def window() -> None:
            for _ in range(n):
                graphs[ctr[0] % len(graphs)].replay()
                ctr[0] += 1
            for k in range(rest):
                tail[k % len(tail)].replay()

        return window

    graphs = [capture([k]) for k in range(nb)]
    t1 = time_windows(replay_window(graphs, 1), args.steps, args.warmup)
    graph1_us = t1["us_per_step"]
    log(f"graph {graph1_us:.1f} us/step (one step per graph; median of {t1['windows']} windows of {args.steps}, "
        f"{t1['min']:.1f}-{t1['max']:.1f})")
    graphs4 = [capture([(j + i) % nb for i in range(4)]) for j in range(nb)]
    t4 = time_windows(replay_window(graphs4, 4, tail=graphs), args.steps, args.warmup)
    graph_us = t4["us_per_step"]
    graph_ms = graph_us * 1e-3
    log(f"graph {graph_us:.1f} us/step (four steps per graph; median of {t4['windows']} windows of {args.steps}, "
        f"{t4['min']:.1f}-{t4['max']:.1f}, wall mean {t4['wall_mean']:.1f})")
    # the same step with the reference shell's route debug tensors (int64
    # indices and f32 margins written by every call, layers/base.py:78-83)
    layer.cache_route_debug = True
    graphs_dbg = [capture([(j + i) % nb for i in range(4)]) for j in range(nb)]
    td = time_windows(replay_window(graphs_dbg, 4, tail=graphs_dbg), args.steps, args.warmup)
    layer.cache_route_debug = False
    del graphs_dbg
    log(f"graph {td['us_per_step']:.1f} us/step with cache_route_debug=True")

    # ---- eager steps back to back: the host-bound rate of plain autograd
    # steps (the reference harness's loop), then per-kernel durations over
    # eager steps whose kernels stamp armed events
    ctr = [0]

    def eager_window() -> None:
        for _ in range(args.steps):
            step(ctr[0] % nb)
            ctr[0] += 1

    te = time_windows(eager_window, args.steps, args.warmup)
    eager_us = te["us_per_step"]
    log(f"eager {eager_us:.1f} us/step")
    # the same steps with torch's calling-thread autograd engine: the default
    # engine hands every backward to its device thread and back
    with torch.autograd.set_multithreading_enabled(False):
        tc = time_windows(eager_window, args.steps, args.warmup)
    eager_ct_us = tc["us_per_step"]
    log(f"eager {eager_ct_us:.1f} us/step (torch.autograd.set_multithreading_enabled(False))")
    fused, scatter = backward_path()
    algo = algorithmic_bytes(fused, scatter=scatter)
    comp = compulsory_bytes(fused, scatter=scatter)
    names = tuple(algo)
    ksteps = 20 if args.quick else 200
    evs = _kernel_events(names, ksteps)
    torch.cuda.synchronize()
    for k in range(ksteps):
        for n in names:
            arm_kernel_events(n, *evs[n][k])
        step(k % nb)
    torch.cuda.synchronize()
    spread = {n: _spread([1e3 * e0.elapsed_time(e1) for e0, e1 in evs[n]]) for n in names}
    kern_us = {n: spread[n]["mean"] for n in names}
    log("kernels (us, mean): " + ", ".join(f"{n}={v:.2f}" for n, v in kern_us.items()))

    dom = max(names, key=lambda n: kern_us[n])
    traffic = {n: measured_traffic(n) for n in names}
    kernels = {
        n: {"avg_us": round(kern_us[n], 3), "median_us": round(spread[n]["median"], 3),
            "min_us": round(spread[n]["min"], 3), "max_us": round(spread[n]["max"], 3),
            "algorithmic_bytes": algo[n], "compulsory_bytes": comp[n],
            "hbm_traffic_bytes": traffic[n], "l2_hit_rate": l2_hit_rate(n),
            "hbm_frac": round(traffic[n] / (kern_us[n] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4) if traffic[n] else None}
        for n in names
    }

    cpu = None
    zig = None
    if args.cpu_budget > 0:
        log("timing the CPU baselines")
        cpu = cpu_torch_train(I, O, T, C, B, args.cpu_budget, "c2")
        zig = cpu_zig_eval(I, O, T, C, B, "f32", min(args.cpu_budget, 3.0), "c2 (forward only: the zig path has no backward)")
        log(f"cpu baseline {cpu['value']:.0f} samples/s on {cpu['cores']} cores; zig-equivalent forward "
            f"{zig['ms_per_call']:.3f} ms/call")

    value = B / (graph_ms * 1e-3)
    total_algo = sum(algo.values())
    step_traffic = sum(traffic.values()) if all(v is not None for v in traffic.values()) else None
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
            "mode": "hip-graph replay of the module fwd+bwd, four steps (one per resident batch) per graph, "
            "cache_route_debug=False; ms_per_step = median over back-to-back windows of --steps steps",
        },
        **window_fields(t4),
        "us_per_step_route_debug": round(td["us_per_step"], 3),
        "roofline": roofline(dom, kern_us[dom], algo[dom], comp[dom], "c2"),
        "cpu_baseline": cpu,
        "cpu_zig_forward_ms": zig["ms_per_call"] if zig else None,
        "peak_bytes": {"forward": fwd_peak, "train_step": train_peak,
                       "backward_workspace": backward_workspace_bytes(B, I, O, T, C, False)},
        "step": {
            "hbm_traffic_bytes": step_traffic,
            "hbm_frac": round(step_traffic / (graph_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4) if step_traffic else None,
            "compulsory_bytes": sum(comp.values()),
            "compulsory_frac": round(sum(comp.values()) / (graph_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "algorithmic_bytes": total_algo,
            "algorithmic_frac": round(total_algo / (graph_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        },
        "us_per_step_one_step_per_graph": round(graph1_us, 3),
        "eager_us_per_step": round(eager_us, 3),
        "eager_us_per_step_calling_thread_engine": round(eager_ct_us, 3),
        "kernels": kernels,
    }
    if cpu:
        cpu["sample"] = cpu["sample"].split(", oracle/")[0] + ", oracle/pairwise_torch.py"
        out["speedup_vs_cpu"] = round(value / cpu["value"], 1)
        out["eager_speedup_vs_cpu"] = round(B / (eager_us * 1e-6) / cpu["value"], 1)
    return out


def _cpu_us(cpus: list, path_prefix: str) -> float | None:
    for c in cpus or []:
        if c and c["path"].startswith(path_prefix):
            return round(c["ms_per_call"] * 1e3, 2)
    return None


def compact_c1(r: dict) -> dict:
    return {
        "us_per_call": r["value"], "graph_us_per_call": r["graph_us_per_call"],
        "abi_us_per_call": r["abi_us_per_call"],
        "sync_latency_us": r["sync_latency_us"], "kernel_us": r["kernel_us"],
        "frac": r["roofline"]["frac"], "l2_hit_rate": r["roofline"]["l2_hit_rate"],
        "cpu_zig_us": _cpu_us(r["cpu_baselines"], "Zig"), "cpu_torch_us": _cpu_us(r["cpu_baselines"], "torch"),
        "forward_peak_bytes": r["peak_bytes"]["forward"], "windows": r["windows"],
    }


def compact_c3(r: dict) -> dict:
    out = {}
    for b, res in r["per_batch"].items():
        cpus = res.get("cpu_baselines")
        out[f"b{b}"] = {
            "us_per_call": res["us_per_call"], "mode": res["mode"], "abi_us_per_call": res["abi_us_per_call"],
            "kernel_us": res["kernel_us"],
            "samples_per_s": res["samples_per_s"], "cpu_zig_us": _cpu_us(cpus, "Zig"),
            "cpu_torch_us": _cpu_us(cpus, "torch"), "forward_peak_bytes": res["forward_peak_bytes"],
        }
    out["b8192"]["frac"] = r["roofline"]["frac"]
    out["b8192"]["l2_hit_rate"] = r["roofline"]["l2_hit_rate"]
    return out


def compact_c4(r: dict) -> dict:
    cpu = r.get("cpu_baseline")
    rf = r["roofline"]
    return {
        "ms_per_step": round(r["ms_per_step"], 4), "samples_per_s": r["value"], "windows": r["windows"],
        "kernel": rf["kernel"], "kernel_ms": round(rf["avg_us"] * 1e-3, 4), "frac": rf["frac"],
        "l2_hit_rate": rf["l2_hit_rate"], "step_hbm_frac": r["step"]["hbm_frac"],
        "step_compulsory_frac": r["step"]["compulsory_frac"],
        "kernel_ms_all": {n: round(k["avg_us"] * 1e-3, 4) for n, k in r["kernels"].items()},
        "cpu_torch_ms_per_step_batch8": cpu["ms_per_call"] if cpu else None,
        "speedup_per_sample": r.get("speedup_vs_cpu"),
        "train_peak_bytes": r["peak_bytes"]["train_step"], "workspace_bytes": r["peak_bytes"]["backward_workspace"],
    }


def compact_c5(r: dict) -> dict:
    cpu = r.get("cpu_baseline")
    curve = r.get("loss_curve") or {}
    return {
        "us_per_step": round(r["ms_per_step"] * 1e3, 3), "samples_per_s": r["value"], "windows": r["windows"],
        "window_min_us": r["window_min_us"], "window_max_us": r["window_max_us"],
        "cpu_torch_ms_per_step": round(512 / cpu["value"] * 1e3, 3) if cpu else None,
        "speedup_vs_cpu": r.get("speedup_vs_cpu"),
        "curve_steps": curve.get("steps"),
        "first_step_codes_differ": curve.get("first_step_codes_differ"),
        "max_rel_loss_diff_while_codes_equal": curve.get("max_rel_loss_diff_while_codes_equal"),
        "loss_first_last": [curve["hip"][0], curve["hip"][-1]] if curve.get("hip") else None,
        "train_peak_bytes": r["peak_bytes"]["train_step"],
    }


def other_configs(args, dev) -> dict:
    """Compact records of the other four BASELINE.json configs, measured in
    the same run on the same device after the headline: c1 (latency), c3 at
    batch 1 / 64 / 8192, c4 fwd+bwd and the c5 training step with its loss
    curve. Each runs its --workload function at fewer steps and shorter CPU
    samples (c4's torch-CPU leg at batch 8, >= 3 steps); the full records
    come from `--workload cN`. A workload that raises is recorded as its
    error, so the headline line is still printed."""
    import gc

    import torch

    plan = (
        ("c1", bench_c1, compact_c1, {"steps": 20, "warmup": 5, "cpu_budget": min(args.cpu_budget, 1.5)}),
        ("c3", bench_c3, compact_c3, {"steps": 20, "warmup": 5, "cpu_budget": min(args.cpu_budget, 1.0)}),
        ("c4", bench_c4, compact_c4, {"steps": 4, "warmup": 2, "cpu_budget": min(args.cpu_budget, 1.0)}),
        ("c5", bench_c5, compact_c5, {"steps": 20, "warmup": 5, "cpu_budget": min(args.cpu_budget, 3.0),
                                      "curve_steps": 100}),
    )
    out = {"host_cores": host_threads()}
    for name, fn, compact, over in plan:
        sub = argparse.Namespace(**{**vars(args), **over})
        t0 = time.perf_counter()
        log(f"other config {name}")
        try:
            out[name] = compact(fn(sub, dev))
        except Exception as exc:  # noqa: BLE001 -- recorded, the headline line still prints
            out[name] = {"error": f"{type(exc).__name__}: {exc}"[:300]}
        out[name]["bench_s"] = round(time.perf_counter() - t0, 1)
        gc.collect()
        torch.cuda.empty_cache()
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument(
        "--workload",
        choices=("c1", "c2", "c3", "c4", "c5"),
        default="c2",
        help="c2: the BASELINE metric (default); c1: the small f32 eval forward at batch 8 (latency); "
        "c3: f16 eval forward at batch 1 / 64 / 8192; c4: the large f16-LUT layer fwd+bwd at batch 8192; "
        "c5: the EMNIST classifier training step and its loss curve",
    )
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default 500; 20 for c4)")
    ap.add_argument("--warmup", type=int, default=None, help="warmup steps (default 50; 3 for c4)")
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU baseline work (0 = skip)")
    ap.add_argument("--curve-steps", type=int, default=100, help="c5: steps of the loss curve (0 = skip)")
    ap.add_argument(
        "--other-configs",
        choices=("on", "off"),
        default="on",
        help="with the default c2 workload, also measure c1, c3, c4 and c5 in the same run and add their "
        "compact records under other_configs (off: the c2 line alone)",
    )
    ap.add_argument(
        "--quick",
        action="store_true",
        help="minimal timing for rocprofv3 counter passes (every dispatch serialised): two windows, no time "
        "floors, 20 event-stamped steps; the times it prints are not benchmarks",
    )
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
    if args.quick:
        WINDOW_FLOORS.update(windows=2, steps=0, seconds=0.0, warmup_s=0.0)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py measures one GPU only: the PairwiseLinear path is built and measured on a single MI355X "
            "(multi-GPU sharding is a design note, not part of this build). Run with --gpus 1.",
            file=sys.stderr,
        )
        return 2

    import torch

    from tropnn_amd.backends.pairwise_hip import library_path

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log(f"device {torch.cuda.get_device_name(dev)}, library {library_path()}, host cores {host_threads()}")
    runner = {"c1": bench_c1, "c2": bench_c2, "c3": bench_c3, "c4": bench_c4, "c5": bench_c5}[args.workload]
    out = runner(args, dev)
    if args.workload == "c2" and args.other_configs == "on":
        out["other_configs"] = other_configs(args, dev)
    if args.calibrate_copy_bytes > 0:
        calibration_copy(args.calibrate_copy_bytes, dev)
    print(json.dumps(out, separators=(",", ":")))
    return 0


if __name__ == "__main__":
    sys.exit(main())
