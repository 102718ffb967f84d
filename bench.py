#!/usr/bin/env python3
"""Throughput of the RDT4quant fused forward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload block]

Default workload (the metric's configuration): the RMSNorm -> Mamba-3 block
forward, fp32, 64 windows x 32 tokens, d_model 64, 4 heads of 32, d_state 16,
expand 2, GroupedRMSNorm with 8 groups: one step is
x + out_proj(mamba3(in_proj(GroupedRMSNorm(x)))) over the 64 windows, and the
value is windows/s. Other workloads: ``mhc`` (the residual mix alone, 8192
tokens, tokens/s), ``mla`` (causal MLA, 256 x 128 tokens, windows/s),
``decode`` (65536 streams x 2 Mamba-3 blocks + head, stream-steps/s),
``stack`` (the 4-layer hybrid stack, 1024 x 256 tokens, windows/s),
``norms`` (RMSNorm + add-RMSNorm + LayerNorm over 262144 x 256, rows/s).

Timing: W untimed steps (replays of one-step HIP graphs), then exactly K
steps as one replay of a HIP graph that holds the K steps in order, between
two HIP events, synchronized on both sides; ms_per_step is that region's
time / K. Further replays of the same graph (30, or as many as fit in 10 s)
give the median and spread of the per-step time. Inputs are resident in HBM
before timing.

With no --workload, the line is the block's and, under "configs", the other
workloads' figures from the same run (value, ms per step, median, the
dominant kernel's roofline and counter traffic, the CPU baseline); --configs
none measures the named workload alone.

Prints one JSON line: whole-job throughput, the roofline of the dominant
kernel (per-launch average from HIP events over graph replays of that kernel
on the stream it runs on) and the CPU baseline: the reference's CPU kernels
compiled from its sources into oracle/_ref (the oracle port where that
library is absent) with torch CPU for GEMMs and SDPA, timed on this host with
every core and with one thread, warm-up 5 then the median of at least 30
steps, FTZ/DAZ on.
"""

from __future__ import annotations

import argparse
import copy
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT, ROOT / "montlok.cpp_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

HBM_PEAK_GBS = 8000.0
METRIC = "windows/sec for the RDT4quant block fwd at 1 GPU; % HBM or MFMA roofline"

# mHC residual mix alone, n = 4, d = 128, 8192 tokens (stored as 64 x 128), 20 Sinkhorn iterations.
MHC = dict(n=4, d=128, windows=64, seq=128, iters=20)


def mhc_bytes(n: int, d: int, T: int) -> tuple[int, int]:
    """Algorithmic HBM bytes per launch: every input, weight and output once.

    prepare: streams (T n d) + agg (T d) + pre, post (T n) + res (T n n) in
             fp32, proj weights (2n + n^2) d in fp64, norm weight d, biases.
    combine: streams (T n d) + res + post + out (T d) read, new streams written.
    """
    f = 4
    prepare = T * n * d * f + T * d * f + 2 * T * n * f + T * n * n * f + (2 * n + n * n) * d * 8 + d * f + \
        (2 * n + n * n) * f + 3 * f
    combine = T * n * d * f + T * n * n * f + T * n * f + T * d * f + T * n * d * f
    return prepare, combine


def cpu_baseline_mhc(cfg: dict, budget_s: float = 12.0) -> dict:
    """The reference's own CPU kernels (oracle/_ref) on the same workload (the oracle port where that library
    is absent)."""
    import numpy as np

    from oracle import Oracle, Reference, reference_available

    n, d, T = cfg["n"], cfg["d"], cfg["windows"] * cfg["seq"]
    rng = np.random.default_rng(0)
    s = rng.standard_normal((cfg["windows"], cfg["seq"], n, d)).astype(np.float32)
    nw = (rng.random(d) + 0.5).astype(np.float32)
    pw = (rng.standard_normal((2 * n + n * n, d)) / np.sqrt(d)).astype(np.float64)
    pb, qb = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    rb = rng.standard_normal((n, n)).astype(np.float32)
    ref = reference_available()
    lib = Reference() if ref else Oracle()

    def make_step(threads):
        if ref:
            lib.set_threads(threads)

        def step():
            agg, pre, post, res = lib.mhc_prepare(s, nw, 1e-5, pw, pb, qb, rb, 0.7, 0.7, 0.7, cfg["iters"])
            lib.mhc_combine(s, res, post, agg)
        return step

    line = _cpu_legs(make_step, T, "tokens/s", "reference" if ref else "port",
                     f"full steps (prepare + combine, {T} tokens each) in the "
                     f"{'reference ' + lib.variant if ref else 'oracle'} build, OpenMP threads = torch threads",
                     budget_s)
    return line


def _graph(fn_list, prerun: bool = True):
    """Capture the given launch closures, in order, into one HIP graph (after one eager run of them on a
    side stream, unless `prerun` is false: every kernel they launch must then have run once already)."""
    import torch

    if prerun:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for fn in fn_list:
                fn()
        torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for fn in fn_list:
            fn()
    return g


def _upload(g) -> None:
    """hipGraphUpload of an instantiated graph on the current stream, so that its first replay launches the
    prepared graph (kernel arguments and packets already set up on the device) rather than preparing it
    inside the timed region. Runs none of the graph's work."""
    import ctypes

    import torch

    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipGraphUpload.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    hip.hipGraphUpload.restype = ctypes.c_int
    rc = hip.hipGraphUpload(ctypes.c_void_p(g.raw_cuda_graph_exec()),
                            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    if rc != 0:
        raise RuntimeError(f"hipGraphUpload failed with HIP error {rc}")
    torch.cuda.synchronize()


def _time_graph(g, replays: int) -> float:
    """Milliseconds per replay, HIP events on the replay stream."""
    import torch

    stream = torch.cuda.current_stream()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(replays):
        g.replay()
    stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / replays


def _gpu_steps(step_fns, steps: int, warmup: int, budget_s: float = 10.0) -> dict:
    """Times exactly `steps` steps; step i runs step_fns[i % len(step_fns)].

    The `steps` steps are captured, in order, into one HIP graph (capture runs nothing; the caller has run
    every step function once). The warm-up runs `warmup` steps back to back right before the timed region:
    as one replay of a graph of warmup % steps steps (those just before the timed graph's first in the
    rotation of step functions) and warmup // steps replays of the timed graph itself (so the timed replay
    is not its first launch when warmup >= steps). The timed region is one replay of the `steps`-step graph between two HIP events,
    synchronized on both sides, no host work between the steps; ms_per_step is its time / steps. Further
    replays of the same graph (30, or as many as fit in `budget_s`, at least 3) give the median and the
    spread of the per-step time. With several step functions the timed steps continue the warm-up's
    rotation only when steps is a multiple of their count (as in every workload here)."""
    import statistics

    import torch

    n = len(step_fns)
    g = _graph([step_fns[i % n] for i in range(steps)], prerun=False)
    _upload(g)
    full, rest = divmod(warmup, steps)
    if rest > 0:  # the steps just before the timed graph's first in the rotation
        wg = _graph([step_fns[(i - rest) % n] for i in range(rest)], prerun=False)
        _upload(wg)
        wg.replay()
    for _ in range(full):
        g.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    g.replay()
    stop.record(stream)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(stop)

    reps = 30 if 30 * total_ms * 1e-3 <= budget_s else max(3, int(budget_s / max(total_ms * 1e-3, 1e-9)))
    per = []
    for _ in range(reps):
        start.record(stream)
        g.replay()
        stop.record(stream)
        torch.cuda.synchronize()
        per.append(start.elapsed_time(stop) / steps)
    per.sort()
    return {"steps": steps, "ms_per_step": total_ms / steps, "timed_region_ms": total_ms,
            "median_ms_per_step": statistics.median(per), "p10_ms_per_step": per[int(0.1 * (reps - 1))],
            "p90_ms_per_step": per[int(0.9 * (reps - 1))], "median_replays": reps}


def _floor_ms(shapes, steps: int) -> float:
    """Milliseconds per step of a HIP graph holding `steps` steps of empty kernels in the given launch shapes
    (blocks, threads, dynamic LDS bytes): the floor a step of launches in those shapes pays before any work."""
    from montlok import _C

    g = _graph([lambda s=s: _C.empty_kernel(*s) for _ in range(steps) for s in shapes])
    _upload(g)
    g.replay()
    return _time_graph(g, 10) / steps


def _timing_fields(t: dict) -> dict:
    return {k: t[k] for k in ("timed_region_ms", "median_ms_per_step", "p10_ms_per_step", "p90_ms_per_step",
                              "median_replays")}


MFMA_PEAK_TFS = {"bf16": 2500.0, "f32": 157.3}
RIDGE = {k: v * 1e3 / HBM_PEAK_GBS for k, v in MFMA_PEAK_TFS.items()}  # flop per byte


def _op_times(ops: dict, replays: int, reps: int = 8) -> dict:
    """Per-op milliseconds per launch: each op captured `reps` times in its own graph and replayed. An op
    given as a list of closures ("fns", one per input set) rotates over them, so its inputs are as cold as
    in the timed steps."""
    times = {}
    for name, op in ops.items():
        fns = op.get("fns") or [op["fn"]]
        g = _graph([fns[i % len(fns)] for i in range(max(reps, len(fns)))])
        for _ in range(2):
            g.replay()
        times[name] = _time_graph(g, replays) / max(reps, len(fns))
    return times


def _kernel_table(ops: dict, times: dict, precision: str) -> dict:
    table = {}
    for name, op in ops.items():
        ms = times[name]
        entry = {"launch_ms": ms, "algorithmic_bytes": op["bytes"], "achieved_GBs": op["bytes"] / (ms * 1e-3) / 1e9}
        if op.get("flops"):
            entry["flops"] = op["flops"]
            entry["achieved_TFs"] = op["flops"] / (ms * 1e-3) / 1e12
            entry["mfma_frac"] = entry["achieved_TFs"] / MFMA_PEAK_TFS[op.get("precision", precision)]
        entry["hbm_frac"] = entry["achieved_GBs"] / HBM_PEAK_GBS
        table[name] = entry
    return table


def _roofline(name: str, entry: dict, op: dict, precision: str, traffic=None) -> dict:
    """HBM or MFMA roofline of one kernel, whichever its arithmetic intensity makes binding."""
    prec = op.get("precision", precision)
    flops = op.get("flops") or 0
    if flops and flops / op["bytes"] > RIDGE[prec]:
        return {"bound": "mfma", "kernel": name, "achieved": entry["achieved_TFs"], "peak": MFMA_PEAK_TFS[prec],
                "unit": "TFLOP/s", "frac": entry["mfma_frac"], "traffic": traffic, "algorithmic_flops": flops,
                "launch_ms": entry["launch_ms"]}
    return {"bound": "hbm", "kernel": name, "achieved": entry["achieved_GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": entry["hbm_frac"], "traffic": traffic, "algorithmic_bytes": op["bytes"],
            "launch_ms": entry["launch_ms"]}


def _traffic(tag: str, kernel: str):
    """HBM bytes per launch of `kernel` from the committed counter summary profiles/<tag>_traffic.json
    (FETCH_SIZE and WRITE_SIZE passes of rocprofv3 over this workload, scaled by a plain copy's), or None."""
    path = ROOT / "profiles" / f"{tag}_traffic.json"
    if not path.exists():
        return None
    return json.loads(path.read_text()).get(kernel)


def _base_line(value, unit, steps, warmup, ms, dtype, data, config) -> dict:
    return {"metric": METRIC, "value": value, "unit": unit, "n_gpus": 1, "steps": steps, "warmup": warmup,
            "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
            "data": data, "config": config}


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_median(fn, budget_s: float, warmup: int = 5, min_samples: int = 30) -> tuple[float, int, float]:
    """The reference harness's procedure (tools/rdt/bench_montlok_kernel.py:90-107): `warmup` untimed calls,
    then timed calls until there are `min_samples` of them and `budget_s` has passed (at most 2 x budget_s);
    returns (median seconds per call, samples, seconds spent)."""
    import statistics

    for _ in range(warmup):
        fn()
    samples, t_all = [], time.perf_counter()
    while True:
        t0 = time.perf_counter()
        fn()
        samples.append(time.perf_counter() - t0)
        spent = time.perf_counter() - t_all
        if (len(samples) >= min_samples and spent >= budget_s) or spent >= 2 * budget_s or len(samples) >= 100000:
            return statistics.median(samples), len(samples), spent


def _cpu_legs(make_step, units: float, unit: str, kind: str, sample: str, budget_s: float) -> dict:
    """Times `make_step(threads)` with every host core and with one thread, FTZ/DAZ on (torch's flag, as the
    reference harness sets it, bench_montlok_kernel.py:264-265; the reference recurrence sets its own guard,
    montlok_kernel.h:439). `units` windows (or streams) per step."""
    import torch

    cores = len(os.sched_getaffinity(0))
    torch.set_flush_denormal(True)
    legs = {}
    for threads in (cores, 1):
        torch.set_num_threads(threads)
        med, n, spent = _cpu_median(make_step(threads), budget_s / 2)
        legs[threads] = (units / med, n, spent, med)
    torch.set_num_threads(cores)
    value, n, spent, med = legs[cores]
    return {"value": value, "unit": unit, "cores": cores, "kind": kind,
            "sample": f"{sample}; median of {n} steps after 5 warm-up ({med * 1e3:.3f} ms per step, {spent:.1f} s), "
                      f"FTZ/DAZ on",
            "one_thread_value": legs[1][0],
            "one_thread_sample": f"median of {legs[1][1]} steps after 5 warm-up ({legs[1][3] * 1e3:.3f} ms per step)",
            "cpu_model": _cpu_model(), "torch_threads": cores}


# ---------------------------------------------------------------- workloads


def bench_mhc(steps: int, warmup: int, cpu: bool) -> dict:
    import torch

    from montlok import _C

    cfg = MHC
    n, d, W, L, iters = cfg["n"], cfg["d"], cfg["windows"], cfg["seq"], cfg["iters"]
    T = W * L
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(0)
    sets = 16  # 16 x 16 MiB of streams > the 256 MB Infinity Cache
    streams = [torch.randn(W, L, n, d, generator=g).to(dev) for _ in range(sets)]
    norm_w = (torch.rand(d, generator=g) + 0.5).to(dev)
    proj_w = (torch.randn(2 * n + n * n, d, generator=g, dtype=torch.float64) / d ** 0.5).to(dev)
    pre_b = torch.randn(n, generator=g).to(dev)
    post_b = torch.randn(n, generator=g).to(dev)
    res_b = torch.randn(n, n, generator=g).to(dev)
    alphas = [torch.tensor(0.7, device=dev) for _ in range(3)]
    outs = [torch.empty(W, L, n, d, device=dev) for _ in range(sets)]
    agg = [torch.empty(W, L, d, device=dev) for _ in range(sets)]
    pre = [torch.empty(W, L, n, device=dev) for _ in range(sets)]
    post = [torch.empty(W, L, n, device=dev) for _ in range(sets)]
    res = [torch.empty(W, L, n, n, device=dev) for _ in range(sets)]
    lib = _C.library()
    ptr = lambda t: t.data_ptr()  # noqa: E731

    def prepare(i):
        def run():
            st = lib.mlk_mhc_prepare(ptr(streams[i]), T, n, d, d, n * d, ptr(norm_w), 1e-5, ptr(proj_w), ptr(pre_b),
                                     ptr(post_b), ptr(res_b), ptr(alphas[0]), ptr(alphas[1]), ptr(alphas[2]), iters,
                                     None, 0.0, ptr(agg[i]), ptr(pre[i]), ptr(post[i]), ptr(res[i]),
                                     torch.cuda.current_stream().cuda_stream)
            if st != 0:
                raise RuntimeError(lib.mlk_last_error().decode())
        return run

    def combine(i):
        def run():
            st = lib.mlk_mhc_combine(ptr(streams[i]), T, n, d, d, n * d, ptr(res[i]), ptr(post[i]), ptr(agg[i]),
                                     ptr(outs[i]), None, torch.cuda.current_stream().cuda_stream)
            if st != 0:
                raise RuntimeError(lib.mlk_last_error().decode())
        return run

    def step(i):
        p, c = prepare(i), combine(i)

        def run():
            p()
            c()
        return run

    # Correctness guard on the timed configuration before timing: eager run, then the graphs, bit-identical.
    step(0)()
    torch.cuda.synchronize()
    eager = outs[0].clone()
    assert torch.isfinite(eager).all().item()
    t = _gpu_steps([step(i) for i in range(sets)], steps, warmup)
    assert torch.equal(outs[0], eager), "graph replay differs from the eager step"
    ms_per_step = t["ms_per_step"]
    # Per-kernel launch times: 16 launches of one kernel over the 16 sets in one graph, replayed.
    replays = max(4, steps // sets)
    prep_ms = _time_graph(_graph([prepare(i) for i in range(sets)]), replays) / sets
    comb_ms = _time_graph(_graph([combine(i) for i in range(sets)]), replays) / sets

    prep_bytes, comb_bytes = mhc_bytes(n, d, T)
    kernels = {"mhc_prepare": (prep_ms, prep_bytes), "mhc_combine": (comb_ms, comb_bytes)}
    dom = max(kernels, key=lambda k: kernels[k][0])
    dom_ms, dom_bytes = kernels[dom]
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
    traffic = _traffic("mhc_n4_d128_t8192", dom)
    line = _base_line(T / (ms_per_step * 1e-3), "tokens/s", t["steps"], warmup, ms_per_step, "f32 (f64 accumulate)",
                      "synthetic (seeded N(0,1) streams, random-init mHC weights)",
                      {"workload": "mhc_residual_mix", "n_streams": n, "d_model": d, "tokens": T,
                       "sinkhorn_iters": iters, "step": "mhc_prepare + identity fn + mhc_combine",
                       "launch": "the K steps in one HIP graph, rotating over 16 independent input sets (cold HBM)",
                       "parallelism": "single GPU"})
    line["roofline"] = {"bound": "hbm", "kernel": dom, "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": achieved / HBM_PEAK_GBS, "traffic": traffic, "algorithmic_bytes": dom_bytes,
                        "launch_ms": dom_ms}
    line["kernels"] = {k: {"launch_ms": v[0], "algorithmic_bytes": v[1], "achieved_GBs": v[1] / (v[0] * 1e-3) / 1e9}
                       for k, v in kernels.items()}
    line.update(_timing_fields(t))
    line["step_roofline_frac"] = (prep_bytes + comb_bytes) / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS
    line["stream_steps_per_s"] = n * T / (ms_per_step * 1e-3)
    if cpu:
        line["cpu_baseline"] = cpu_baseline_mhc(cfg)
        line["cpu_baseline"]["gpu_over_cpu"] = line["value"] / line["cpu_baseline"]["value"]
    return line


# ------------------------------------------------------------ Mamba-3 block

# RMSNorm -> Mamba-3 block, fp32: 64 windows x 32 tokens, d_model 64, 4 heads, d_state 16, expand 2.
BLOCK = dict(windows=64, seq=32, d_model=64, d_state=16, headdim=32, expand=2, norm_groups=8)


def _mamba_geometry(d_model: int, d_state: int, headdim: int, expand: int) -> dict:
    """Mamba-3 geometry: d_inner = expand d_model, H = d_inner / headdim, R = d_state / 4 rotary angles
    (rope fraction 0.5, mamba3.py:121-124), in_proj width 2 d_inner + 2 N + 3 H + R (one B/C group)."""
    d_inner = expand * d_model
    H = d_inner // headdim
    R = ((d_state // 2) // 2 * 2) // 2
    return dict(d_inner=d_inner, H=H, N=d_state, D=headdim, R=R, G=1, W=2 * d_inner + 2 * d_state + 3 * H + R)


def _mamba_weights(g, d_model: int, geo: dict, dev, dtype=None):
    """nn.Linear default (Kaiming-uniform) projections; dt_bias so softplus(dt_bias) is log-uniform in
    [1e-3, 1e-1] (mamba3.py:128-130); B/C biases, B/C norm weights and D at their init (ones)."""
    import math

    import torch

    W, d_inner, H, N = geo["W"], geo["d_inner"], geo["H"], geo["N"]
    b_in, b_out = 1 / math.sqrt(d_model), 1 / math.sqrt(d_inner)
    in_w = (torch.rand(W, d_model, generator=g) * 2 - 1) * b_in
    out_w = (torch.rand(d_model, d_inner, generator=g) * 2 - 1) * b_out
    dt = torch.exp(torch.rand(H, generator=g) * (math.log(1e-1) - math.log(1e-3)) + math.log(1e-3))
    dt_bias = dt + torch.log(-torch.expm1(-dt))
    params = dict(in_w=in_w, out_w=out_w, b_bias=torch.ones(H, N), c_bias=torch.ones(H, N), b_norm_w=torch.ones(N),
                  c_norm_w=torch.ones(N), dt_bias=dt_bias, skip=torch.ones(H))
    return {k: v.to(dev) if dtype is None or k not in ("in_w", "out_w") else v.to(dev, dtype)
            for k, v in params.items()}


MAMBA_PARAM_KEYS = ("b_bias", "c_bias", "b_norm_w", "c_norm_w", "dt_bias", "skip")


def cpu_baseline_block(cfg: dict, x_cpu, norm_w, weights: dict, geo: dict, budget_s: float = 12.0) -> dict:
    """Reference CPU kernels (oracle/_ref) for the norm and the mixer, torch CPU for the two GEMMs and the
    residual add, as the reference itself calls oneDNN / at::linear (montlok.cpp:67-91)."""
    import torch

    from oracle import Oracle, Reference, reference_available

    ref = reference_available()
    lib = Reference() if ref else Oracle()
    w = {k: v.cpu() for k, v in weights.items()}
    x = x_cpu.numpy()
    nw = norm_w.cpu().numpy()
    p = [w[k].numpy() for k in MAMBA_PARAM_KEYS]
    N, G, H, D, R = geo["N"], geo["G"], geo["H"], geo["D"], geo["R"]

    def make_step(threads):
        if ref:
            lib.set_threads(threads)

        def step():
            h = torch.from_numpy(lib.rms_norm(x, nw, 1e-5, cfg["norm_groups"]))
            proj = torch.nn.functional.linear(h, w["in_w"]).numpy()
            y = lib.mamba3_siso_forward(proj, N, G, H, D, R, *p[:4], 1e-5, 1e-5, p[4], p[5], 1e-4)
            return x_cpu + torch.nn.functional.linear(torch.from_numpy(y), w["out_w"])
        return step

    return _cpu_legs(make_step, cfg["windows"], "windows/s", "reference" if ref else "port",
                     f"full steps ({cfg['windows']} windows x {cfg['seq']} tokens); norm + mixer in the "
                     f"{'reference ' + lib.variant if ref else 'oracle'} build, GEMMs in torch CPU", budget_s)


def bench_block(steps: int, warmup: int, cpu: bool) -> dict:
    import torch

    from montlok import _C

    cfg = BLOCK
    geo = _mamba_geometry(cfg["d_model"], cfg["d_state"], cfg["headdim"], cfg["expand"])
    B, L, d = cfg["windows"], cfg["seq"], cfg["d_model"]
    T = B * L
    N, G, H, D, R, W, d_inner = (geo[k] for k in ("N", "G", "H", "D", "R", "W", "d_inner"))
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(0)
    x_cpu = torch.randn(B, L, d, generator=g)
    x = x_cpu.to(dev)
    norm_w = torch.ones(d, device=dev)
    wts = _mamba_weights(g, d, geo, dev)
    mp = [wts[k] for k in MAMBA_PARAM_KEYS]
    consts = (N, G, H, D, R, 1e-5, 1e-5, 1e-4)
    res = [None]
    block_args = (norm_w, 1e-5, cfg["norm_groups"], wts["in_w"], wts["out_w"], *mp, *consts)

    def step():
        res[0] = _C.mamba3_block(x, *block_args)

    step()
    torch.cuda.synchronize()
    eager = res[0].clone()
    unfused = x + _C.mamba3_siso_layer(_C.rms_norm(x, norm_w, 1e-5, cfg["norm_groups"]), wts["in_w"], wts["out_w"],
                                       *mp, *consts)
    assert torch.equal(eager, unfused), "block step differs from the separate operators"
    t = _gpu_steps([step], steps, warmup)
    assert torch.equal(res[0], eager), "graph replay differs from the eager step"
    ms = t["ms_per_step"]

    f = 4
    total_bytes = (2 * T * d + W * d + d * d_inner) * f + d * f
    total_flops = 2 * T * d * W + 7 * T * H * N * D + 2 * T * d_inner * d
    launches = _C.mamba3_block_launches()
    if launches[0] == "rms_norm_mamba3_forward":
        y = _C.rms_norm_mamba3_forward(x, norm_w, 1e-5, cfg["norm_groups"], wts["in_w"], *mp, *consts)
        ops = {
            # GroupedRMSNorm + in_proj + scan in one kernel: x and the in_proj weight in, y out.
            "rms_norm_mamba3_forward": dict(fn=lambda: _C.rms_norm_mamba3_forward(x, norm_w, 1e-5, cfg["norm_groups"],
                                                                                  wts["in_w"], *mp, *consts),
                                            bytes=(T * d + d + W * d + T * d_inner) * f,
                                            flops=2 * T * d * W + 7 * T * H * N * D),
            "out_proj_residual": dict(fn=lambda: _C.linear_residual(y, wts["out_w"], None, x),
                                      bytes=(T * d_inner + d * d_inner + 2 * T * d) * f, flops=2 * T * d_inner * d),
        }
    else:
        h = _C.rms_norm(x, norm_w, 1e-5, cfg["norm_groups"])
        proj = _C.linear(h, wts["in_w"])
        y = _C.mamba3_siso_forward(proj, None, *mp, *consts)
        ops = {
            "rms_norm_in_proj": dict(fn=lambda: _C.rms_norm_linear(x, norm_w, 1e-5, cfg["norm_groups"], wts["in_w"]),
                                     bytes=(T * d + d + W * d + T * W) * f, flops=2 * T * d * W),
            "mamba3_siso_forward": dict(fn=lambda: _C.mamba3_siso_forward(proj, None, *mp, *consts),
                                        bytes=(T * W + T * d_inner) * f, flops=7 * T * H * N * D),
            "out_proj_residual": dict(fn=lambda: _C.linear_residual(y, wts["out_w"], None, x),
                                      bytes=(T * d_inner + d * d_inner + 2 * T * d) * f, flops=2 * T * d_inner * d),
        }
    table = _kernel_table(ops, _op_times(ops, max(8, steps)), "f32")
    dom = max(table, key=lambda k: table[k]["launch_ms"])
    floor = None
    if launches == ["rms_norm_mamba3_forward", "linear_residual"]:
        # The graph-node floor of the step: empty kernels in the two launches' shapes (the mixer: a block of
        # 8 waves per (window, head) with its dynamic LDS; the out_proj: a wave per 16 x 16 output tile).
        mixer = (B * H, 256, 4 * 32 * ((W + 15) // 16 * 16 + 4))
        out_proj = (-(-T // 16) * -(-d // 16), 64, 0)
        floor = {name: _floor_ms([shape], steps) for name, shape in (("mixer", mixer), ("out_proj", out_proj))}
        floor["step"] = _floor_ms([mixer, out_proj], steps)
        floor["ms_per_step_over_floor"] = ms / floor["step"]
        floor["shapes"] = {"mixer": list(mixer), "out_proj": list(out_proj)}
    line = _base_line(B / (ms * 1e-3), "windows/s", t["steps"], warmup, ms, "f32",
                      "synthetic (seeded N(0,1) inputs, Kaiming-uniform weights, dt bias per mamba3.py:128-130)",
                      {"workload": "rmsnorm_mamba3_block", "windows": B, "seq_len": L, "d_model": d, "heads": H,
                       "d_state": N, "headdim": D, "rope_angles": R, "expand": cfg["expand"],
                       "norm_groups": cfg["norm_groups"], "step": "x + out_proj(mamba3(in_proj(GroupedRMSNorm(x))))",
                       "launches": ", ".join(launches), "launch": "the K steps in one HIP graph",
                       "parallelism": "single GPU"})
    line["roofline"] = _roofline(dom, table[dom], ops[dom], "f32", _traffic("mamba3_block_b64_l32_d64", dom))
    line["kernels"] = table
    line.update(_timing_fields(t))
    line["step_algorithmic_bytes"] = total_bytes
    line["step_algorithmic_flops"] = total_flops
    line["step_hbm_frac"] = total_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS
    line["step_fp32_frac"] = total_flops / (ms * 1e-3) / 1e12 / MFMA_PEAK_TFS["f32"]
    line["tokens_per_s"] = T / (ms * 1e-3)
    if floor is not None:
        line["graph_node_floor_ms"] = floor
    if cpu:
        line["cpu_baseline"] = cpu_baseline_block(cfg, x_cpu, norm_w, wts, geo)
        line["cpu_baseline"]["gpu_over_cpu"] = line["value"] / line["cpu_baseline"]["value"]
    return line


# --------------------------------------------------------------------- MLA

# MLA causal self-attention fwd: 256 windows x 128 tokens, d_model 256, 8 heads of 32 (RoPE slice 16,
# base 10000), KV latent rank 64, bf16 weights N(0, 0.02), fp32 inputs and accumulation.
MLA = dict(windows=256, seq=128, d_model=256, heads=8, head_dim=32, rope=16, kv_rank=64, theta=10000.0)


def rope_tables(length: int, rope_dim: int, theta: float):
    """Token-index RoPE tables, built with torch on the CPU as the reference does
    (reference/Model/layers/rope.py:9-16, 138-166)."""
    import torch

    idx = torch.arange(0, rope_dim, 2, dtype=torch.float32)
    freqs = 1.0 / (theta ** (idx / rope_dim))
    angles = torch.arange(0, length, dtype=torch.float32).unsqueeze(-1) * freqs.unsqueeze(0)
    emb = torch.cat([angles, angles], dim=-1)
    return emb.cos(), emb.sin()


def cpu_baseline_mla(cfg: dict, x_cpu, w: dict, cos, sin, budget_s: float = 12.0, windows: int = 16) -> dict:
    """torch CPU for the GEMMs and SDPA (the reference calls oneDNN and at::scaled_dot_product_attention,
    montlok.cpp:1187-1210), reference CPU kernels for the latent LayerNorm and the rotary step."""
    import torch
    import torch.nn.functional as F

    from oracle import Oracle, Reference, reference_available

    ref = reference_available()
    lib = Reference() if ref else Oracle()
    H, hd, r, kvr = cfg["heads"], cfg["head_dim"], cfg["rope"], cfg["kv_rank"]
    nope = hd - r
    x = x_cpu[:windows].contiguous()
    B, L, d = x.shape
    wf = {k: v.float().cpu() for k, v in w.items()}
    cosn, sinn = cos.numpy(), sin.numpy()
    scale = 1.0 / hd ** 0.5

    def make_step(threads):
        if ref:
            lib.set_threads(threads)

        def step():
            projected = F.linear(x, wf["in_w"])
            q = projected[..., :d].reshape(B, L, H, hd).numpy()
            kv_lat = projected[..., d:d + kvr].contiguous().numpy()
            k_rope = projected[..., d + kvr:].contiguous().numpy()
            kvn = torch.from_numpy(lib.layer_norm(kv_lat, wf["ln_w"].numpy(), wf["ln_b"].numpy(), 1e-5))
            kv = F.linear(kvn, wf["kv_up"]).reshape(B, L, H, nope + hd)
            q, k = lib.mla_rope(q, kv.numpy(), k_rope, cosn, sinn, nope)
            att = F.scaled_dot_product_attention(torch.from_numpy(q).transpose(1, 2),
                                                 torch.from_numpy(k).transpose(1, 2), kv[..., nope:].transpose(1, 2),
                                                 is_causal=True, scale=scale)
            return F.linear(att.transpose(1, 2).reshape(B, L, d), wf["o"])
        return step

    return _cpu_legs(make_step, windows, "windows/s", "reference" if ref else "port",
                     f"steps over {windows} of the {cfg['windows']} windows (the rate scales per window); LayerNorm "
                     f"+ RoPE in the {'reference ' + lib.variant if ref else 'oracle'} build, GEMMs and SDPA in "
                     f"torch CPU (fp32, bf16 weights upcast)", budget_s)


def bench_mla(steps: int, warmup: int, cpu: bool) -> dict:
    import torch

    from montlok import _C

    cfg = MLA
    B, L, d, H, hd, r, kvr = (cfg[k] for k in ("windows", "seq", "d_model", "heads", "head_dim", "rope", "kv_rank"))
    nope = hd - r
    T = B * L
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(0)
    sets = 8  # 8 x 32 MiB inputs plus the intermediates exceed the 256 MB Infinity Cache
    x_cpu = torch.randn(B, L, d, generator=g)
    xs = [x_cpu.to(dev)] + [torch.randn(B, L, d, generator=g).to(dev) for _ in range(sets - 1)]
    bf = torch.bfloat16
    w_cpu = dict(in_w=(torch.randn(d + kvr + r, d, generator=g) * 0.02).to(bf),
                 kv_up=(torch.randn(H * (nope + hd), kvr, generator=g) * 0.02).to(bf),
                 o=(torch.randn(d, H * hd, generator=g) * 0.02).to(bf), ln_w=torch.ones(kvr), ln_b=torch.zeros(kvr))
    w = {k: v.to(dev) for k, v in w_cpu.items()}
    cos_cpu, sin_cpu = rope_tables(L, r, cfg["theta"])
    cos, sin = cos_cpu.to(dev), sin_cpu.to(dev)
    empty = torch.empty(0, device=dev)
    scale = 1.0 / hd ** 0.5
    outs = [None] * sets

    def step(i):
        def run():
            outs[i] = _C.mla_forward(xs[i], w["in_w"], empty, w["ln_w"], w["ln_b"], 1e-5, w["kv_up"], w["o"], cos, sin,
                                     H, hd, nope, kvr, L, True, scale)
        return run

    step(0)()
    torch.cuda.synchronize()
    launches = _C.mla_forward_launches()
    eager = outs[0].clone()
    assert torch.isfinite(eager).all().item()
    separate = _C._mla_forward(xs[0], w["in_w"], empty, w["ln_w"], w["ln_b"], 1e-5, w["kv_up"], w["o"], cos, sin, H,
                               hd, nope, kvr, L, True, scale, allow_fused=True, allow_window=False)
    assert torch.equal(eager, separate), "the step must equal the four-launch path bit for bit"
    t = _gpu_steps([step(i) for i in range(sets)], steps, warmup)
    assert torch.equal(outs[0], eager), "graph replay differs from the eager step"
    steps, ms = t["steps"], t["ms_per_step"]

    # Per-kernel launches on each input set's intermediates, rotating over the sets as the steps do.
    projs = [_C.linear(xs[i], w["in_w"]).view(T, d + kvr + r) for i in range(sets)]
    lats = [_C._latent_normed(projs[i], d, kvr, w["ln_w"], w["ln_b"], 1e-5) for i in range(sets)]
    atts = [_C._attend_normed(projs[i], lats[i], B, L, d, H, hd, nope, kvr, w["kv_up"], cos, sin, scale).view(B, L, d)
            for i in range(sets)]
    f, h2 = 4, 2
    pairs = B * H * L * (L + 1) // 2
    total_bytes = 2 * T * d * f + ((d + kvr + r) * d + H * (nope + hd) * kvr + d * d) * h2
    separate_ops = {
        "in_proj": dict(fns=[lambda i=i: _C.linear(xs[i], w["in_w"]) for i in range(sets)],
                        bytes=T * d * f + (d + kvr + r) * d * h2 + T * (d + kvr + r) * f,
                        flops=2 * T * d * (d + kvr + r)),
        # The latent's LayerNorm once per row, to bf16.
        "latent_layer_norm": dict(fns=[lambda i=i: _C._latent_normed(projs[i], d, kvr, w["ln_w"], w["ln_b"], 1e-5)
                                       for i in range(sets)],
                                  bytes=T * kvr * (f + h2) + 2 * kvr * f),
        # kv_up + RoPE + causal attention in one kernel: q, the normalised latent and k_rope in, attention out.
        "mla_attend": dict(fns=[lambda i=i: _C._attend_normed(projs[i], lats[i], B, L, d, H, hd, nope, kvr, w["kv_up"],
                                                              cos, sin, scale) for i in range(sets)],
                           bytes=T * (d + r) * f + T * kvr * h2 + H * (nope + hd) * kvr * h2 + T * d * f,
                           flops=2 * T * kvr * H * (nope + hd) + 4 * pairs * hd),
        "o_proj": dict(fns=[lambda i=i: _C.linear(atts[i], w["o"]) for i in range(sets)],
                       bytes=2 * T * d * f + d * d * h2, flops=2 * T * d * d),
    }
    total_flops = sum(op.get("flops", 0) for op in separate_ops.values())
    if launches == ["mla_forward"]:
        # The whole forward in one kernel: x in, the output projection out, the bf16 weights once.
        ops = {"mla_forward": dict(fns=[step(i) for i in range(sets)], bytes=total_bytes, flops=total_flops)}
    else:
        ops = separate_ops
    table = _kernel_table(ops, _op_times(ops, max(4, steps // 8)), "bf16")
    dom = max(table, key=lambda k: table[k]["launch_ms"])
    line = _base_line(B / (ms * 1e-3), "windows/s", steps, warmup, ms, "bf16 weights and contraction operands, fp32 accumulate",
                      "synthetic (seeded N(0,1) inputs, N(0,0.02) bf16 weights)",
                      {"workload": "mla_causal_fwd", "windows": B, "seq_len": L, "d_model": d, "heads": H,
                       "head_dim": hd, "rope_dim": r, "kv_rank": kvr, "rope_theta": cfg["theta"],
                       "step": "mla_forward: in_proj, latent LayerNorm, kv_up, RoPE, causal attention, o_proj",
                       "launches": ", ".join(launches),
                       "launch": f"the K steps in one HIP graph, rotating over {sets} input sets",
                       "parallelism": "single GPU"})
    line["roofline"] = _roofline(dom, table[dom], ops[dom], "bf16", _traffic("mla_b256_l128_d256_h8", dom))
    line["kernels"] = table
    if ops is not separate_ops:  # the four-launch path the kernel replaces, for comparison
        line["separate_path_kernels"] = _kernel_table(separate_ops, _op_times(separate_ops, max(4, steps // 8)),
                                                      "bf16")
    line.update(_timing_fields(t))
    line["step_algorithmic_bytes"] = total_bytes
    line["step_algorithmic_flops"] = total_flops
    line["step_hbm_frac"] = total_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS
    line["step_mfma_frac"] = total_flops / (ms * 1e-3) / 1e12 / MFMA_PEAK_TFS["bf16"]
    if cpu:
        line["cpu_baseline"] = cpu_baseline_mla(cfg, x_cpu, w_cpu, cos_cpu, sin_cpu)
        line["cpu_baseline"]["gpu_over_cpu"] = line["value"] / line["cpu_baseline"]["value"]
    return line


# ---------------------------------------------------------- streaming decode

# 65536 streams, one bar each through 2 Mamba-3 layers (d_model 128, d_state 64, 4 heads of 64, expand 2),
# then RMSNorm and a Linear(128 -> 1) head; fp32 weights and state. State init: ssm, k, v ~ N(0, 0.1),
# rotary phase ~ U[0, 2 pi) (fp64), mid-sequence (started).
DECODE = dict(streams=65536, layers=2, d_model=128, d_state=64, headdim=64, expand=2, norm_groups=8)


def _decode_state_bytes(S: int, geo: dict) -> int:
    H, N, D, R = geo["H"], geo["N"], geo["D"], geo["R"]
    return S * H * ((N * D + N + D) * 4 + max(R, 1) * 8)


def cpu_baseline_decode(cfg: dict, geo: dict, stack, states: list, x_cpu, budget_s: float = 12.0,
                        streams: int = 1024) -> dict:
    """No reference step operator exists: the oracle's step restatement for the mixer, its streams split over
    OpenMP threads, the reference CPU RMSNorm and torch CPU GEMMs, on the first `streams` streams."""
    import numpy as np
    import torch

    from oracle import Oracle, Reference, reference_available

    orc = Oracle()
    ref = Reference() if reference_available() else orc
    N, G, H, D, R = geo["N"], geo["G"], geo["H"], geo["D"], geo["R"]
    x = x_cpu[:streams].contiguous()
    st = [{"ssm": s["ssm"][:streams].cpu().numpy().copy(), "k_prev": s["k"][:streams].cpu().numpy().copy(),
           "v_prev": s["v"][:streams].cpu().numpy().copy(), "angle": s["angle"][:streams].cpu().numpy().copy(),
           "started": 1} for s in states]
    f32 = lambda t: t.detach().float().cpu()  # noqa: E731
    layers = [dict(norm=f32(b.norm.weight).numpy(), in_w=f32(b.mamba.in_proj.weight), out_w=f32(b.mamba.out_proj.weight),
                   p=[f32(t).numpy() for t in b.mamba._mixer_args()]) for b in stack.layers]
    fw, hw, hb = (f32(t) for t in (stack.final_norm.weight, stack.head.weight, stack.head.bias))

    def make_step(threads):
        if isinstance(ref, Reference):
            ref.set_threads(threads)

        def mixer(proj, state, p):
            return orc.mamba3_step(proj, state, N, G, H, D, R, *p[:4], 1e-5, 1e-5, p[4], p[5], 1e-4, threads=threads)

        def step():
            hcur = x
            for lw, s_l in zip(layers, st):
                nrm = ref.rms_norm(hcur.numpy(), lw["norm"], 1e-5, cfg["norm_groups"])
                proj = torch.nn.functional.linear(torch.from_numpy(nrm), lw["in_w"]).numpy()
                y = mixer(proj, s_l, lw["p"])
                hcur = hcur + torch.nn.functional.linear(torch.from_numpy(y), lw["out_w"])
            fin = torch.from_numpy(ref.rms_norm(hcur.numpy(), fw.numpy(), 1e-5, 1))
            return torch.nn.functional.linear(fin, hw, hb)
        return step

    return _cpu_legs(make_step, streams, "stream-steps/s", "port",
                     f"steps of {streams} of the {cfg['streams']} streams (the rate scales per stream); mixer step in "
                     f"the oracle's C restatement (no reference step operator exists), the streams split over OpenMP "
                     f"threads; RMSNorm in the {'reference' if isinstance(ref, Reference) else 'oracle'} build; GEMMs "
                     f"in torch CPU", budget_s)


def bench_decode(steps: int, warmup: int, cpu: bool) -> dict:
    import math

    import torch

    from montlok import _C
    from montlok.rdt.block import DecodeStackHIP

    cfg = DECODE
    S, d = cfg["streams"], cfg["d_model"]
    geo = _mamba_geometry(d, cfg["d_state"], cfg["headdim"], cfg["expand"])
    N, G, H, D, R, W, d_inner = (geo[k] for k in ("N", "G", "H", "D", "R", "W", "d_inner"))
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(0)
    x_cpu = torch.randn(S, d, generator=g)
    x = x_cpu.to(dev)
    stack = DecodeStackHIP(d_model=d, n_layers=cfg["layers"], d_state=N, expand=cfg["expand"], headdim=D,
                           num_groups=cfg["norm_groups"]).eval()
    with torch.no_grad():
        for block in stack.layers:
            w = _mamba_weights(g, d, geo, "cpu")
            m = block.mamba
            m.in_proj.weight.copy_(w["in_w"])
            m.out_proj.weight.copy_(w["out_w"])
            m.dt_bias.copy_(w["dt_bias"])
        bound = 1 / math.sqrt(d)
        stack.head.weight.copy_((torch.rand(1, d, generator=g) * 2 - 1) * bound)
        stack.head.bias.copy_((torch.rand(1, generator=g) * 2 - 1) * bound)
    stack = stack.to(dev)
    states = stack.new_state(S, dev)
    for st in states:
        st["ssm"].normal_(0.0, 0.1)
        st["k"].normal_(0.0, 0.1)
        st["v"].normal_(0.0, 0.1)
        st["angle"].uniform_(0.0, 2 * math.pi)
        st["started"] = True
    states_cpu = [{k: (v.cpu() if torch.is_tensor(v) else v) for k, v in st.items()} for st in states]
    result = {}

    def step():
        result["out"] = stack.step(x, states)

    # One eager step checks the path and leaves the state one bar further; the CPU leg starts from the
    # initial state copied above.
    with torch.no_grad():
        step()
        torch.cuda.synchronize()
        assert torch.isfinite(result["out"]).all().item()
        t = _gpu_steps([step], steps, warmup)
    steps, ms = t["steps"], t["ms_per_step"]

    blk = stack.layers[0]
    m = blk.mamba
    mp = m._mixer_args()
    consts = m._geometry()
    proj = _C.rms_norm_linear(x, blk.norm.weight, 1e-5, cfg["norm_groups"], m.in_proj.weight)
    y = _C.mamba3_siso_step(proj, states[0], *mp, *consts)
    f = 4
    state_bytes = _decode_state_bytes(S, geo)
    ops = {
        "rms_norm_in_proj": dict(fn=lambda: _C.rms_norm_linear(x, blk.norm.weight, 1e-5, cfg["norm_groups"],
                                                               m.in_proj.weight),
                                 bytes=(S * d + W * d + S * W) * f, flops=2 * S * d * W, precision="f32"),
        "mamba3_siso_step": dict(fn=lambda: _C.mamba3_siso_step(proj, states[0], *mp, *consts),
                                 bytes=2 * state_bytes + (S * W + S * d_inner) * f),
        "out_proj_residual": dict(fn=lambda: _C.linear_residual(y, m.out_proj.weight, None, x),
                                  bytes=(S * d_inner + d * d_inner + 2 * S * d) * f, flops=2 * S * d_inner * d,
                                  precision="f32"),
    }
    # Six launches per graph: with two, each replay's start-up cost (about 0.2 ms at these sizes) lands on
    # the per-launch time.
    table = _kernel_table(ops, _op_times(ops, max(4, steps // 4), reps=6), "f32")
    dom = max(table, key=lambda k: table[k]["launch_ms"])
    total_bytes = cfg["layers"] * (2 * state_bytes + (W * d + d * d_inner) * f) + S * d * f + S * f
    line = _base_line(S / (ms * 1e-3), "stream-steps/s", steps, warmup, ms, "f32 (fp64 rotary phase)",
                      "synthetic (seeded N(0,1) bar inputs, Kaiming-uniform weights, state ~ N(0,0.1))",
                      {"workload": "streaming_decode", "streams": S, "layers": cfg["layers"], "d_model": d,
                       "d_state": N, "heads": H, "headdim": D, "rope_angles": R, "norm_groups": cfg["norm_groups"],
                       "step": "2 x [x + out_proj(mamba3_step(in_proj(GroupedRMSNorm(x))))], RMSNorm, Linear(128->1)",
                       "launch": "the K steps in one HIP graph (state carried in place)",
                       "parallelism": "single GPU"})
    line["roofline"] = _roofline(dom, table[dom], ops[dom], "f32", _traffic("decode_s65536_2layers_d128_n64", dom))
    line["kernels"] = table
    line.update(_timing_fields(t))
    line["step_algorithmic_bytes"] = total_bytes
    line["step_hbm_frac"] = total_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS
    line["state_bytes_per_layer"] = state_bytes
    if cpu:
        line["cpu_baseline"] = cpu_baseline_decode(cfg, geo, stack, states_cpu, x_cpu)
        line["cpu_baseline"]["gpu_over_cpu"] = line["value"] / line["cpu_baseline"]["value"]
    return line


# ------------------------------------------------------------------- stack

# Full stack: 1024 windows x 256 tokens of 40 raw features (N(0,1) clipped to [-8, 8]) -> Linear(40 -> 256),
# 4 mHC residual layers (n = 4, 20 Sinkhorn iterations) alternating Mamba-3 (d_state 64, 8 heads of 64,
# expand 2) and MLA (4 heads of 64, RoPE 32, kv rank 64), collapse; bf16 GEMM weights N(0, 0.02), fp32 state.
STACK = dict(windows=1024, seq=256, features=40, d_model=256, layers=4, n_streams=4, iters=20, d_state=64,
             mamba_headdim=64, expand=2, heads=4, head_dim=64, rope=32, kv_rank=64)


def _build_stack(cfg: dict, g):
    import torch

    from montlok.rdt.stack import HybridStackHIP

    torch.manual_seed(int(torch.randint(0, 2 ** 31 - 1, (1,), generator=g)))
    stack = HybridStackHIP(cfg["features"], d_model=cfg["d_model"], n_layers=cfg["layers"],
                           n_streams=cfg["n_streams"], sinkhorn_iters=cfg["iters"], d_state=cfg["d_state"],
                           mamba_headdim=cfg["mamba_headdim"], expand=cfg["expand"], n_heads=cfg["heads"],
                           head_dim=cfg["head_dim"], rope_head_dim=cfg["rope"], kv_lora_rank=cfg["kv_rank"]).eval()
    with torch.no_grad():
        for w in stack.linear_weights():
            w.normal_(0.0, 0.02, generator=g)
        for hc in stack.hcs:  # data-dependent mixing: alphas 0.7, projections N(0, 1/d), mixing logits N(0, 1)
            for a in (hc.pre_alpha, hc.post_alpha, hc.res_alpha):
                a.fill_(0.7)
            for w in (hc.pre_proj.weight, hc.post_proj.weight, hc.res_proj.weight):
                w.normal_(0.0, cfg["d_model"] ** -0.5, generator=g)
            hc.res_bias.normal_(generator=g)
    return stack


def cpu_baseline_stack(cfg: dict, stack, feats_cpu, budget_s: float = 12.0, windows: int = 2) -> dict:
    """Reference CPU kernels (mHC, norms, Mamba-3 mixer, RoPE) with torch CPU GEMMs and SDPA, on `windows` of
    the windows; the same chain as the GPU stack."""
    import torch
    import torch.nn.functional as F

    from montlok.rdt.mla import rope_tables
    from oracle import Oracle, Reference, reference_available

    lib = Reference() if reference_available() else Oracle()
    kind = "reference" if isinstance(lib, Reference) else "port"
    x = feats_cpu[:windows].contiguous()
    B, L, _ = x.shape
    f32 = lambda t: t.detach().float().cpu()  # noqa: E731
    hcs = [dict(nw=f32(h.dyn_norm.weight).numpy(), eps=h.dyn_norm.eps, w64=h._projection_block().cpu().numpy(),
                pb=f32(h.pre_bias).numpy(), qb=f32(h.post_bias).numpy(), rb=f32(h.res_bias).numpy(),
                al=(h.pre_alpha.item(), h.post_alpha.item(), h.res_alpha.item()), iters=h.sinkhorn_iters)
           for h in stack.hcs]
    norms = [f32(nm.weight).numpy() for nm in stack.norms]
    mix = []
    for i, m in enumerate(stack.mixers):
        mix.append({k: f32(v) for k, v in m.state_dict().items()})
    fw, fb = f32(stack.feature_proj.weight), f32(stack.feature_proj.bias)
    mla = stack.mixers[1]
    cos, sin = (t.numpy() for t in rope_tables(L, mla.rope_dim, mla.rope.theta))
    m0 = stack.mixers[0]

    def mamba(p, a):
        proj = F.linear(torch.from_numpy(a), p["in_proj.weight"]).numpy()
        y = lib.mamba3_siso_forward(proj, m0.d_state, m0.num_bc_heads, m0.nheads, m0.headdim, m0.num_rope_angles,
                                    p["B_bias"].numpy(), p["C_bias"].numpy(), p["B_norm.weight"].numpy(),
                                    p["C_norm.weight"].numpy(), 1e-5, 1e-5, p["dt_bias"].numpy(), p["D"].numpy(),
                                    m0.A_floor)
        return F.linear(torch.from_numpy(y), p["out_proj.weight"]).numpy()

    def attn(p, a):
        H, hd, nope, kvr, d = mla.n_heads, mla.head_dim, mla.nope_dim, mla.kv_lora_rank, mla.d_model
        xa = torch.from_numpy(a)
        projected = F.linear(xa, torch.cat([p["q_proj.weight"], p["kv_down.weight"], p["k_rope_proj.weight"]]))
        q = projected[..., :d].reshape(B, L, H, hd).numpy()
        kvn = lib.layer_norm(projected[..., d:d + kvr].contiguous().numpy(), p["kv_norm.weight"].numpy(),
                             p["kv_norm.bias"].numpy(), 1e-5)
        kv = F.linear(torch.from_numpy(kvn), p["kv_up.weight"]).reshape(B, L, H, nope + hd)
        q, k = lib.mla_rope(q, kv.numpy(), projected[..., d + kvr:].contiguous().numpy(), cos, sin, nope)
        o = F.scaled_dot_product_attention(torch.from_numpy(q).transpose(1, 2), torch.from_numpy(k).transpose(1, 2),
                                           kv[..., nope:].transpose(1, 2), is_causal=True, scale=mla.scale)
        return F.linear(o.transpose(1, 2).reshape(B, L, d), p["o_proj.weight"]).numpy()

    def prep(i, streams, n_streams):
        h = hcs[i]
        return lib.mhc_prepare(streams, h["nw"], h["eps"], h["w64"], h["pb"], h["qb"], h["rb"], *h["al"], h["iters"],
                               n_streams, norms[i], 1e-5)

    def step():
        hb = F.linear(x, fw, fb).numpy()
        agg, pre, post, res = prep(0, hb, stack.n_streams)
        out = mamba(mix[0], agg)
        streams = hb
        for i in range(1, len(hcs)):
            if kind == "reference":
                h = hcs[i]
                streams, agg, pre, post, res = lib.mhc_combine_prepare(streams, res, post, out, h["nw"], h["eps"],
                                                                       h["w64"], h["pb"], h["qb"], h["rb"], *h["al"],
                                                                       h["iters"], norms[i], 1e-5)
            else:
                streams = lib.mhc_combine(streams, res, post, out)
                agg, pre, post, res = prep(i, streams, 0)
            out = mamba(mix[i], agg) if i % 2 == 0 else attn(mix[i], agg)
        return lib.mhc_combine(streams, res, post, out, collapse=True, materialize=False)

    def make_step(threads):
        if kind == "reference":
            lib.set_threads(threads)
        return step

    return _cpu_legs(make_step, windows, "windows/s", kind,
                     f"steps over {windows} of the {cfg['windows']} windows (the rate scales per window); mHC, norms, "
                     f"Mamba-3 mixer and RoPE in the {'reference ' + lib.variant if kind == 'reference' else 'oracle'} "
                     f"build, GEMMs and SDPA in torch CPU (fp32, bf16 weights upcast)", budget_s)


def bench_stack(steps: int, warmup: int, cpu: bool) -> dict:
    import torch

    from montlok import _C

    cfg = STACK
    B, L, d, n = cfg["windows"], cfg["seq"], cfg["d_model"], cfg["n_streams"]
    T = B * L
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(0)
    feats_cpu = torch.randn(B, L, cfg["features"], generator=g).clamp_(-8.0, 8.0)
    feats = feats_cpu.to(dev)
    stack_cpu = _build_stack(cfg, g)
    stack = copy.deepcopy(stack_cpu).to(dev)
    for w in stack.linear_weights():
        w.data = w.data.bfloat16()
    result = {}

    def step():
        result["out"] = stack(feats)

    with torch.no_grad():
        step()
        torch.cuda.synchronize()
        eager = result["out"].clone()
        assert torch.isfinite(eager).all().item()
        t = _gpu_steps([step], steps, warmup)
        assert torch.equal(result["out"], eager), "graph replay differs from the eager step"
        steps, ms = t["steps"], t["ms_per_step"]

        # Per-operator launches on the tensors of one eager pass.
        c = _C
        hc0, hc1, m0, m1 = stack.hcs[0], stack.hcs[1], stack.mixers[0], stack.mixers[1]
        h = c.linear(feats, stack.feature_proj.weight, stack.feature_proj.bias)
        _, prep0 = hc0._prepare(h, allow_broadcast=True, output_norm=stack.norms[0])
        agg = prep0[0]
        out0 = m0(agg)
        streams1, prep1 = hc0._combine_prepare(h, prep0, out0, hc1, output_norm=stack.norms[1])
        out1 = m1(prep1[0])
        proj = c.linear(agg, m0.in_proj.weight)
        y = m0.forward_projected(proj)
        W, di = m0.in_proj.weight.shape[0], m0.d_inner
        f, h2 = 4, 2
        ops = {
            "feature_proj": dict(fn=lambda: c.linear(feats, stack.feature_proj.weight, stack.feature_proj.bias),
                                 bytes=T * (cfg["features"] + d) * f, flops=2 * T * cfg["features"] * d),
            "mhc_prepare_broadcast": dict(fn=lambda: hc0._prepare(h, allow_broadcast=True, output_norm=stack.norms[0]),
                                          bytes=T * (2 * d + 2 * n + n * n) * f),
            "mhc_combine_prepare": dict(fn=lambda: hc1._combine_prepare(streams1, prep1, out1, stack.hcs[2],
                                                                        output_norm=stack.norms[2]),
                                        # reads: old streams, res, post, the layer output; writes: the new
                                        # streams (never read back) and the next agg, pre, post, res
                                        bytes=T * (n * d + n * n + n + d) * f + T * n * d * f +
                                        T * (d + 2 * n + n * n) * f),
            "mhc_combine_collapse": dict(fn=lambda: hc1._combine_collapse(streams1, prep1, out1),
                                         bytes=T * (n * d + n * n + n + 2 * d) * f),
            "mamba_in_proj": dict(fn=lambda: c.linear(agg, m0.in_proj.weight), bytes=T * (d + W) * f + W * d * h2,
                                  flops=2 * T * d * W, precision="bf16"),
            "mamba3_siso_forward": dict(fn=lambda: m0.forward_projected(proj), bytes=T * (W + di) * f,
                                        flops=7 * T * m0.nheads * m0.d_state * m0.headdim, precision="f32"),
            "mamba_out_proj": dict(fn=lambda: c.linear(y, m0.out_proj.weight), bytes=T * (di + d) * f + d * di * h2,
                                   flops=2 * T * di * d, precision="bf16"),
            "mla_forward": dict(fn=lambda: m1(prep1[0]), bytes=2 * T * d * f,
                                flops=2 * T * d * (d + m1.kv_lora_rank + m1.rope_dim) +
                                2 * T * m1.kv_lora_rank * m1.n_heads * (m1.nope_dim + m1.head_dim) +
                                4 * B * m1.n_heads * (L * (L + 1) // 2) * m1.head_dim + 2 * T * d * d,
                                precision="bf16"),
        }
        # Eight launches per graph: with two, each replay's start-up cost (about 0.2 ms at these sizes)
        # lands on the per-launch time (combine + prepare: 673 against 562 us).
        table = _kernel_table(ops, _op_times(ops, 4, reps=8), "bf16")
    dom = max(table, key=lambda k: table[k]["launch_ms"])
    flops = sum(ops[k]["flops"] for k in ("feature_proj",)) + 2 * (ops["mamba_in_proj"]["flops"] +
                                                                   ops["mamba3_siso_forward"]["flops"] +
                                                                   ops["mamba_out_proj"]["flops"]) + \
        2 * ops["mla_forward"]["flops"]
    line = _base_line(B / (ms * 1e-3), "windows/s", steps, warmup, ms,
                      "bf16 weights and contraction operands, fp32 accumulate and state",
                      "synthetic (seeded N(0,1) features clipped to [-8,8], N(0,0.02) bf16 weights)",
                      {"workload": "rdt4quant_stack_4_layers", "windows": B, "seq_len": L, "features": cfg["features"],
                       "d_model": d, "layers": cfg["layers"], "n_streams": n, "sinkhorn_iters": cfg["iters"],
                       "mamba": f"d_state {cfg['d_state']}, {m0.nheads} heads of {cfg['mamba_headdim']}, "
                                f"{m0.num_rope_angles} rotary angles",
                       "mla": f"{cfg['heads']} heads of {cfg['head_dim']}, rope {cfg['rope']}, kv rank {cfg['kv_rank']}",
                       "step": "Linear(40->256), 4 x mHC[fn = mixer(RMSNorm(agg))] alternating Mamba-3 / MLA, collapse",
                       "launch": "the K steps in one HIP graph", "parallelism": "single GPU"})
    line["roofline"] = _roofline(dom, table[dom], ops[dom], "bf16", _traffic("hybrid_stack_b1024_l256_d256", dom))
    line["kernels"] = table
    line.update(_timing_fields(t))
    line["step_flops"] = flops
    line["step_achieved_TFs"] = flops / (ms * 1e-3) / 1e12
    line["tokens_per_s"] = T / (ms * 1e-3)
    if cpu:
        line["cpu_baseline"] = cpu_baseline_stack(cfg, stack_cpu, feats_cpu)
        line["cpu_baseline"]["gpu_over_cpu"] = line["value"] / line["cpu_baseline"]["value"]
    return line


# ------------------------------------------------------------ norms

# The reference's row-wise norm operators alone (RMSNorm, residual add + RMSNorm, LayerNorm) at the
# stack's activation size, 262144 tokens x d_model 256: plain HBM-bound kernels, measured so that their
# fraction of HBM bandwidth is on record beside the fused ones.
NORMS = dict(rows=262144, dim=256)


def cpu_baseline_norms(cfg: dict, budget_s: float = 12.0, rows: int = 65536) -> dict:
    """The reference's own norm kernels (oracle/_ref) on a quarter of the rows (the oracle port where that
    library is absent): its five 64 MB operands and results exceed the host's last-level cache, as the
    workload's exceed the GPU's, where a 16384-row slice would time the CPU from cache."""
    import numpy as np

    from oracle import Oracle, Reference, reference_available

    rng = np.random.default_rng(0)
    d = cfg["dim"]
    x = rng.standard_normal((rows, d)).astype(np.float32)
    r = rng.standard_normal((rows, d)).astype(np.float32)
    w = (rng.random(d) + 0.5).astype(np.float32)
    b = rng.standard_normal(d).astype(np.float32)
    ref = reference_available()
    lib = Reference() if ref else Oracle()

    def make_step(threads):
        if ref:
            lib.set_threads(threads)

        def step():
            lib.rms_norm(x, w, 1e-5)
            lib.add_rms_norm(x, r, w, 1e-5)
            lib.layer_norm(x, w, b, 1e-5)
        return step

    return _cpu_legs(make_step, rows, "rows/s", "reference" if ref else "port",
                     f"rms_norm + add_rms_norm + layer_norm over {rows} of the {cfg['rows']} rows (x {cfg['dim']}) in the "
                     f"{'reference ' + lib.variant if ref else 'oracle'} build", budget_s)


def bench_norms(steps: int, warmup: int, cpu: bool) -> dict:
    import torch

    from montlok import _C

    cfg = NORMS
    R, d = cfg["rows"], cfg["dim"]
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(0)
    sets = 4  # 4 x 2 x 256 MiB of inputs > the 256 MB Infinity Cache
    xs = [torch.randn(R, d, generator=g).to(dev) for _ in range(sets)]
    rs = [torch.randn(R, d, generator=g).to(dev) for _ in range(sets)]
    w = (torch.rand(d, generator=g) + 0.5).to(dev)
    b = torch.randn(d, generator=g).to(dev)
    out = {}

    def rms(i):
        return lambda: out.__setitem__("rms", _C.rms_norm(xs[i], w, 1e-5, 1))

    def add(i):
        return lambda: out.__setitem__("add", _C.add_rms_norm(xs[i], rs[i], w, 1e-5, 1))

    def ln(i):
        return lambda: out.__setitem__("ln", _C.layer_norm(xs[i], w, b, 1e-5))

    def step(i):
        fns = (rms(i), add(i), ln(i))

        def run():
            for f in fns:
                f()
        return run

    def outputs():
        return {k: torch.cat([u.reshape(-1) for u in (v if isinstance(v, tuple) else (v,))]) for k, v in out.items()}

    eager = []
    for i in range(sets):
        step(i)()
        eager.append({k: v.clone() for k, v in outputs().items()})
    torch.cuda.synchronize()
    t = _gpu_steps([step(i) for i in range(sets)], steps, warmup)
    last = eager[(steps - 1) % sets]  # the timed graph's last step leaves its outputs in `out`
    for k, v in outputs().items():
        assert torch.equal(v, last[k]), f"graph replay of {k} differs from the eager step"
    ms = t["ms_per_step"]
    replays = max(4, steps // sets)
    f = 4
    kernels = {}
    for name, mk, byts in (("rms_norm", rms, 2 * R * d * f), ("add_rms_norm", add, 4 * R * d * f),
                           ("layer_norm", ln, 2 * R * d * f)):
        k_ms = _time_graph(_graph([mk(i) for i in range(sets)]), replays) / sets
        kernels[name] = {"launch_ms": k_ms, "algorithmic_bytes": byts, "achieved_GBs": byts / (k_ms * 1e-3) / 1e9,
                         "hbm_frac": byts / (k_ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
    dom = max(kernels, key=lambda k: kernels[k]["launch_ms"])
    line = _base_line(R / (ms * 1e-3), "rows/s", t["steps"], warmup, ms, "f32 (f64 accumulate)",
                      "synthetic (seeded N(0,1) rows)",
                      {"workload": "norms_262144x256", "rows": R, "dim": d,
                       "step": "rms_norm + add_rms_norm + layer_norm over the same rows",
                       "launch": "the K steps in one HIP graph, rotating over 4 independent input sets (cold HBM)",
                       "parallelism": "single GPU"})
    k = kernels[dom]
    line["roofline"] = {"bound": "hbm", "kernel": dom, "achieved": k["achieved_GBs"], "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": k["hbm_frac"], "traffic": _traffic("norms_r262144_d256", dom),
                        "algorithmic_bytes": k["algorithmic_bytes"], "launch_ms": k["launch_ms"]}
    line["kernels"] = kernels
    line.update(_timing_fields(t))
    line["step_roofline_frac"] = (8 * R * d * f) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS
    if cpu:
        line["cpu_baseline"] = cpu_baseline_norms(cfg)
        line["cpu_baseline"]["gpu_over_cpu"] = line["value"] / line["cpu_baseline"]["value"]
    return line


WORKLOADS = {"mhc": bench_mhc, "block": bench_block, "mla": bench_mla, "decode": bench_decode, "stack": bench_stack,
             "norms": bench_norms}


def copy_bandwidth(mib: int = 1024, reps: int = 10) -> float:
    """GB/s (bytes read + written) of a plain device-to-device copy of `mib` MiB: the HBM rate a kernel that
    streams its bytes once can reach on this device, beside the 8 TB/s peak the roofline quotes."""
    import torch

    x = torch.empty(mib << 18, device="cuda:0")
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        y.copy_(x)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del x, y
    return 2 * (mib << 20) / (ms * 1e-3) / 1e9


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--workload", default="block", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--configs", choices=("all", "none"), default="all",
                    help="also measure the other workloads, each summarised under \"configs\" (default: all)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}). The workloads "
              f"shard by independent windows, tokens and streams, one share per GPU, with no exchange between "
              f"GPUs inside a step.", file=sys.stderr)
        return 2
    import torch

    t0 = time.perf_counter()
    line = WORKLOADS[args.workload](args.steps, args.warmup, cpu=not args.no_cpu)
    print(f"bench: {args.workload} done in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    copy = copy_bandwidth()
    if line["roofline"]["bound"] == "hbm":
        line["roofline"]["copy_GBs"] = copy
        line["roofline"]["frac_of_copy"] = line["roofline"]["achieved"] / copy
    if args.configs == "all":
        line["configs"] = {args.workload: "this line"}
        for name, fn in WORKLOADS.items():
            if name == args.workload:
                continue
            t1 = time.perf_counter()
            sub = fn(args.steps, args.warmup, cpu=not args.no_cpu)
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
            line["configs"][name] = _config_summary(sub, copy)
            print(f"bench: {name} done in {time.perf_counter() - t1:.1f} s", file=sys.stderr, flush=True)
    print(json.dumps(line))
    return 0


def _config_summary(sub: dict, copy_gbs: float) -> dict:
    """The fields of another workload's line that the default line carries for it."""
    roof = {k: sub["roofline"][k] for k in ("kernel", "bound", "achieved", "peak", "unit", "frac", "traffic",
                                            "launch_ms")}
    if roof["bound"] == "hbm":
        roof["copy_GBs"] = copy_gbs
        roof["frac_of_copy"] = roof["achieved"] / copy_gbs
    out = {"value": sub["value"], "unit": sub["unit"], "steps": sub["steps"],
           "warmup": sub["warmup"], "ms_per_step": sub["ms_per_step"],
           "median_ms_per_step": sub["median_ms_per_step"], "dtype": sub["dtype"], "config": sub["config"],
           "roofline": roof, "kernels": sub.get("kernels")}
    for k in ("step_hbm_frac", "step_roofline_frac", "step_mfma_frac", "step_fp32_frac"):
        if k in sub:
            out[k] = sub[k]
    if "cpu_baseline" in sub:
        cb = sub["cpu_baseline"]
        out["cpu_baseline"] = {k: cb[k] for k in ("value", "unit", "cores", "kind", "sample", "one_thread_value",
                                                 "gpu_over_cpu") if k in cb}
    return out


if __name__ == "__main__":
    sys.exit(main())
