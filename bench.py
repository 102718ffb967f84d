#!/usr/bin/env python3
"""Throughput of the RDT4quant fused forward on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload mhc]

Default workload: the mHC residual mix alone, fp32, n = 4 streams, d = 128,
8192 tokens (64 windows of 128 tokens), 20 Sinkhorn iterations. One step is
one hyper-connection over one batch: mhc_prepare (coefficients + aggregate),
the wrapped layer as the identity (out = agg), mhc_combine (new streams).
Inputs are resident in HBM before timing; the step rotates over enough
independent input/output sets (more than the 256 MB Infinity Cache) that each
step reads cold data.

Prints one JSON line: whole-job throughput (windows/s), the roofline of the
dominant kernel (per-launch average from HIP events recorded on the kernels'
stream inside the timed region) and the CPU baseline (the reference's CPU
kernels compiled from its sources into oracle/_ref, timed on this host on a
bounded sample, or the oracle port when that library is absent).
"""

from __future__ import annotations

import argparse
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

# mHC residual mix, n = 4, d = 128, 8192 tokens (64 windows x 128 tokens).
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
    """The reference's own CPU kernels (oracle/_ref) on the same workload."""
    import numpy as np

    from oracle import Oracle, Reference, host_isa, reference_available

    n, d, T = cfg["n"], cfg["d"], cfg["windows"] * cfg["seq"]
    rng = np.random.default_rng(0)
    s = rng.standard_normal((cfg["windows"], cfg["seq"], n, d)).astype(np.float32)
    nw = (rng.random(d) + 0.5).astype(np.float32)
    pw = (rng.standard_normal((2 * n + n * n, d)) / np.sqrt(d)).astype(np.float64)
    pb, qb = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    rb = rng.standard_normal((n, n)).astype(np.float32)
    cores = len(os.sched_getaffinity(0))
    if reference_available():
        lib, kind = Reference(), "reference"
        lib.set_threads(cores)
        threads = cores
        variant = lib.variant
    else:
        lib, kind = Oracle(), "port"
        threads = 1
        variant = "oracle"

    def step():
        agg, pre, post, res = lib.mhc_prepare(s, nw, 1e-5, pw, pb, qb, rb, 0.7, 0.7, 0.7, cfg["iters"])
        lib.mhc_combine(s, res, post, agg)

    step()
    reps, t0 = 0, time.perf_counter()
    while True:
        step()
        reps += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= budget_s or reps >= 100000:
            break
    windows_per_s = reps * cfg["windows"] / elapsed
    return {"value": windows_per_s, "unit": "windows/s", "cores": threads, "kind": kind,
            "sample": f"{reps} full steps (prepare + combine, {T} tokens each) in {elapsed:.1f} s, "
                      f"{variant} build, {threads} OpenMP threads of {cores} host cores"}


def _graph(fn_list):
    """Capture the given launch closures, in order, into one HIP graph."""
    import torch

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

    # Correctness guard on the timed configuration before timing: eager run,
    # then the captured graph, bit-identical.
    prepare(0)()
    combine(0)()
    torch.cuda.synchronize()
    eager = outs[0].clone()
    assert torch.isfinite(eager).all().item()
    step_graph = _graph([f for i in range(sets) for f in (prepare(i), combine(i))])
    prep_graph = _graph([prepare(i) for i in range(sets)])
    comb_graph = _graph([combine(i) for i in range(sets)])
    step_graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(outs[0], eager), "graph replay differs from the eager step"

    replays = max(1, steps // sets)
    steps = replays * sets
    for _ in range(max(1, warmup // sets)):
        step_graph.replay()
    # Timed region: `steps` steps (graph replays of 16 steps each) between two
    # synchronisations.
    ms_per_step = _time_graph(step_graph, replays) / sets
    prep_ms = _time_graph(prep_graph, replays) / sets
    comb_ms = _time_graph(comb_graph, replays) / sets
    # Warm-cache rate: one input set over and over (Infinity-Cache resident).
    warm_graph = _graph([f for _ in range(sets) for f in (prepare(0), combine(0))])
    warm_ms = _time_graph(warm_graph, replays) / sets

    prep_bytes, comb_bytes = mhc_bytes(n, d, T)
    windows_per_s = W / (ms_per_step * 1e-3)
    kernels = {"mhc_prepare": (prep_ms, prep_bytes), "mhc_combine": (comb_ms, comb_bytes)}
    dom = max(kernels, key=lambda k: kernels[k][0])
    dom_ms, dom_bytes = kernels[dom]
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
    traffic = None
    tfile = ROOT / "profiles" / "mhc_n4_d128_t8192_traffic.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get(dom)
    line = {
        "metric": METRIC,
        "value": windows_per_s,
        "unit": "windows/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (f64 accumulate)",
        "data": "synthetic (seeded N(0,1) streams, random-init mHC weights)",
        "config": {"workload": "mhc_residual_mix", "n_streams": n, "d_model": d, "tokens": T, "windows": W,
                   "seq_len": L, "sinkhorn_iters": iters, "step": "mhc_prepare + identity fn + mhc_combine",
                   "launch": "HIP graph of 16 steps over 16 independent input sets, replayed",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic, "algorithmic_bytes": dom_bytes,
                     "launch_ms": dom_ms},
        "kernels": {k: {"launch_ms": v[0], "algorithmic_bytes": v[1],
                        "achieved_GBs": v[1] / (v[0] * 1e-3) / 1e9} for k, v in kernels.items()},
        "step_roofline_frac": (prep_bytes + comb_bytes) / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "tokens_per_s": T / (ms_per_step * 1e-3),
        "stream_steps_per_s": n * T / (ms_per_step * 1e-3),
        "warm_cache_windows_per_s": W / (warm_ms * 1e-3),
    }
    if cpu:
        line["cpu_baseline"] = cpu_baseline_mhc(cfg)
        line["cpu_baseline"]["gpu_over_cpu"] = windows_per_s / line["cpu_baseline"]["value"]
    return line


WORKLOADS = {"mhc": bench_mhc}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="mhc", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only: every GPU box of this build has one GPU (asked for --gpus "
              f"{args.gpus}, WORLD_SIZE={world}). The workloads shard by independent windows/tokens/streams; "
              f"see DESIGN.md for how the path would shard.", file=sys.stderr)
        return 2
    line = WORKLOADS[args.workload](args.steps, args.warmup, cpu=not args.no_cpu)
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
