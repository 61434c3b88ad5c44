#!/usr/bin/env python3
"""Benchmark of the weight-only quantized Linear hot path on one MI355X.

Default (the driver's line): BASELINE config C2 -- the Llama-3-8B-shaped int4 g128 decode
layer stack, 32 layers x {qkv 4096->6144, o 4096->4096, gate_up 4096->28672, down
14336->4096}, M=1, 32 distinct weight sets (3.7 GB, far past the 256 MB MALL). One "step" is
one pass over the 128 linears, launched back to back on one stream and captured in a HIP graph.

value   = whole-pass algorithmic bytes (int4 codes + bf16 scale/zero + x + y) / step time (GB/s)
roofline= the dominant kernel (the w4 skinny GEMV: all 128 launches) -- algorithmic bytes per
          launch / average launch duration from HIP events bracketing each launch on torch's
          stream, vs the 8 TB/s HBM peak
cpu_baseline = the reference's CPU int4 path (torch tinygemm, oracle/cpu_path.py) on a bounded
          sample (C2 layer 0..L-1 at M=1) on this host's cores

Other configs (--config c1|c3|c4|c5, --m) print lines of the same shape for measurement work.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

HBM_PEAK = 8.0e12       # B/s, MI355X HBM3E
BF16_PEAK = 2.5e15      # dense bf16 MFMA FLOP/s


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5"])
    ap.add_argument("--m", type=int, default=None, help="rows (C2 M / C4 M / C5 T)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-graph", action="store_true", help="eager launches instead of a HIP graph")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    return ap.parse_args()


def _graph_or_eager(fn, use_graph: bool):
    import torch
    fn()
    torch.cuda.synchronize()
    if not use_graph:
        return fn
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g.replay


def _time_steps(step, steps: int, warmup: int):
    import torch
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        step()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps


def _per_launch_ms(launches, reps: int = 3):
    """Average device duration of each launch, from events recorded on torch's current stream
    immediately before and after it (eager, the same kernels as the timed region)."""
    import torch
    evs = []
    for _ in range(reps):
        for fn in launches:
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            evs.append((a, b))
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in evs]


# ---------------------------------------------------------------------------------------------
def bench_c2(args, dev, M: int):
    import torch
    from infinitemodel_amd import ops, workloads as wl
    lins = wl.llama8b_stack(dev)
    x_in = wl.activations(M, 4096, 1, dev)
    x_dn = wl.activations(M, 14336, 2, dev)
    ys = {n: torch.empty((M, N), dtype=torch.bfloat16, device=dev) for n, _, N in wl.LLAMA8B_PROJ}
    launches = []
    for L in lins:
        kind = L.name.split(".")[1]
        x = x_dn if kind == "down" else x_in
        launches.append(lambda L=L, x=x, y=ys[kind]: ops.linear_w4(x, L.q, L.G, (L.s, L.z), out=y))

    def step():
        for fn in launches:
            fn()

    run = _graph_or_eager(step, not args.no_graph)
    ms = _time_steps(run, args.steps, args.warmup)
    total_bytes = sum(L.algorithmic_bytes(M) for L in lins)
    per = _per_launch_ms(launches)
    avg_ms = sum(per) / len(per)
    avg_bytes = total_bytes / len(lins)
    ach = avg_bytes / (avg_ms * 1e-3)
    line = {
        "metric": "w4a16 decode GEMV GB/s & % HBM peak at 8B shapes; prefill TFLOP/s % MFMA",
        "value": round(total_bytes / (ms * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int4-w/bf16-a (fp32 acc)",
        "data": "synthetic (random N(0,0.02) weights RTN-packed int4 g128; x ~ N(0,1))",
        "config": {"workload": f"C2 llama-3-8b int4 g128 decode stack, 32 layers x 4 linears, M={M}",
                   "layers": 32, "M": M, "graph": not args.no_graph,
                   "bytes_per_step": total_bytes, "hbm_frac_whole_step": round(total_bytes / (ms * 1e-3) / HBM_PEAK, 4)},
        "roofline": {"bound": "hbm", "achieved": round(ach / 1e9, 2), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK, 4), "traffic": None,
                     "kernel": "imq w4_skinny_kernel", "avg_launch_us": round(avg_ms * 1e3, 3),
                     "avg_algorithmic_bytes_per_launch": int(avg_bytes)},
    }
    cpu = None
    if not args.no_cpu:
        cpu = cpu_c2(args, M)
    line["cpu_baseline"] = cpu
    return line


def cpu_c2(args, M: int):
    """Reference CPU int4 path (tinygemm) on C2 layers 0..L-1 at the same M, bounded by time."""
    import torch
    from oracle import cpu_path
    from infinitemodel_amd import workloads as wl
    n = cpu_path.tune_cpu_threads()
    cpu = torch.device("cpu")
    layers = []
    nbytes = 0
    for p, (name, K, N) in enumerate(wl.LLAMA8B_PROJ):
        L = wl.rtn_int4_linear(N, K, 1000 + p, cpu, name=name)
        mat2, sz = cpu_path.tinygemm_prepare(L.q, L.s, L.z, 128)
        layers.append((name, K, mat2, sz))
        nbytes += L.algorithmic_bytes(M)
    x_in = torch.randn(M, 4096).to(torch.bfloat16)
    x_dn = torch.randn(M, 14336).to(torch.bfloat16)

    def one_layer():
        for name, K, mat2, sz in layers:
            cpu_path.tinygemm_linear(x_dn if name == "down" else x_in, mat2, 128, sz)

    one_layer()
    times = []
    t_end = time.perf_counter() + args.cpu_seconds
    while time.perf_counter() < t_end or len(times) < 5:
        t0 = time.perf_counter()
        one_layer()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": n, "kind": "port",
            "sample": f"C2 layer 0 (qkv, o, gate_up, down) int4 g128, M={M}, torch tinygemm "
                      f"_weight_int4pack_mm_for_cpu, median of {len(times)} passes over {args.cpu_seconds:.0f}s",
            "ms_per_layer": round(med * 1e3, 3), "cpu": _cpu_model()}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return "unknown"


def main():
    args = _parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures one GPU only: the quantized-linear hot path runs "
                                   "per GPU and the GPU boxes here have one GPU; run with --gpus 1"}))
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no ROCm GPU visible"}))
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.config == "c2":
        line = bench_c2(args, dev, args.m or 1)
    else:
        from infinitemodel_amd import bench_configs
        line = bench_configs.run(args, dev)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
