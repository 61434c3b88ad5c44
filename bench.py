#!/usr/bin/env python3
"""Benchmark of the weight-only quantized Linear hot path on one MI355X.

Default line (the driver's): BASELINE config C2 -- the Llama-3-8B-shaped int4 g128 decode layer
stack, 32 layers x {qkv 4096->6144, o 4096->4096, gate_up 4096->28672, down 14336->4096}, M=1,
32 distinct weight sets (3.7 GB, far past the 256 MB MALL). One step is one pass over the 128
linears, launched back to back on one stream and replayed as a HIP graph.

  value        whole-pass algorithmic bytes (int4 codes + bf16 scale/zero + x + y) / step time
  roofline     the dominant (here: only) kernel, imq's w4 line kernel (the M=1 decode GEMV):
               algorithmic bytes per launch / average launch duration, both over the timed
               region (HIP events on the stream the graph replays on); ``traffic`` = HBM bytes
               per launch (every kernel of one linear or MoE layer) from the committed
               rocprofv3 FETCH_SIZE / WRITE_SIZE summary, scaled by a copy-kernel calibration
               (profiles/traffic.json), null when no summary matches the workload
  cpu_baseline the reference's CPU int4 path (torch tinygemm, as worker_quant.py:732-759 binds
               it) on a bounded sample: 8 layers of the same shapes (0.93 GB, beyond host cache),
               median pass time on this host's cores
  also         measured after the C2 line in the same run (--no-also skips them): C4 prefill's
               fused step, int4 and int8 at M = 2048 and 512, TFLOP/s (the naive, bf16-GEMM and
               CPU legs are --config c4's)

Other configs print lines of the same shape: --config c1 (single 1x4096->4096 linear), c3 (int2
g64 70B shapes), c4 (prefill, --quant int4|int8, --m 512|2048), c5 (OLMoE fused MoE, --m = T),
gptoss (gpt-oss-20b fused experts, --m = T), head (int8 lm_head decode at the Qwen2.5-7B head,
152064 x 3584, --m rows, two distinct copies) and the hardware ceilings of libimq's probes:
``ceiling`` (the C2 weights read by the read-only stream probe, one launch per linear and one
persistent launch, beside the decode kernels), ``stream`` (4 GiB read-only and 1 GiB copies),
``launch`` (a chain of empty kernels), ``mfma`` (the bf16 MFMA issue peak) and ``copy`` (torch's
device copy, which calibrates the PMC byte counters).

Profiles of a line: ``rocprofv3 --kernel-trace --output-format csv -d DIR -o NAME -- python bench.py
...`` records every dispatch; ``python bench.py --trace-summary DIR/NAME_kernel_trace.csv --steps K``
summarizes the timed steps -- the dispatches between the two marker kernels (one empty workgroup,
outside the timing events) that bracket them -- per kernel and per launch position, with the
kernel time per step to set beside the line's ms_per_step (profile the default line with
--no-also, or pick its region with --region 0).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK = 8.0e12       # B/s, MI355X HBM3E
BF16_PEAK = 2.5e15      # dense bf16 MFMA FLOP/s
METRIC = "w4a16 decode GEMV GB/s & % HBM peak at 8B shapes; prefill TFLOP/s % MFMA"


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5", "gptoss", "head", "copy", "ceiling", "stream",
                                                    "launch", "mfma"])
    ap.add_argument("--m", type=int, default=None, help="rows: C2/C3/C4 M, C5 tokens T")
    ap.add_argument("--quant", default="int4", choices=["int4", "int8"], help="C4 weight format")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-graph", action="store_true", help="eager launches instead of a HIP graph")
    ap.add_argument("--no-also", action="store_true",
                    help="default run: skip the C4 prefill lines measured after the C2 line")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--trace-summary", default=None, metavar="CSV",
                    help="summarize the timed steps of a rocprofv3 kernel-trace CSV of a bench run (no GPU)")
    ap.add_argument("--region", type=int, default=-1, help="which timed region of the traced run (-1: the last)")
    ap.add_argument("--period", type=int, default=None, help="launches per step, for per-position means")
    return ap.parse_args()


# ---------------------------------------------------------------------------------------------
# timing helpers
# ---------------------------------------------------------------------------------------------
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


MARK_KERNEL = "probe_empty_kernel"


def _mark():
    """One empty one-workgroup kernel (imq_probe_empty) on the current stream: it delimits the
    timed steps in a rocprofv3 kernel trace (outside the timing events)."""
    import torch
    from infinitemodel_amd import _lib
    _lib.call("imq_probe_empty", 1, torch.cuda.current_stream().cuda_stream)


def _packed_module_layout(qs, bits: int, N_of, G: int):
    """The packed layout the drop-in module binds for these weights (QuantLinear4 / QuantLinear2 on
    ROCm: line-tiled where the shape fits it, worker_quant._bind_group_rocm): the weights to pass
    (row-layout arrays replaced by their tiled copies, so the footprint is unchanged), the op that
    reads them and the layout's name."""
    from infinitemodel_amd import ops
    from infinitemodel_amd import worker_quant as wq
    fits = all(wq._LINE_TILED and G == (128 if bits == 4 else 64) and N_of(i) % 16 == 0 and q.shape[1] % 128 == 0
               and q.is_contiguous() for i, q in enumerate(qs))
    row_op = ops.linear_w4 if bits == 4 else ops.linear_w2
    if not fits:
        return list(qs), row_op, "row"
    return [ops.line_tile(q) for q in qs], (ops.linear_w4_tiled if bits == 4 else ops.linear_w2_tiled), "line-tiled"


def _w8_module_layout(pairs):
    """The int8 weights as the drop-in QuantLinear binds them: each (q, scale) goes through the
    module's own binding (worker_quant._w8_binding, then the line-tiled layout when its op serves
    every M). Returns the (q, scale) pairs to pass, the op that reads them and the layout's name."""
    from infinitemodel_amd import ops
    from infinitemodel_amd import worker_quant as wq
    out, tiled = [], []
    for q, s in pairs:
        mod = wq._quant_linear_cls()(q, s, None)
        mod.prepare_fused()
        tiled.append(bool(getattr(mod, "_line_tiled", False)))
        out.append((mod.qweight, s))
        del mod
    if all(tiled):
        return out, ops.linear_w8_tiled, "line-tiled"
    return [(ops.line_untile(q) if t else q, s) for (q, s), t in zip(out, tiled)], ops.linear_w8, "row"


def _w4_module_layout(lins):
    """_packed_module_layout over int4 Linear4 records, in place."""
    qs, op, layout = _packed_module_layout([L.q for L in lins], 4, lambda i: lins[i].N, lins[0].G if lins else 128)
    for L, q in zip(lins, qs):
        L.q = q
    return op, layout


def _time_steps(step, steps: int, warmup: int) -> float:
    """ms per step: warmup, then EXACTLY ``steps`` steps bracketed by a device synchronize and
    HIP events on the current stream (the stream the graph replays on). A marker kernel is
    launched just before the first event and just after the second, so a kernel trace of the run
    shows exactly which dispatches the line's time covers (``--trace-summary``)."""
    import torch
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    _mark()
    t0.record()
    for _ in range(steps):
        step()
    t1.record()
    _mark()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps


def _cpu_time(fn, seconds: float, min_runs: int = 3) -> tuple:
    fn()
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < min_runs:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def _cpu_model() -> str:
    """Host CPU model, sockets and physical cores (from /proc/cpuinfo)."""
    model, sockets, cores = "unknown", set(), set()
    try:
        with open("/proc/cpuinfo") as f:
            phys = None
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name":
                    model = v
                elif k == "physical id":
                    phys = v
                    sockets.add(v)
                elif k == "core id":
                    cores.add((phys, v))
    except Exception:
        pass
    return f"{model}, {max(1, len(sockets))} socket(s), {len(cores) or '?'} physical cores"


def _traffic(key: str):
    """HBM bytes per launch (one linear or one MoE layer, every hot-path kernel of it) for workload
    ``key`` from the committed PMC summary (FETCH_SIZE x 2 + WRITE_SIZE, copy-calibrated), or None."""
    path = os.path.join(HERE, "profiles", "traffic.json")
    try:
        with open(path) as f:
            d = json.load(f)
        v = d.get(key)
        return None if v is None else float(v["bytes_per_launch"])
    except Exception:
        return None


def _line(value, unit, ms, args, config, roofline, cpu, hib=True, dtype="bf16",
          data="synthetic: random weights of the named shapes, RTN-packed; x ~ N(0,1) bf16"):
    return {"metric": METRIC, "value": value, "unit": unit, "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": hib,
            "scaling": "weak", "vs_baseline": None, "dtype": dtype, "data": data, "config": config,
            "roofline": roofline, "cpu_baseline": cpu}


def _hbm_roofline(kernel: str, bytes_per_launch: float, us_per_launch: float, traffic):
    ach = bytes_per_launch / (us_per_launch * 1e-6)
    return {"bound": "hbm", "achieved": round(ach / 1e9, 2), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
            "frac": round(ach / HBM_PEAK, 4), "traffic": traffic, "kernel": kernel,
            "avg_launch_us": round(us_per_launch, 3), "algorithmic_bytes_per_launch": int(bytes_per_launch)}


# ---------------------------------------------------------------------------------------------
# C2: Llama-3-8B int4 decode stack (the default line)
# ---------------------------------------------------------------------------------------------
def bench_c2(args, dev):
    import torch
    from infinitemodel_amd import ops, workloads as wl
    M = args.m or 1
    lins = wl.llama8b_stack(dev)
    op, layout = _w4_module_layout(lins)
    x_in = wl.activations(M, 4096, 1, dev)
    x_dn = wl.activations(M, 14336, 2, dev)
    ys = {n: torch.empty((M, N), dtype=torch.bfloat16, device=dev) for n, _, N in wl.LLAMA8B_PROJ}
    launches = []
    for L in lins:
        kind = L.name.split(".")[1]
        x = x_dn if kind == "down" else x_in
        launches.append(lambda L=L, x=x, y=ys[kind]: op(x, L.q, L.G, (L.s, L.z), out=y))

    def step():
        for fn in launches:
            fn()

    ms = _time_steps(_graph_or_eager(step, not args.no_graph), args.steps, args.warmup)
    total = sum(L.algorithmic_bytes(M) for L in lins)
    per_launch_us = ms * 1e3 / len(lins)
    roof = _hbm_roofline(_w4_decode_kernel(M, layout), total / len(lins), per_launch_us, _traffic(f"c2_m{M}"))
    cfg = {"workload": f"C2 llama-3-8b int4 g128 decode stack, 32 layers x (qkv, o, gate_up, down), M={M}",
           "layers": 32, "M": M, "launches_per_step": len(lins), "graph": not args.no_graph,
           "bytes_per_step": total, "distinct_bytes_per_step": total,
           "weights": "int4 g128 asymmetric, bf16 scale/zero", "packed_layout": layout}
    del lins
    torch.cuda.empty_cache()
    cpu = None if args.no_cpu else cpu_c2(args, M)
    return _line(round(total / (ms * 1e-3) / 1e9, 2), "GB/s", ms, args, cfg, roof, cpu)


def _w4_decode_kernel(M: int, layout: str = "row") -> str:
    """The kernels the int4 decode entry runs for M decode rows at the C1 / C2 shapes (gemv.hip)."""
    entry = "imq_linear_w4_tiled" if layout == "line-tiled" else "imq_linear_w4"
    if M <= 4:
        return f"w4_line_kernel ({entry}, M={M})"
    if layout == "line-tiled":
        return (f"w4_wsplit_kernel (gate_up) + w4_ksplit_kernel + splitk_rows_reduce_kernel (qkv, o, down) "
                f"({entry}, M={M})")
    return (f"w4_wsplit_kernel (qkv, o, gate_up) + w4_ksplit_kernel + splitk_rows_reduce_kernel (down) "
            f"({entry}, M={M})")


def _cpu_int4_random(N, K, seed, G=128):
    """CPU int4 linear with random codes and scale/zero (timing sample; values do not change the
    work of the tinygemm kernel)."""
    import torch
    g = torch.Generator().manual_seed(seed)
    ng = K // G
    q = torch.randint(0, 256, (N, K // 2), generator=g, dtype=torch.uint8)
    s = (torch.rand(N, ng, generator=g) * 0.01 + 0.001).to(torch.bfloat16)
    z = torch.randint(0, 16, (N, ng), generator=g).to(torch.bfloat16)
    return q, s, z


def cpu_c2(args, M: int, layers: int = 8):
    import torch
    from oracle import cpu_path
    from infinitemodel_amd import workloads as wl
    n = cpu_path.tune_cpu_threads()
    packs = []
    nbytes = 0
    for l in range(layers):
        for p, (name, K, N) in enumerate(wl.LLAMA8B_PROJ):
            q, s, z = _cpu_int4_random(N, K, 1000 + 4 * l + p)
            mat2, sz = cpu_path.tinygemm_prepare(q, s, z, 128)
            packs.append((name, mat2, sz))
            nbytes += N * K // 2 + N * (K // 128) * 4 + M * K * 2 + M * N * 2
            del q, s, z
    x_in = torch.randn(M, 4096).to(torch.bfloat16)
    x_dn = torch.randn(M, 14336).to(torch.bfloat16)

    def one_pass():
        for name, mat2, sz in packs:
            cpu_path.tinygemm_linear(x_dn if name == "down" else x_in, mat2, 128, sz)

    med, runs = _cpu_time(one_pass, args.cpu_seconds)
    del packs
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": n, "kind": "port",
            "sample": f"C2 shapes, {layers} layers x 4 linears (0.93 GB of int4 weights, beyond host cache), "
                      f"M={M}, torch tinygemm _weight_int4pack_mm_for_cpu, median of {runs} passes",
            "ms_per_layer": round(med * 1e3 / layers, 3), "cpu": _cpu_model(),
            "naive": _cpu_naive_int4(args, [(N, K) for _, K, N in wl.LLAMA8B_PROJ] * 2, M,
                                     "C2 shapes, 2 layers x 4 linears (232 MB of int4 weights)")}


def _cpu_naive_int4(args, shapes, M: int, what: str) -> dict:
    """The reference's naive CPU int4 forward (worker_quant.py:847-853: the bf16 dequant and a bf16
    F.linear below 16 rows, the fp32 dequant and an fp32 GEMM from 16 rows) over ``shapes``
    (N, K), timed beside tinygemm on the same host cores."""
    import torch
    from oracle import cpu_path
    n = cpu_path.tune_cpu_threads()
    packs = [(K, _cpu_int4_random(N, K, 7000 + i)) for i, (N, K) in enumerate(shapes)]
    xs = {K: torch.randn(M, K).to(torch.bfloat16) for _, K in shapes}

    def one():
        for K, (q, s, z) in packs:
            cpu_path.naive_linear(xs[K], q, s, z, K, 128, bits=4)

    med, runs = _cpu_time(one, max(2.0, args.cpu_seconds / 2), min_runs=2)
    nbytes = sum(N * K // 2 + N * (K // 128) * 4 + M * K * 2 + M * N * 2 for N, K in shapes)
    rule = "bf16 dequant + bf16 F.linear" if M < 16 else "fp32 dequant + fp32 GEMM"
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": n,
            "sample": f"{what}, M={M}, naive rule ({rule}), median of {runs} passes"}


# ---------------------------------------------------------------------------------------------
# C1: one int4 linear 1 x 4096 -> 4096 (rotated over 64 distinct copies, 571 MB)
# ---------------------------------------------------------------------------------------------
def bench_c1(args, dev):
    import torch
    from infinitemodel_amd import ops, workloads as wl
    M = args.m or 1
    lins = [wl.rtn_int4_linear(4096, 4096, i, dev, name=f"c1.{i}") for i in range(64)]
    op, layout = _w4_module_layout(lins)
    x = wl.activations(M, 4096, 0, dev)
    y = torch.empty((M, 4096), dtype=torch.bfloat16, device=dev)

    def step():
        for L in lins:
            op(x, L.q, 128, (L.s, L.z), out=y)

    ms = _time_steps(_graph_or_eager(step, not args.no_graph), args.steps, args.warmup)
    b = lins[0].algorithmic_bytes(M)
    us = ms * 1e3 / len(lins)
    roof = _hbm_roofline(_w4_decode_kernel(M, layout), b, us, _traffic(f"c1_m{M}"))
    cfg = {"workload": f"C1 single int4 g128 linear {M}x4096->4096, {len(lins)} distinct copies per step",
           "M": M, "launches_per_step": len(lins), "distinct_bytes_per_step": b * len(lins),
           "packed_layout": layout}
    cpu = None
    if not args.no_cpu:
        from oracle import cpu_path
        n = cpu_path.tune_cpu_threads()
        packs = [cpu_path.tinygemm_prepare(*_cpu_int4_random(4096, 4096, i), 128) for i in range(48)]
        xc = torch.randn(M, 4096).to(torch.bfloat16)

        def one():
            for mat2, sz in packs:
                cpu_path.tinygemm_linear(xc, mat2, 128, sz)

        med, runs = _cpu_time(one, args.cpu_seconds)
        cpu = {"value": round(b * len(packs) / med / 1e9, 3), "unit": "GB/s", "cores": n, "kind": "port",
               "sample": f"C1 shape, 48 distinct weights (0.43 GB), torch tinygemm, median of {runs} passes",
               "cpu": _cpu_model(),
               "naive": _cpu_naive_int4(args, [(4096, 4096)] * 8, M, "C1 shape, 8 distinct weights (71 MB)")}
    return _line(round(b * len(lins) / (ms * 1e-3) / 1e9, 2), "GB/s", ms, args, cfg, roof, cpu)


# ---------------------------------------------------------------------------------------------
# C3: int2 g64 at 70B shapes (fp16 s/z, non-integer zeros), 8 copies of each shape
# ---------------------------------------------------------------------------------------------
def bench_c3(args, dev):
    import torch
    from infinitemodel_amd import ops, workloads as wl
    M = args.m or 1
    shapes = [(28672, 8192), (8192, 28672)]
    sets = []
    for i in range(8):
        for j, (N, K) in enumerate(shapes):
            q, s, z = wl.int2_random_linear(N, K, 2000 + 2 * i + j, dev)
            sets.append((N, K, q, s, z))
    qs, op, layout = _packed_module_layout([t[2] for t in sets], 2, lambda i: sets[i][0], 64)
    sets = [(N, K, q, s, z) for (N, K, _, s, z), q in zip(sets, qs)]
    xs = {K: wl.activations(M, K, 7, dev) for _, K in shapes}
    ys = {N: torch.empty((M, N), dtype=torch.bfloat16, device=dev) for N, _ in shapes}

    def step():
        for N, K, q, s, z in sets:
            op(xs[K], q, 64, (s, z), out=ys[N])

    ms = _time_steps(_graph_or_eager(step, not args.no_graph), args.steps, args.warmup)
    nbytes = sum(q.numel() + s.numel() * 2 + z.numel() * 2 + M * K * 2 + M * N * 2 for N, K, q, s, z in sets)
    us = ms * 1e3 / len(sets)
    entry = "imq_linear_w2_tiled" if layout == "line-tiled" else "imq_linear_w2"
    if M == 2:   # the line kernel's 16 waves hold K 8192 at M = 2, not 28672
        kern = "w2_line_kernel (8192->28672) + " + ("w2_ksplit_kernel + splitk_rows_reduce_kernel (28672->8192)"
                                                    if layout == "line-tiled" else "w2_skinny_kernel (28672->8192)")
    else:
        kern = ("w2_line_kernel" if M == 1 else
                "w2_ksplit_kernel + splitk_rows_reduce_kernel" if M <= 16 and (M > 4 or layout == "line-tiled") else
                "w2_skinny_kernel" if M <= 16 else "gemm_wq_kernel<2>")
    roof = _hbm_roofline(f"{kern} ({entry}, M={M})", nbytes / len(sets), us, _traffic(f"c3_m{M}"))
    cfg = {"workload": f"C3 int2 g64 70B shapes 8192->28672 and 28672->8192, M={M}, 8 copies each", "M": M,
           "launches_per_step": len(sets), "distinct_bytes_per_step": nbytes,
           "weights": "int2 g64, fp16 scale ~U(0.005,0.05), zero ~U(0,3)", "packed_layout": layout}
    cpu = None
    if not args.no_cpu:
        from oracle import cpu_path
        n = cpu_path.tune_cpu_threads()
        g = torch.Generator().manual_seed(1)
        cs = [(torch.randint(0, 256, (N, K // 4), generator=g, dtype=torch.uint8),
               (torch.rand(N, K // 64, generator=g) * 0.045 + 0.005).half(),
               (torch.rand(N, K // 64, generator=g) * 3).half(), K) for N, K in shapes]
        xc = {K: torch.randn(M, K).to(torch.bfloat16) for _, K in shapes}

        def one():
            for q, s, z, K in cs:
                cpu_path.naive_linear(xc[K], q, s, z, K, 64, bits=2)

        med, runs = _cpu_time(one, args.cpu_seconds, min_runs=2)
        cb = sum(q.numel() + s.numel() * 4 + M * K * 2 + M * q.shape[0] * 2 for q, s, z, K in cs)
        cpu = {"value": round(cb / med / 1e9, 3), "unit": "GB/s", "cores": n, "kind": "port",
               "sample": f"C3 both shapes once, naive dequant + F.linear (the reference's only CPU int2 path), "
                         f"M={M}, median of {runs}", "cpu": _cpu_model()}
    return _line(round(nbytes / (ms * 1e-3) / 1e9, 2), "GB/s", ms, args, cfg, roof, cpu)


# ---------------------------------------------------------------------------------------------
# C4: prefill dequant-GEMM (int4 g128 or int8 per-row), 4096->14336 and 14336->4096
# ---------------------------------------------------------------------------------------------
def _c4_module_path(quant: str, shapes, dev) -> dict:
    """Which path the drop-in module itself keeps for prefill at each C4 shape: the QuantLinear4 /
    int8 QuantLinear built over the same kind of weights, prepare_fused run (its self-check and
    its measured naive-vs-fused rule at the production prefill chunk), the decision read back.
    The module's log lines are kept out of stdout (one JSON line there)."""
    import contextlib
    import io
    from infinitemodel_amd import workloads as wl, worker_quant as wq
    out = {}
    log = io.StringIO()
    with contextlib.redirect_stdout(log):
        for i, (N, K) in enumerate(shapes):
            if quant == "int4":
                L = wl.rtn_int4_linear(N, K, 5000 + i, dev)
                mod = wq._quant4_linear_cls()(L.q, L.s, L.z, None, K, 128)
                mod.prepare_fused()
                thr = getattr(mod, "_naive_m_min", 0)
                path = ("naive (fused op not bound)" if getattr(mod, "_fused", None) is None
                        else f"naive from row bucket {thr}" if thr else "fused at every M")
            else:
                q, s = wl.int8_linear(N, K, 5000 + i, dev)
                mod = wq._quant_linear_cls()(q, s, None)
                mod.prepare_fused()
                m_max = getattr(mod, "_w8_m_max", None)
                path = ("naive (int8 op not bound)" if getattr(mod, "_w8", None) is None
                        else "fused at every M" if not m_max else f"fused up to M={m_max}")
            out[f"{K}->{N}"] = path
    return out


C4_SHAPES = [(14336, 4096), (4096, 14336)]
_c4_layout = "row"   # the packed layout of the last _c4_fused call's weights


def _c4_fused(quant: str, M: int, dev, steps: int, warmup: int, use_graph: bool = True):
    """The fused prefill step of C4: 6 copies of each shape (374 MB int4 / 705 MB int8, past the
    MALL) through imq_linear_w4 / imq_linear_w8, timed as _time_steps does. Returns (ms per step,
    TFLOP/s, the (N, K, fn) sets, the activations by K, the outputs by N)."""
    import torch
    from infinitemodel_amd import ops, workloads as wl
    sets = []
    for i in range(6):
        for j, (N, K) in enumerate(C4_SHAPES):
            if quant == "int4":
                L = wl.rtn_int4_linear(N, K, 5000 + 2 * i + j, dev)
                op, layout = _w4_module_layout([L])
                sets.append((N, K, lambda x, y, L=L, op=op: op(x, L.q, 128, (L.s, L.z), out=y)))
            else:
                pairs, op8, layout = _w8_module_layout([wl.int8_linear(N, K, 5000 + 2 * i + j, dev)])
                q, s = pairs[0]
                sets.append((N, K, lambda x, y, q=q, s=s, op8=op8: op8(x, q, s, out=y)))
    xs = {K: wl.activations(M, K, 9, dev) for _, K in C4_SHAPES}
    ys = {N: torch.empty((M, N), dtype=torch.bfloat16, device=dev) for N, _ in C4_SHAPES}

    def step():
        for N, K, fn in sets:
            fn(xs[K], ys[N])

    ms = _time_steps(_graph_or_eager(step, use_graph), steps, warmup)
    flops = sum(2.0 * M * N * K for N, K, _ in sets)
    global _c4_layout
    _c4_layout = layout
    return ms, flops / (ms * 1e-3), sets, xs, ys


def also_c4(args, dev) -> list:
    """C4's fused prefill lines (int4 / int8 at M = 2048 and 512), measured inside the default
    run after its own line so that they run under the same clock; value in TFLOP/s of the fused
    step alone (the naive, bf16-GEMM and CPU legs are bench.py --config c4's)."""
    import torch
    out = []
    steps, warmup = min(args.steps, 20), min(args.warmup, 5)
    for quant in ("int4", "int8"):
        for M in (2048, 512):
            ms, tf, sets, xs, ys = _c4_fused(quant, M, dev, steps, warmup, not args.no_graph)
            out.append({"workload": f"C4 prefill {quant} 4096->14336 and 14336->4096, M={M}",
                        "value": round(tf / 1e12, 3), "unit": "TFLOP/s", "ms_per_step": round(ms, 5),
                        "steps": steps, "warmup": warmup, "frac_of_peak": round(tf / BF16_PEAK, 4),
                        "launches_per_step": len(sets)})
            del sets, xs, ys
            torch.cuda.empty_cache()
    return out


def bench_c4(args, dev):
    import torch
    from infinitemodel_amd import ops, workloads as wl
    M = args.m or 2048
    shapes = C4_SHAPES
    ms, tf, sets, xs, ys = _c4_fused(args.quant, M, dev, args.steps, args.warmup, not args.no_graph)
    flops = sum(2.0 * M * N * K for N, K, _ in sets)
    # the module's naive prefill path on the same weights: the bit-exact HIP dequant to bf16, then
    # the bf16 GEMM (hipBLASLt, as F.linear) -- what _bench_large_m_naive weighs the fused kernel
    # against
    naive_sets = []
    for i, (N, K, _fn) in enumerate(sets[:2]):
        if args.quant == "int4":
            L = wl.rtn_int4_linear(N, K, 5000 + i, dev)
            naive_sets.append((N, K, lambda x, y, L=L, K=K: torch.mm(
                x, ops.dequant_w4(L.q, L.s, L.z, K, 128, torch.bfloat16).t(), out=y)))
        else:
            q, s_ = wl.int8_linear(N, K, 5000 + i, dev)
            naive_sets.append((N, K, lambda x, y, q=q, s_=s_: torch.mm(
                x, ops.dequant_w8(q, s_, torch.bfloat16).to(torch.bfloat16).t(), out=y)))

    def naive_step():
        for N, K, fn in naive_sets:
            fn(xs[K], ys[N])

    ms_naive = _time_steps(naive_step, max(3, args.steps // 4), 2)
    tf_naive = sum(2.0 * M * N * K for N, K, _ in naive_sets) / (ms_naive * 1e-3)
    # the platform's own bf16 GEMM (hipBLASLt through torch.mm) on unquantized bf16 weights of the
    # same shapes, no dequantization: the rate the vendor library reaches on this box and shape
    dense_sets = []
    for i, (N, K, _fn) in enumerate(sets[:2]):
        if args.quant == "int4":
            L = wl.rtn_int4_linear(N, K, 5000 + i, dev)
            wt = ops.dequant_w4(L.q, L.s, L.z, K, 128, torch.bfloat16)
        else:
            q, s_ = wl.int8_linear(N, K, 5000 + i, dev)
            wt = ops.dequant_w8(q, s_, torch.bfloat16).to(torch.bfloat16)
        dense_sets.append((N, K, wt))

    def dense_step():
        for N, K, wt in dense_sets:
            torch.mm(xs[K], wt.t(), out=ys[N])

    ms_dense = _time_steps(dense_step, max(3, args.steps // 4), 2)
    tf_dense = sum(2.0 * M * N * K for N, K, _ in dense_sets) / (ms_dense * 1e-3)
    del dense_sets
    bits = 4 if args.quant == "int4" else 8
    gemm = (f"gemm_rb_kernel<{bits}> + splitk_sum_kernel (register-B GEMM" if M > 512
            else f"gemm_wq_kernel<{bits}> + splitk_sum_kernel (LDS-dequant GEMM")
    roof = {"bound": "mfma", "achieved": round(tf / 1e12, 2), "peak": BF16_PEAK / 1e12, "unit": "TFLOP/s",
            "frac": round(tf / BF16_PEAK, 4), "traffic": _traffic(f"c4_{args.quant}_m{M}"),
            "kernel": f"{gemm}, imq_linear_{'w4' if bits == 4 else 'w8'} prefill)",
            "avg_launch_us": round(ms * 1e3 / len(sets), 3), "flops_per_launch": flops / len(sets)}
    wbytes = sum(N * K * (0.53125 if args.quant == "int4" else 1.0) for N, K, _ in sets)
    cfg = {"workload": f"C4 prefill {args.quant} 4096->14336 and 14336->4096, M={M}", "M": M,
           "quant": args.quant, "launches_per_step": len(sets), "distinct_bytes_per_step": int(wbytes),
           "packed_layout": _c4_layout,
           "naive": {"value": round(tf_naive / 1e12, 3), "unit": "TFLOP/s",
                     "path": "imq dequant to bf16 + F.linear (hipBLASLt), both shapes, eager",
                     "fused_speedup": round(tf / tf_naive, 3)},
           "bf16_gemm": {"value": round(tf_dense / 1e12, 3), "unit": "TFLOP/s",
                         "path": "torch.mm (hipBLASLt) on unquantized bf16 weights, both shapes, eager",
                         "fused_ratio": round(tf / tf_dense, 3)},
           "module_path": _c4_module_path(args.quant, shapes, dev)}
    cpu = None
    if not args.no_cpu:
        from oracle import cpu_path
        n = cpu_path.tune_cpu_threads()
        g = torch.Generator().manual_seed(2)
        xc = {K: torch.randn(M, K).to(torch.bfloat16) for _, K in shapes}
        if args.quant == "int4":
            cs = [(K, _cpu_int4_random(N, K, 7 + K)) for N, K in shapes]

            def one():
                for K, (q, s, z) in cs:
                    cpu_path.naive_linear(xc[K], q, s, z, K, 128, bits=4)
        else:
            cs = [(K, torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8),
                   (torch.rand(N, 1, generator=g) * 1e-3).half()) for N, K in shapes]

            def one():
                for K, q, s in cs:
                    cpu_path.naive_linear_int8(xc[K], q, s)

        med, runs = _cpu_time(one, args.cpu_seconds, min_runs=2)
        cf = sum(2.0 * M * N * K for N, K in shapes)
        cpu = {"value": round(cf / med / 1e12, 4), "unit": "TFLOP/s", "cores": n, "kind": "port",
               "sample": f"C4 both shapes once at M={M}: rows >= 16 -> fp32 dequant + fp32 GEMM "
                         f"(worker_quant.py:847-852 / 411-417), median of {runs}", "cpu": _cpu_model()}
    return _line(round(tf / 1e12, 3), "TFLOP/s", ms, args, cfg, roof, cpu)


# ---------------------------------------------------------------------------------------------
# C5: OLMoE fused MoE experts (E=64, top-8, H=2048, I=1024), 16 layers routed independently
# ---------------------------------------------------------------------------------------------
MOE_LAYERS = 16     # C5 T=1: 16 x 8 hit experts x 3.34 MB = 428 MB of distinct weights, past the MALL


def _moe_kernels(B: int, E: int, gK: int) -> str:
    """The kernels one imq_moe_experts_w4 call launches for B routed rows, E experts and gate_up
    K_pad gK (the dispatch rule of moe.hip): direct decode when 4 B <= 5 E (7 E when gK > 2048:
    line kernel workgroups of more than 4 waves); the register-B grouped GEMM when B gK >= 32768 E
    (8192 E when gK > 2048); the token-sorted line kernels between."""
    if 4 * B <= (7 if gK > 2048 else 5) * E:
        return "moe_gu_line_kernel + moe_dn_line_kernel (direct decode)"
    if B * gK >= (8192 if gK > 2048 else 32768) * E:
        return ("moe_sort_kernel (with the hidden rows' group sums) + gemm_rb_kernel MoE forms "
                "(gate_up, down; scale-folded) + moe_combine_bf16_kernel")
    return "moe_sort_kernel + moe_line_kernel (gate_up, down) + moe_combine_kernel"


def _moe_layer_bytes(idx, per_expert: int, act_bytes: int) -> tuple:
    """(algorithmic bytes, distinct experts) of one MoE layer: each hit expert's weights once, the
    activations in and out, and the routing ids and weights."""
    import torch
    U = int(torch.unique(idx).numel())
    return U * per_expert + act_bytes + idx.numel() * 6, U


def bench_c5(args, dev):
    import torch
    from infinitemodel_amd import ops, workloads as wl
    T = args.m or 1
    layers = [wl.olmoe_layer(dev, seed=3000 + l) for l in range(MOE_LAYERS)]
    routes = [wl.olmoe_routing(T, dev, seed=4 + l) for l in range(MOE_LAYERS)]
    x = wl.activations(T, 2048, 11, dev)

    def step():
        for (gu, dn), (idx, w) in zip(layers, routes):
            ops.moe_experts_w4(x, idx, w, gu, dn, 128)

    ms = _time_steps(_graph_or_eager(step, not args.no_graph), args.steps, args.warmup)
    per_expert = 3342336
    per_layer = [_moe_layer_bytes(idx, per_expert, T * 2048 * 2 * 2) for idx, _ in routes]
    nbytes = sum(b for b, _ in per_layer)
    us = ms * 1e3 / len(layers)
    kern = _moe_kernels(T * 8, 64, 2048)
    roof = _hbm_roofline(f"imq_moe_experts_w4: {kern} (one MoE layer)", nbytes / len(layers), us,
                         _traffic(f"c5_t{T}"))
    cfg = {"workload": f"C5 OLMoE fused MoE experts, T={T}, top-8 of 64, H=2048, I=1024, {len(layers)} layers "
                       f"routed independently", "T": T,
           "distinct_experts_per_layer": [u for _, u in per_layer], "layers_per_step": len(layers),
           "distinct_bytes_per_step": nbytes}
    cpu = None
    if not args.no_cpu:
        from oracle import cpu_path
        n = cpu_path.tune_cpu_threads()
        cl = wl.olmoe_layer(torch.device("cpu"), seed=3000)
        idx, w = routes[0]
        xc, ic, wc = x.cpu(), idx.cpu(), w.cpu()
        med, runs = _cpu_time(lambda: cpu_path.moe_eager_cpu(xc, ic, wc, cl[0], cl[1], 128), args.cpu_seconds,
                              min_runs=2)
        cpu = {"value": round(per_layer[0][0] / med / 1e9, 3), "unit": "GB/s", "cores": n, "kind": "port",
               "sample": f"C5 one layer at T={T}: the eager per-expert loop over bf16 dequantized experts "
                         f"(modeling_olmoe.py:301-325 over Packed4Tensor3D), median of {runs}",
               "cpu": _cpu_model()}
    return _line(round(nbytes / (ms * 1e-3) / 1e9, 2), "GB/s", ms, args, cfg, roof, cpu)


# ---------------------------------------------------------------------------------------------
# gpt-oss-20b fused experts (transpose-packed int4, interleaved clamped GLU, per-expert biases)
# ---------------------------------------------------------------------------------------------
def bench_gptoss(args, dev):
    import torch
    from infinitemodel_amd import ops, workloads as wl
    T = args.m or 1
    E, k, H, I = 32, 4, 2880, 2880
    layers = [wl.gptoss_layer(dev, seed=5000 + 7 * l) for l in range(MOE_LAYERS)]
    routes = [wl.olmoe_routing(T, dev, E=E, k=k, seed=40 + l) for l in range(MOE_LAYERS)]
    x = wl.activations(T, H, 13, dev)

    def step():
        for (gu, dn, bgu, bdn), (idx, w) in zip(layers, routes):
            ops.moe_experts_w4(x, idx, w, gu, dn, 128, act="gptoss", gu_bias=bgu, dn_bias=bdn)

    ms = _time_steps(_graph_or_eager(step, not args.no_graph), args.steps, args.warmup)
    ng = -(-H // 128)                      # 23 groups: the reference's packed K_pad 2944
    per_expert = (2 * I + H) * (ng * 64 + ng * 2 * 2) + (2 * I + H) * 2     # codes + s/z + biases
    per_layer = [_moe_layer_bytes(idx, per_expert, T * H * 2 * 2) for idx, _ in routes]
    nbytes = sum(b for b, _ in per_layer)
    us = ms * 1e3 / len(layers)
    kern = _moe_kernels(T * k, E, 3072)
    roof = _hbm_roofline(f"imq_moe_experts_w4_ex gptoss: {kern} (one MoE layer)", nbytes / len(layers), us,
                         _traffic(f"gptoss_t{T}"))
    cfg = {"workload": f"gpt-oss-20b fused experts, T={T}, top-{k} of {E}, H=I={H}, {len(layers)} layers routed "
                       f"independently", "T": T,
           "distinct_experts_per_layer": [u for _, u in per_layer], "layers_per_step": len(layers),
           "distinct_bytes_per_step": nbytes,
           "note": "algorithmic bytes count the reference's K_pad 2944 packing; the kernel layout "
                   "reads rows padded to 3072"}
    return _line(round(nbytes / (ms * 1e-3) / 1e9, 2), "GB/s", ms, args, cfg, roof, None)


# ---------------------------------------------------------------------------------------------
# int8 lm_head decode (head_quant=int8) at the Qwen2.5-7B head
# ---------------------------------------------------------------------------------------------
def bench_head(args, dev):
    """Two distinct copies of the head (1.09 GB, past the 256 MB MALL) launched alternately, so no
    launch finds its matrix cached from the one before."""
    import torch
    from infinitemodel_amd import ops, workloads as wl
    M = args.m or 1
    N, K = 152064, 3584
    heads, op, layout = _w8_module_layout([wl.int8_linear(N, K, 17 + i, dev, dtype=torch.bfloat16) for i in range(2)])
    x = wl.activations(M, K, 18, dev)
    y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)

    def step():
        for q, s in heads:
            op(x, q, s, out=y)

    ms = _time_steps(_graph_or_eager(step, not args.no_graph), args.steps, args.warmup)
    nbytes = N * K + N * 2 + M * K * 2 + M * N * 2
    entry = "imq_linear_w8_tiled" if layout == "line-tiled" else "imq_linear_w8"
    roof = _hbm_roofline(f"{'w8_line_kernel' if M <= 4 else 'w8_skinny_kernel'} ({entry}, M={M})", nbytes,
                         ms * 1e3 / len(heads), _traffic(f"head_m{M}"))
    cfg = {"workload": f"int8 lm_head 3584 -> 152064 (Qwen2.5-7B), M={M}, {len(heads)} distinct copies per step",
           "M": M, "launches_per_step": len(heads), "packed_layout": layout,
           "weights": "int8 per-row symmetric, bf16 scale", "distinct_bytes_per_step": nbytes * len(heads)}
    cpu = None
    if not args.no_cpu:
        from oracle import cpu_path
        n = cpu_path.tune_cpu_threads()
        rows = 16384
        q, s = heads[0]
        qc, sc_, xc = q[:rows].cpu(), s[:rows].cpu(), x.cpu()
        med, runs = _cpu_time(lambda: cpu_path.naive_linear_int8(xc, qc, sc_), args.cpu_seconds)
        cb = rows * K + rows * 2 + M * K * 2 + M * rows * 2
        cpu = {"value": round(cb / med / 1e9, 3), "unit": "GB/s", "cores": n, "kind": "port",
               "sample": f"the reference's CPU int8 forward (naive dequant + F.linear, worker_quant.py:"
                         f"411-417, 439-440) over the first {rows} head rows, median of {runs}",
               "cpu": _cpu_model()}
    return _line(round(nbytes * len(heads) / (ms * 1e-3) / 1e9, 2), "GB/s", ms, args, cfg, roof, cpu)


# ---------------------------------------------------------------------------------------------
# Hardware ceilings (the measurement probes of libimq, csrc/probe.hip)
# ---------------------------------------------------------------------------------------------
PROBE_SWEEP = [(u, w, nt) for u in (2, 4, 8, 16) for w in (1, 2, 4, 8) for nt in (0, 1)]


class _Probe:
    """Read-only stream launches (imq_probe_stream) over fixed buffer lists."""

    def __init__(self, dev):
        import torch
        from infinitemodel_amd import _lib
        self.L = _lib.lib()
        self.call = _lib.call
        self.dev = dev
        self.sink = torch.empty(int(self.L.imq_probe_sink_bytes()) // 4 + 1, dtype=torch.int32, device=dev)

    def buffers(self, bufs):
        """(ptrs, n16s, total) device tables for a list of contiguous 16-byte-aligned tensors."""
        import torch
        for b in bufs:
            nb = b.numel() * b.element_size()
            assert b.is_contiguous() and nb % 16 == 0 and b.data_ptr() % 16 == 0 and nb >= 16
        ptrs = torch.tensor([b.data_ptr() for b in bufs], dtype=torch.int64, device=self.dev)
        n16 = [b.numel() * b.element_size() // 16 for b in bufs]
        return ptrs, torch.tensor(n16, dtype=torch.int64, device=self.dev), sum(n16), len(bufs)

    def read(self, tab, cfg):
        import torch
        ptrs, n16, total, nbuf = tab
        u, w, nt = cfg
        self.call("imq_probe_stream", ptrs.data_ptr(), n16.data_ptr(), nbuf, total, u, w, nt,
                  self.sink.data_ptr(), self.sink.numel() * 4, torch.cuda.current_stream(self.dev).cuda_stream)


def _cfg_name(cfg) -> str:
    return f"U{cfg[0]}_wg{cfg[1]}{'_nt' if cfg[2] else ''}"


def bench_ceiling(args, dev):
    """The C2 stack's weights (codes + scale + zero of all 128 linears, 3.7 GB) read by the
    read-only stream probe, every probe configuration of PROBE_SWEEP (loads per lane, workgroups
    per CU, non-temporal loads):
      per kind (qkv / o / gate_up / down): 32 launches of that kind's 32 distinct linears as one
        graph, the fastest configuration per kind -- the per-launch ceiling of that linear -- beside
        the decode kernels (imq_linear_w4 at M=1) on the same 32 linears;
      the whole pass: 128 launches in layer order with each kind's fastest configuration (value),
        the decode kernels over the same pass, and one persistent launch over all 384 buffers
        (the same bytes with no launch boundary, fastest configuration)."""
    import torch
    from infinitemodel_amd import ops, workloads as wl
    pr = _Probe(dev)
    lins = wl.llama8b_stack(dev)
    op, layout = _w4_module_layout(lins)
    kinds = [n for n, _, _ in wl.LLAMA8B_PROJ]
    tabs = [pr.buffers([L.q, L.s, L.z]) for L in lins]
    kind_of = [L.name.split(".")[1] for L in lins]
    wbytes = [16 * t[2] for t in tabs]
    x_in = wl.activations(1, 4096, 1, dev)
    x_dn = wl.activations(1, 14336, 2, dev)
    ys = {n: torch.empty((1, N), dtype=torch.bfloat16, device=dev) for n, _, N in wl.LLAMA8B_PROJ}
    g = not args.no_graph
    st, wu = max(5, args.steps // 2), 2

    def t_us(fn, n):
        return _time_steps(_graph_or_eager(fn, g), st, wu) * 1e3 / n

    per_kind = {}
    best = {}
    for k in kinds:
        ids = [i for i, kk in enumerate(kind_of) if kk == k]
        sweep = {}
        for cfg in PROBE_SWEEP:
            sweep[_cfg_name(cfg)] = round(t_us(lambda ids=ids, cfg=cfg: [pr.read(tabs[i], cfg) for i in ids],
                                               len(ids)), 3)
        bname = min(sweep, key=sweep.get)
        best[k] = next(c for c in PROBE_SWEEP if _cfg_name(c) == bname)
        x = x_dn if k == "down" else x_in

        def dec(ids=ids, x=x, k=k):
            for i in ids:
                L = lins[i]
                op(x, L.q, L.G, (L.s, L.z), out=ys[k])

        d_us = t_us(dec, len(ids))
        b = wbytes[ids[0]]
        per_kind[k] = {"weight_bytes": b, "probe_best": bname, "probe_us": sweep[bname],
                       "probe_gbs": round(b / (sweep[bname] * 1e-6) / 1e9, 1),
                       "decode_us": round(d_us, 3), "decode_over_probe": round(d_us / sweep[bname], 3),
                       "sweep_us": sweep}

    def pass_probe():
        for i in range(len(lins)):
            pr.read(tabs[i], best[kind_of[i]])

    def pass_decode():
        for L, k in zip(lins, kind_of):
            op(x_dn if k == "down" else x_in, L.q, L.G, (L.s, L.z), out=ys[k])

    ms_a = _time_steps(_graph_or_eager(pass_probe, g), args.steps, args.warmup)
    ms_c = _time_steps(_graph_or_eager(pass_decode, g), args.steps, args.warmup)
    all_tab = pr.buffers([b for L in lins for b in (L.q, L.s, L.z)])
    pers = {}
    for cfg in PROBE_SWEEP:
        pers[_cfg_name(cfg)] = round(_time_steps(_graph_or_eager(lambda cfg=cfg: pr.read(all_tab, cfg), g), st, wu), 5)
    pbest = min(pers, key=pers.get)
    total = sum(wbytes)
    gbs = lambda ms: round(total / (ms * 1e-3) / 1e9, 2)   # noqa: E731
    roof = _hbm_roofline("probe_stream_kernel (one launch per linear, fastest configuration per kind)",
                         total / len(lins), ms_a * 1e3 / len(lins), None)
    cfg = {"workload": "C2 llama-3-8b int4 weights (128 linears, codes + scale + zero), read-only ceilings",
           "weight_bytes_per_step": total, "distinct_bytes_per_step": total,
           "per_launch_pass_gbs": gbs(ms_a), "decode_pass_gbs": gbs(ms_c), "decode_ms": round(ms_c, 5),
           "persistent_best": pbest, "persistent_ms": pers[pbest], "persistent_gbs": gbs(pers[pbest]),
           "persistent_sweep_ms": pers, "per_kind": per_kind,
           "note": "GB/s over the weight bytes only (the decode line adds x and y, 0.1%); per-kind figures "
                   "are 32 launches of one kind as one graph"}
    return _line(gbs(ms_a), "GB/s", ms_a, args, cfg, roof, None, data="synthetic: the C2 stack's RTN-packed weights")


def bench_stream(args, dev):
    """HBM stream ceilings on buffers far past the 256 MB MALL: the read-only probe over one 4 GiB
    buffer (every PROBE_SWEEP configuration, one launch per step), the probe's copy kernel and
    torch's copy over 1 GiB -> 1 GiB. value = the fastest read-only configuration."""
    import torch
    pr = _Probe(dev)
    big = torch.empty(4 << 30, dtype=torch.uint8, device=dev).fill_(3)
    tab = pr.buffers([big])
    st, wu = max(5, args.steps // 2), 2
    reads = {}
    for cfg in PROBE_SWEEP:
        ms = _time_steps(lambda cfg=cfg: pr.read(tab, cfg), st, wu)
        reads[_cfg_name(cfg)] = round(big.numel() / (ms * 1e-3) / 1e9, 1)
    del big, tab
    torch.cuda.empty_cache()
    n = 1 << 30
    a = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    b = torch.empty_like(a)
    copies = {}
    for u in (2, 4, 8):
        for w in (2, 4, 8):
            ms = _time_steps(lambda u=u, w=w: pr.call("imq_probe_copy", b.data_ptr(), a.data_ptr(), n, u, w,
                                                      torch.cuda.current_stream(dev).cuda_stream), st, wu)
            copies[f"U{u}_wg{w}"] = round(2 * n / (ms * 1e-3) / 1e9, 1)
    ok = bool(torch.equal(a[:: 1 << 20], b[:: 1 << 20]))
    ms_t = _time_steps(lambda: b.copy_(a), st, wu)
    rbest = max(reads, key=reads.get)
    cbest = max(copies, key=copies.get)
    ms = big_ms = 4 * (1 << 30) / (reads[rbest] * 1e9) * 1e3
    roof = _hbm_roofline(f"probe_stream_kernel {rbest} (4 GiB read-only)", 4 << 30, big_ms * 1e3, None)
    cfg = {"workload": "HBM stream ceilings: 4 GiB read-only, 1 GiB -> 1 GiB copy", "read_best": rbest,
           "read_sweep_gbs": reads, "copy_best": cbest, "copy_gbs": copies[cbest], "copy_sweep_gbs": copies,
           "copy_checked": ok, "torch_copy_gbs": round(2 * n / (ms_t * 1e-3) / 1e9, 1),
           "note": "copy GB/s count bytes read + bytes written"}
    return _line(reads[rbest], "GB/s", ms, args, cfg, roof, None, data="synthetic: constant-filled buffers")


def bench_launch(args, dev):
    """Launch cost of a chain of dependent kernels on one stream: 128 empty kernels (one
    workgroup per CU, and one workgroup), replayed as a HIP graph and launched eagerly.
    value = µs per launch, graph, one workgroup per CU."""
    import torch
    from infinitemodel_amd import _lib
    L = _lib.lib()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    st = lambda: torch.cuda.current_stream(dev).cuda_stream   # noqa: E731
    out = {}
    for grid in (cus, 1):
        def chain(grid=grid):
            for _ in range(128):
                _lib.call("imq_probe_empty", grid, st())
        out[f"graph_grid{grid}_us"] = round(_time_steps(_graph_or_eager(chain, True), args.steps, args.warmup)
                                            * 1e3 / 128, 3)
        out[f"eager_grid{grid}_us"] = round(_time_steps(chain, max(5, args.steps // 4), 2) * 1e3 / 128, 3)
    v = out[f"graph_grid{cus}_us"]
    cfg = {"workload": "128 dependent empty kernels per step on one stream", "cus": cus, **out}
    return _line(v, "us/launch", v * 128 / 1e3, args, cfg, None, None, hib=False, dtype="none",
                 data="synthetic: empty kernels")


def bench_mfma(args, dev):
    """MFMA issue peak: 4 independent accumulator chains per wave of v_mfma_f32_32x32x16_bf16
    (and v_mfma_f32_16x16x32_bf16) on register operands, 1 / 2 / 4 workgroups of 4 waves per CU.
    value = the fastest 32x32x16 figure (TFLOP/s)."""
    import torch
    pr = _Probe(dev)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    iters = 20000
    res, mss = {}, {}
    for kind, name, fl in ((0, "32x32x16", 32768), (1, "16x16x32", 16384)):
        for w in (1, 2, 4):
            ms = _time_steps(lambda kind=kind, w=w: pr.call("imq_probe_mfma", kind, iters, w, pr.sink.data_ptr(),
                                                           pr.sink.numel() * 4,
                                                           torch.cuda.current_stream(dev).cuda_stream),
                             max(5, args.steps // 4), 2)
            flops = cus * w * 4 * 4 * iters * fl
            res[f"{name}_wg{w}"] = round(flops / (ms * 1e-3) / 1e12, 1)
            mss[f"{name}_wg{w}"] = ms
    best = max((k for k in res if k.startswith("32x32")), key=res.get)
    roof = {"bound": "mfma", "achieved": res[best], "peak": BF16_PEAK / 1e12, "unit": "TFLOP/s",
            "frac": round(res[best] * 1e12 / BF16_PEAK, 4), "traffic": None, "kernel": f"probe_mfma_kernel {best}"}
    cfg = {"workload": "bf16 MFMA issue peak on register operands", "iters": iters, "tflops": res}
    return _line(res[best], "TFLOP/s", mss[best], args, cfg, roof, None, data="synthetic: register operands")


# ---------------------------------------------------------------------------------------------
def bench_copy(args, dev):
    """Plain device copy of 1 GiB (read 1 GiB + write 1 GiB per launch): calibrates the PMC
    FETCH_SIZE / WRITE_SIZE counters against known bytes."""
    import torch
    n = 1 << 30
    a = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    b = torch.empty_like(a)
    ms = _time_steps(lambda: b.copy_(a), args.steps, args.warmup)
    roof = _hbm_roofline("copy (elementwise_kernel)", 2 * n, ms * 1e3, None)
    return _line(round(2 * n / (ms * 1e-3) / 1e9, 2), "GB/s", ms, args,
                 {"workload": "device copy 1 GiB -> 1 GiB", "bytes_read": n, "bytes_written": n}, roof, None)


def trace_summary(path: str, steps: int, region: int = -1, period=None) -> str:
    """Markdown summary of the timed steps in a rocprofv3 kernel-trace CSV: the dispatches between
    the two marker kernels ``_time_steps`` launches around them (``region``: which timed region of
    the run, -1 = the last), per kernel the count, mean / min / max duration (µs) and total; with
    ``period`` (launches per step) the mean per launch position; and the kernel time per step
    (total / steps), to set beside the line's ms_per_step."""
    import csv
    rows = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if r.get("Kind", "KERNEL_DISPATCH") != "KERNEL_DISPATCH":
                continue
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    rows.sort()
    marks = [i for i, (_, _, n) in enumerate(rows) if MARK_KERNEL in n]
    if len(marks) < 2 or len(marks) % 2:
        raise SystemExit(f"{path}: {len(marks)} marker dispatches ({MARK_KERNEL}), expected pairs")
    pairs = list(zip(marks[0::2], marks[1::2]))
    a, b = pairs[region]
    sel = rows[a + 1:b]
    if not sel or len(sel) % steps:
        raise SystemExit(f"{path}: {len(sel)} dispatches in the timed region, not a multiple of {steps} steps")
    by = {}
    for t0, t1, n in sel:
        by.setdefault(n, []).append((t1 - t0) / 1e3)
    total = sum(sum(v) for v in by.values())
    out = [f"timed region {region} of {len(pairs)}: {len(sel)} dispatches = {steps} steps x {len(sel) // steps}, "
           f"window {(sel[-1][1] - sel[0][0]) / 1e3:.1f} µs, kernel time {total:.1f} µs, "
           f"**kernel time per step {total / steps:.2f} µs**", "",
           "| kernel | count | mean µs | min µs | max µs | total µs |", "|---|---|---|---|---|---|"]
    for n, v in sorted(by.items(), key=lambda kv: -sum(kv[1])):
        short = n if len(n) <= 110 else n[:107] + "..."
        out.append(f"| `{short}` | {len(v)} | {sum(v) / len(v):.3f} | {min(v):.3f} | {max(v):.3f} | {sum(v):.1f} |")
    if period:
        out += ["", f"mean µs per launch position (period {period}):", "",
                "| position | kernel | mean µs |", "|---|---|---|"]
        for p in range(period):
            v = [(t1 - t0) / 1e3 for i, (t0, t1, n) in enumerate(sel) if i % period == p]
            out.append(f"| {p} | `{sel[p][2][:70]}` | {sum(v) / len(v):.3f} |")
    return "\n".join(out)


BENCH = {"c1": bench_c1, "c2": bench_c2, "c3": bench_c3, "c4": bench_c4, "c5": bench_c5, "gptoss": bench_gptoss,
         "head": bench_head, "copy": bench_copy, "ceiling": bench_ceiling, "stream": bench_stream,
         "launch": bench_launch, "mfma": bench_mfma}


def main():
    args = _parse()
    if args.trace_summary:
        print(trace_summary(args.trace_summary, args.steps, args.region, args.period), flush=True)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the quantized-linear hot path runs per GPU and this "
              "build's GPU boxes have one GPU; use --gpus 1",
              file=sys.stderr, flush=True)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("no ROCm GPU visible", file=sys.stderr, flush=True)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    line = BENCH[args.config](args, dev)
    if args.config == "c2" and args.m in (None, 1) and not args.no_also:
        line["also"] = also_c4(args, dev)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
