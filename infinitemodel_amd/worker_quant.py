"""Reference-compatible quantized Linear modules, backed by the gfx950 kernels of libimq.

This module is the plugin boundary of the reference's worker_quant.py: a caller switches by import
and finds the same lazy class factories, constructors, buffer names (``qweight``/``scale``/``zero``
are state_dict keys), attributes (``in_features``, ``group_size``, ``bias``, ``_fused``,
``_fused_tried``, ``_naive_m_min``), methods (``forward``, ``_dequant``, ``prepare_fused``), op
builders with the reference's call signatures, packers, scope walkers, the streamed expert
builders and the CPU helpers its callers import (client.py:539-549).

Layout of this file:
  flags and small helpers | device timing and the prefill dispatch rule | op builders | dequant |
  QuantLinear4 / QuantLinear2 | QuantLinear (int8) | packed expert weights (tensor subclasses) |
  Packed4Tensor3D | fused MoE forwards | int8 experts | lm_head option | packers | scope walkers
  (in-memory and streamed) | MoE layer structure helpers | CPU path | placement sweep.

Device behaviour:

* ROCm device: every kernel is a hand-written HIP kernel of libimq. ``prepare_fused`` binds the
  fused op after a self-check (never raises; on failure the module keeps the naive path). The
  naive path is ``F.linear(x, _dequant(dtype))`` where ``_dequant`` is libimq's bit-exact dequant
  kernel, so a missing library raises ``ImqUnavailable`` from forward instead of silently running
  a torch substitute.
* CPU device: the reference's CPU semantics in torch: the int4 module binds torch's CPU tinygemm
  op after the same kind of self-check, the others dequantize in ``dtype``, and rows >= 16 take
  an fp32 dequant + fp32 GEMM (worker_quant.py:725-815, 847-852).

Op builder names: the reference names its builders after Triton (``_w4a16_triton_op`` ...). Those
names are kept as aliases because other code reads them; the callables they return launch HIP
kernels (``_w4a16_hip_op`` ...). There is no Triton anywhere in this package.
"""
from __future__ import annotations

import contextlib
import os
import threading

from . import shard_compile as _sc

# ---- flags (worker_quant.py:97-115, 183-198; same environment switches) ---------------------
_FUSED_INT4 = os.environ.get("IM_FUSED_INT4", "1") != "0"
_FUSED_W8A16 = os.environ.get("IM_FUSED_W8A16", "1") != "0"
_FUSED_INT2 = os.environ.get("IM_FUSED_INT2", "1") != "0"
_LARGE_M_NAIVE = os.environ.get("IM_LARGE_M_NAIVE", "1") != "0"
# int4 / int2 modules on ROCm hold their packed weight in the line-tiled layout once bound (this
# build's own switch, no counterpart in the reference; "0" keeps the row layout, de-aliased rows)
_LINE_TILED = os.environ.get("IM_LINE_TILED", "1") != "0"

# CPU-resident matmuls upcast to fp32 from this many activation rows (fp32 GEMM beats the bf16
# GEMV once compute-bound); tune_cpu_threads lowers it to 1 on CPUs whose bf16 GEMM is unusable.
_CPU_FP32_MIN_ROWS = 16
_CPU_FP32_GEMM = True
_CPU_BF16_GEMM_OK = None

_INT4_GROUP = _sc.INT4_GROUP
_INT2_GROUP = _sc.INT2_GROUP
_W8_PROBE_M = 256            # prefill-shaped probe of the int8 bind decision (worker_quant.py:885)

# Self-check bounds (the reference's): fused linears mean rel < 0.05; fused MoE mean < 0.03 and
# max < 0.1. Prefill dispatch: the naive path must be >= 13% faster to take over.
_LINEAR_CHECK_REL = 0.05
_MOE_CHECK_MEAN, _MOE_CHECK_MAX = 0.03, 0.1
_NAIVE_MARGIN = 0.87

# Leaf names of MoE routers that are bare nn.Linear modules; never quantized (worker_quant.py:3051).
_ROUTER_LEAF_NAMES = frozenset({"gate", "router", "wg"})

# Token counts up to this take the fused MoE path; larger ones the eager per-expert loop. The
# reference fuses only T <= 8 because its kernel re-reads each expert's weight once per routed
# row; the HIP path groups rows by expert, so prefill-sized T stays on it.
_FUSED_MOE_T_MAX = int(os.environ.get("IM_FUSED_MOE_T_MAX", "4096"))

# Streamed expert builds fetch at most this many bf16 bytes of experts per request.
_STREAM_CHUNK_BYTES = 256 << 20
_STREAM_CHUNK_MAX = 64

_BUILD_LOCK = threading.RLock()


def _log(msg: str) -> None:
    print(msg, flush=True)


def _rows(x) -> int:
    """Flattened row count of an activation ``[*, in_features]``."""
    n = 1
    for d in x.shape[:-1]:
        n *= int(d)
    return n


def _m_bucket(m: int) -> int:
    """The row bucket a call of m rows is dispatched by: the next power of two (0 and 1 stay)."""
    return m if m <= 1 else 1 << (int(m) - 1).bit_length()


def _cpu_fp32_worth(x) -> bool:
    import torch
    return (_CPU_FP32_GEMM and x.device.type == "cpu" and x.dtype != torch.float32
            and _rows(x) >= _CPU_FP32_MIN_ROWS)


def _is_rocm_device(dev) -> bool:
    import torch
    return dev.type == "cuda" and getattr(torch.version, "hip", None) is not None


def _rel_err(y, ref) -> tuple:
    """(mean relative error, max relative error) of y against ref, the self-check metrics
    mean|y-ref| / (mean|ref| + 1e-6) and max|y-ref| / (max|ref| + 1e-6)."""
    d = (y.float() - ref.float()).abs()
    r = ref.float().abs()
    return (d.mean() / (r.mean() + 1e-6)).item(), (d.max() / (r.max() + 1e-6)).item()


def _bf16_rows(m: int, k: int, dev, scale: float = 1.0):
    import torch
    return torch.randn(m, k, device=dev, dtype=torch.bfloat16) * scale


def _pad_cols(x, width: int):
    """x with zero columns appended up to ``width`` (the packed K), contiguous."""
    import torch.nn.functional as F
    if x.shape[-1] != width:
        x = F.pad(x, (0, width - x.shape[-1]))
    return x.contiguous()


# ---- device timing and the prefill dispatch rule ---------------------------------------------
def _device_ms(fn, dev, iters: int, warmup: int) -> float:
    """Mean device time per call of ``fn`` in ms, between two HIP events on the device's current
    stream (the launches' own clock, without host-side launch overhead)."""
    import torch
    with torch.cuda.device(dev):
        for _ in range(warmup):
            fn()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(iters):
            fn()
        stop.record()
        stop.synchronize()
        return start.elapsed_time(stop) / max(1, iters)


def _time_cuda(fn, dev, iters: int = 30, warmup: int = 8) -> float:
    """ms per call of ``fn`` on ``dev`` (the reference's helper signature, worker_quant.py:888-899),
    measured on the device's event clock."""
    return _device_ms(fn, dev, iters, warmup)


_LARGE_M_CHOICE: dict = {}


def _prefill_bench_m() -> int:
    """Row bucket of the production prefill chunk (INFINITEMODEL_PREFILL_CHUNK, default 2048)."""
    raw = os.environ.get("INFINITEMODEL_PREFILL_CHUNK", "") or "2048"
    chunk = int(raw) if raw.strip().isdigit() else 2048
    return _m_bucket(chunk if chunk > 1 else 2048)


def _naive_threshold(top: int, fused_ms: float, naive_ms) -> int:
    """Smallest row bucket from which the naive dequant + BLAS GEMM replaces the fused kernel, or
    0 for "fused at every M" -- the decision of worker_quant.py:1290-1310 as a pure rule over
    timings. ``naive_ms(m)`` times the naive path at m rows (called lazily, top first). Naive
    must beat the fused time at ``top`` by the margin; then each halved bucket down to 16 keeps
    naive while it still beats the fused time extrapolated linearly in rows."""
    if not naive_ms(top) < _NAIVE_MARGIN * fused_ms:
        return 0
    per_row = fused_ms / max(1, top)
    chosen, m = top, top // 2
    while m >= 16 and naive_ms(m) < _NAIVE_MARGIN * per_row * m:
        chosen, m = m, m // 2
    return chosen


def _bench_large_m_naive(mod, tag: str) -> int:
    """Measured prefill dispatch threshold of a module whose fused op is bound in ``mod._fused``
    (worker_quant.py:1252-1335): times the fused op and the naive path on the device and applies
    ``_naive_threshold``. One measurement per (tag, N, K_pad, group), cached; a failing
    measurement returns 0 (fused everywhere) and is not cached."""
    if not _LARGE_M_NAIVE:
        return 0
    try:
        import torch
        import torch.nn.functional as F
        qw, packed, op, in_pad = mod._fused
        key = (tag, int(qw.shape[0]), int(in_pad), int(getattr(mod, "group_size", 0)))
        if key in _LARGE_M_CHOICE:
            return _LARGE_M_CHOICE[key]
        dev = qw.device
        if tag == "int8":
            fused = lambda x: op(x, qw, packed)                      # noqa: E731
        else:
            fused = lambda x: op(x, qw, mod.group_size, packed)      # noqa: E731
        top = _prefill_bench_m()
        x_top = _bf16_rows(top, mod.in_features, dev)
        x_top_k = _pad_cols(x_top, in_pad)
        t_fused = _device_ms(lambda: fused(x_top_k), dev, iters=2, warmup=1)
        seen = {}

        def naive_ms(m: int) -> float:
            x = x_top if m == top else _bf16_rows(m, mod.in_features, dev)
            seen[m] = _device_ms(lambda: F.linear(x, mod._dequant(torch.bfloat16)), dev, iters=2, warmup=1)
            return seen[m]

        thr = _naive_threshold(top, t_fused, naive_ms)
        _LARGE_M_CHOICE[key] = thr
        _log(f"[{tag}] prefill dispatch N={key[1]} K_pad={in_pad}: fused {t_fused:.3f} ms at M={top}, naive "
             + ", ".join(f"M={m} {t:.3f} ms" for m, t in sorted(seen.items(), reverse=True))
             + f" -> {'naive from row bucket ' + str(thr) if thr else 'fused at every M'}")
        return thr
    except Exception as exc:
        _log(f"[{tag}] prefill dispatch measurement skipped ({exc!r}) -> fused at every M")
        return 0


# ---- op builders (worker_quant.py:926-1225, 1342-1495): HIP kernels behind the same signatures --
_OPS: dict = {}


def _build_op(name: str, make):
    """Thread-safe lazy build; None (and one log line) when libimq cannot be loaded."""
    if name in _OPS:
        return _OPS[name]
    with _BUILD_LOCK:
        if name not in _OPS:
            try:
                from . import _lib
                _lib.lib()
                _OPS[name] = make()
            except Exception as exc:
                _log(f"[imq] {name} unavailable ({exc!r})")
                _OPS[name] = None
    return _OPS[name]


def _ops_attr(attr: str):
    def make():
        from . import ops
        return getattr(ops, attr)
    return make


def _w4a16_hip_op():
    """``op(x[M,Kpad] bf16, qweight u8[N,Kpad/2], group, (scale, zero) [N,ng]) -> y[M,N] bf16``."""
    return _build_op("w4a16", _ops_attr("linear_w4"))


def _w4a16_tiled_hip_op():
    """``op(x[M,Kpad] bf16, qweight_tiled u8[N,Kpad/2], 128, (scale, zero) [N,ng]) -> y[M,N] bf16``
    on weights in the line-tiled layout (ops.line_tile)."""
    return _build_op("w4a16_tiled", _ops_attr("linear_w4_tiled"))


def _w2a16_tiled_hip_op():
    """``op(x[M,Kpad] bf16, qweight_tiled u8[N,Kpad/4], 64, (scale, zero) [N,ng]) -> y[M,N] bf16``
    on weights in the line-tiled layout (ops.line_tile)."""
    return _build_op("w2a16_tiled", _ops_attr("linear_w2_tiled"))


def _w2a16_hip_op():
    """``op(x[M,Kpad] bf16, qweight u8[N,Kpad/4], group, (scale, zero) [N,ng]) -> y[M,N] bf16``."""
    return _build_op("w2a16", _ops_attr("linear_w2"))


def _w8a16_hip_op():
    """``op(x[M,K] bf16, qweight int8[N,K], scale[N,1]) -> y[M,N] bf16``."""
    return _build_op("w8a16", _ops_attr("linear_w8"))


def _w8a16_tiled_hip_op():
    """``op(x[M,K] bf16, qweight_tiled int8[N,K], scale[N,1]) -> y[M,N] bf16`` on weights in the
    line-tiled layout (ops.line_tile)."""
    return _build_op("w8a16_tiled", _ops_attr("linear_w8_tiled"))


def _w4a16_moe_hip_op():
    """``op(x[B,Kin] bf16, eid[B], q u8[E,N,Kpad/2], scale, zero [E,N,ng], group, in_features)
    -> y[B,N] bf16``: each row b against expert eid[b]."""
    return _build_op("w4a16_moe", _ops_attr("moe_rows_w4"))


# Reference builder names, kept for callers that look them up by name.
_w4a16_triton_op = _w4a16_hip_op
_w2a16_triton_op = _w2a16_hip_op
_w8a16_triton_op = _w8a16_hip_op
_w4a16_moe_op = _w4a16_moe_hip_op


# ---- dequant helpers ------------------------------------------------------------------------
def _dequant_g_torch(qweight, scale, zero, in_features: int, group_size: int, dtype, bits: int):
    """The reference dequant in torch (worker_quant.py:638-648, 1652-1664): unpack, ``.to(dtype)``,
    ``(qf - zero.to(dtype)) * scale.to(dtype)``, slice. Used for CPU-resident modules."""
    import torch
    out = qweight.shape[0]
    mask = (1 << bits) - 1
    fields = [((qweight >> (bits * i)) & mask).to(torch.int16) for i in range(8 // bits)]
    q = torch.stack(fields, dim=2).reshape(out, -1)
    ng = scale.shape[-1]
    qf = q.reshape(out, ng, group_size).to(dtype)
    w = (qf - zero.to(dtype).unsqueeze(2)) * scale.to(dtype).unsqueeze(2)
    return w.reshape(out, ng * group_size)[:, :in_features].contiguous()


def _dequant_g(qweight, scale, zero, in_features: int, group_size: int, dtype, bits: int):
    import torch
    if qweight.device.type == "cuda":
        from . import ops
        if dtype not in (torch.bfloat16, torch.float16, torch.float32):
            raise TypeError(f"dequant to {dtype} is not supported on the GPU path")
        f = ops.dequant_w4 if bits == 4 else ops.dequant_w2
        return f(qweight, scale, zero, in_features, group_size, dtype)
    return _dequant_g_torch(qweight, scale, zero, in_features, group_size, dtype, bits)


def _selfcheck_rel(op_call, ref_w, in_features: int, in_pad: int, dev, Ms=(1, 8)):
    """Worst mean relative error of ``op_call(x_padded)`` against ``F.linear(x, ref_w)`` over the
    row counts ``Ms``; returns (rel, first failing M or 0) under the < 0.05 rule. Both the decode
    rows (M 1) and a multi-row call are checked: they run different kernels."""
    import torch.nn.functional as F
    worst = 0.0
    for m in Ms:
        x = _bf16_rows(m, in_features, dev)
        rel, _ = _rel_err(op_call(_pad_cols(x, in_pad)), F.linear(x, ref_w))
        worst = max(worst, rel)
        if not rel < _LINEAR_CHECK_REL:
            return rel, m
    return worst, 0


def _dealias_rows(qw):
    """Re-home a packed weight on rows padded by 64 bytes, returning the ``[:, :rs]`` view
    (worker_quant.py:680-690): a power-of-two row stride puts every row on the same HBM channel
    set; the kernels read through ``stride(0)`` so the view needs no other change."""
    import torch
    if qw.shape[1] % 128 != 0:
        return qw
    buf = torch.zeros((qw.shape[0], qw.shape[1] + 64), dtype=torch.uint8, device=qw.device)
    buf[:, :qw.shape[1]].copy_(qw)
    return buf[:, :qw.shape[1]]


# ---- group-wise int4 / int2 linear modules ---------------------------------------------------
def _line_tiling_fits(mod, bits: int, in_pad: int) -> bool:
    """Whether a group-wise module's packed weight can take the line-tiled layout: rows a multiple
    of 16, dense rows of whole 128-byte line-steps (K_pad a multiple of 256 codes for int4, 512
    for int2), the kernels' groups (128 for int4, 64 for int2), scale and zero of one dtype."""
    cpb = 8 // bits
    return (_LINE_TILED and mod.group_size == (128 if bits == 4 else 64) and mod.qweight.shape[0] % 16 == 0
            and mod.qweight.shape[1] * cpb == in_pad and mod.qweight.shape[1] % 128 == 0
            and mod.scale.dtype == mod.zero.dtype)


def _bind_line_tiled(mod, bits: int, in_pad: int, tag: str) -> bool:
    """Bind QuantLinear4/2 to the line-tiled kernels: tile the packed weight (a dense copy), check
    the tiled op against the bf16 dequant at M 1 and 8, then replace ``qweight`` with the tiled
    array (the row-layout buffer is released; ``_dequant`` and ``state_dict`` convert back).
    False (module unchanged) when the tiled op is unavailable or fails the check."""
    import torch
    from . import ops
    op = _w4a16_tiled_hip_op() if bits == 4 else _w2a16_tiled_hip_op()
    if op is None:
        return False
    tiled = ops.line_tile(mod.qweight)
    pair = (mod.scale, mod.zero)
    G = mod.group_size
    rel, bad_m = _selfcheck_rel(lambda xk: op(xk, tiled, G, pair), mod._dequant(torch.bfloat16),
                                mod.in_features, in_pad, tiled.device)
    if bad_m:
        _log(f"[{tag}] hip w{bits}a16 (line-tiled) self-check rel={rel:.3f} at M={bad_m} -> row layout")
        return False
    mod.qweight = tiled
    mod._line_tiled = True
    mod._fused = (tiled, pair, op, in_pad)
    return True


def _bind_group_rocm(mod, bits: int, tag: str) -> None:
    """ROCm binding of QuantLinear4/2 (worker_quant.py:668-724): weights that fit it take the
    line-tiled layout; otherwise de-alias the packed rows, check the HIP op against the bf16
    dequant at M 1 and 8 and bind ``_fused``; then measure the prefill dispatch threshold. Raises
    on errors; the caller keeps the naive path."""
    import torch
    op = _w4a16_hip_op() if bits == 4 else _w2a16_hip_op()
    if op is None:
        return
    G = mod.group_size
    in_pad = mod.scale.shape[1] * G
    if _line_tiling_fits(mod, bits, in_pad) and _bind_line_tiled(mod, bits, in_pad, tag):
        mod._naive_m_min = _bench_large_m_naive(mod, tag)
        return
    mod.qweight = _dealias_rows(mod.qweight)
    pair = (mod.scale, mod.zero)
    rel, bad_m = _selfcheck_rel(lambda xk: op(xk, mod.qweight, G, pair), mod._dequant(torch.bfloat16),
                                mod.in_features, in_pad, mod.qweight.device)
    if bad_m:
        _log(f"[{tag}] hip w{bits}a16 self-check rel={rel:.3f} at M={bad_m} -> naive")
        return
    mod._fused = (mod.qweight, pair, op, in_pad)
    mod._naive_m_min = _bench_large_m_naive(mod, tag)


def _bind_int4_cpu_tinygemm(mod) -> None:
    """CPU binding of QuantLinear4 (worker_quant.py:725-815): torch's CPU int4 GEMM over the same
    codes, no re-quantization -- ``(q - z) s`` is fed as ``(q - 8) S + (8 - z) S`` with
    ``sz = [ng, N, 2]`` bf16 pairs (S, (8 - z) S). Bound when it agrees with the naive dequant on
    a 4-row input (mean rel < 0.05); the packed copy then replaces qweight / scale / zero, which
    are released (the reference's memory rule for this path)."""
    import torch
    import torch.nn.functional as F
    aten = torch.ops.aten
    if not (hasattr(aten, "_weight_int4pack_mm_for_cpu") and hasattr(aten, "_convert_weight_to_int4pack_for_cpu")):
        return
    G = mod.group_size
    out, ng = mod.scale.shape
    in_pad = ng * G
    codes = torch.stack(((mod.qweight & 0x0F), (mod.qweight >> 4)), dim=2).reshape(out, in_pad)
    S = mod.scale.float()
    pairs = torch.stack((S, (8.0 - mod.zero.float()) * S), dim=2)          # [N, ng, 2]
    sz = pairs.permute(1, 0, 2).contiguous().to(torch.bfloat16)            # [ng, N, 2]
    mat2 = aten._convert_weight_to_int4pack_for_cpu(codes.to(torch.int32).contiguous(), 8)
    op = aten._weight_int4pack_mm_for_cpu
    x = _bf16_rows(4, mod.in_features, mod.qweight.device)
    rel, _ = _rel_err(op(_pad_cols(x, in_pad), mat2, G, sz), F.linear(x, mod._dequant(torch.bfloat16)))
    if not rel < _LINEAR_CHECK_REL:
        _log(f"[int4] cpu int4 GEMM self-check rel={rel:.3f} -> naive")
        return
    mod._fused = (mat2, sz, op, in_pad)
    mod.qweight = None
    mod.scale = None
    mod.zero = None


def _line_untile_torch(qt):
    """Line-tiled -> row layout with torch index ops (host-resident tensors): row r of a 16-row
    tile holds at piece p of line-step l the block's slot 64 h + (r & 7) + 8 ((p >> 2) ^ h) +
    16 (p & 3), h = r >> 3."""
    import torch
    N, KB = qt.shape
    KL = KB // 128
    slot = torch.tensor([64 * (r >> 3) + (r & 7) + 8 * ((p >> 2) ^ (r >> 3)) + 16 * (p & 3)
                         for r in range(16) for p in range(8)], dtype=torch.long, device=qt.device)
    blocks = qt.reshape(N // 16, KL, 128, 16)[:, :, slot]           # [tile, l, (r, p), byte]
    return blocks.reshape(N // 16, KL, 16, 8, 16).permute(0, 2, 1, 3, 4).reshape(N, KB).contiguous()


def _untile_on_save(module, state_dict, prefix, local_metadata):
    """state_dict hook: a line-tiled qweight is saved in the row layout."""
    key = prefix + "qweight"
    if getattr(module, "_line_tiled", False) and state_dict.get(key) is not None:
        state_dict[key] = module._row_qweight().detach()


def _tile_on_load(module, state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys, error_msgs):
    """load_state_dict pre-hook: a row-layout qweight loaded into a line-tiled module is tiled
    first, so the copy lands in the layout the bound kernels read."""
    key = prefix + "qweight"
    incoming = state_dict.get(key)
    if getattr(module, "_line_tiled", False) and incoming is not None and module.qweight is not None:
        from . import ops
        if tuple(incoming.shape) == tuple(module.qweight.shape):
            state_dict[key] = ops.line_tile(incoming.to(module.qweight.device))


def _make_group_linear_cls(bits: int):
    import torch
    from torch import nn
    import torch.nn.functional as F

    tag = "int4" if bits == 4 else "int2"

    class _GroupQuantLinear(nn.Module):
        def __init__(self, qweight, scale, zero, bias, in_features, group_size):
            super().__init__()
            self.register_buffer("qweight", qweight)   # uint8 [out, in_pad*bits/8]
            self.register_buffer("scale", scale)        # [out, n_groups]
            self.register_buffer("zero", zero)          # [out, n_groups]
            self.bias = bias
            self.in_features = in_features
            self.group_size = group_size
            # a bound module may hold qweight line-tiled (_line_tiled); state_dict and
            # load_state_dict keep the reference's row layout
            self._line_tiled = False
            self.register_state_dict_post_hook(_untile_on_save)
            self.register_load_state_dict_pre_hook(_tile_on_load)

        def _row_qweight(self):
            """The packed weight in the row layout (a converted copy while line-tiled)."""
            if not self._line_tiled:
                return self.qweight
            if self.qweight.is_cuda:
                from . import ops
                return ops.line_untile(self.qweight)
            return _line_untile_torch(self.qweight)   # a tiled module moved off the GPU

        def _dequant(self, dtype):
            """The dequantized weight ``[out, in_features]`` in ``dtype``, bit-exact to the
            reference dequant (libimq kernel on a ROCm device, torch on CPU)."""
            return _dequant_g(self._row_qweight(), self.scale, self.zero, self.in_features, self.group_size,
                              dtype, bits)

        def prepare_fused(self):
            """Bind the fused op once the module sits on its final device (ROCm: the HIP op;
            CPU, int4: torch's CPU int4 GEMM). Idempotent; never raises; any failure keeps the
            naive path (worker_quant.py:650-815, 1666-1722)."""
            enabled = _FUSED_INT4 if bits == 4 else _FUSED_INT2
            if (not enabled or getattr(self, "_fused", None) is not None or getattr(self, "_fused_tried", False)
                    or self.qweight is None):
                return
            self._fused_tried = True
            dev = self.qweight.device
            try:
                if _is_rocm_device(dev):
                    _bind_group_rocm(self, bits, tag)
                elif dev.type == "cpu" and bits == 4:
                    _bind_int4_cpu_tinygemm(self)
            except Exception as exc:
                self._fused = None
                _log(f"[{tag}] fused w{bits}a16 bind failed on {dev} ({exc!r}) -> naive")

        def _takes_fused(self, x) -> bool:
            if getattr(self, "_fused", None) is None:
                return False
            threshold = getattr(self, "_naive_m_min", 0)
            return not (threshold and self.qweight is not None and _m_bucket(_rows(x)) >= threshold)

        def forward(self, x):
            if self._takes_fused(x):
                packed, pair, op, in_pad = self._fused
                xs = x.reshape(-1, self.in_features).to(torch.bfloat16)
                y = op(_pad_cols(xs, in_pad), packed, self.group_size, pair)
                y = y.reshape(*x.shape[:-1], y.shape[-1]).to(x.dtype)
                return y if self.bias is None else y + self.bias.to(y.dtype)
            if _cpu_fp32_worth(x):
                b = None if self.bias is None else self.bias.float()
                return F.linear(x.float(), self._dequant(torch.float32), b).to(x.dtype)
            return F.linear(x, self._dequant(x.dtype), self.bias)

    _GroupQuantLinear.__name__ = _GroupQuantLinear.__qualname__ = "QuantLinear4" if bits == 4 else "QuantLinear2"
    return _GroupQuantLinear


_CLASSES: dict = {}


def _lazy_class(name: str, make):
    """Build a module/tensor class on first use (torch imported lazily), once, under the lock."""
    cls = _CLASSES.get(name)
    if cls is None:
        with _BUILD_LOCK:
            cls = _CLASSES.get(name)
            if cls is None:
                cls = make()
                if cls is not None:
                    _CLASSES[name] = cls
    return cls


def _quant4_linear_cls():
    """QuantLinear4(qweight u8[N,K_pad/2], scale[N,ng], zero[N,ng], bias, in_features,
    group_size) (worker_quant.py:621-856)."""
    return _lazy_class("QuantLinear4", lambda: _make_group_linear_cls(4))


def _quant2_linear_cls():
    """QuantLinear2(qweight u8[N,K_pad/4], scale, zero, bias, in_features, group_size)
    (worker_quant.py:1635-1761)."""
    return _lazy_class("QuantLinear2", lambda: _make_group_linear_cls(2))


# ---- int8 per-row linear ---------------------------------------------------------------------
def _dequant8(qweight, scale, dtype):
    """``qweight.to(dtype) * scale`` with torch's promotion (worker_quant.py:439)."""
    if qweight.device.type == "cuda":
        from . import ops
        return ops.dequant_w8(qweight, scale, dtype)
    return qweight.to(dtype) * scale


def _w8_binding(mod):
    """Decide whether QuantLinear's HIP int8 op serves the module (worker_quant.py:442-505).

    Three measured gates, in order: the op agrees with the bf16 dequant at M 1 and 4 (mean rel
    < 0.05); it beats dequant + F.linear at one decode row; and a prefill-shaped probe (M 256)
    decides whether it also serves prefill. Returns (op, m_max) -- m_max 0 serves every M, 1
    decode only -- or None with the reason logged."""
    import torch
    import torch.nn.functional as F
    op = _w8a16_hip_op()
    if op is None:
        return None
    dev = mod.qweight.device
    K = int(mod.qweight.shape[1])
    s_bf16 = mod.scale.to(torch.bfloat16)
    naive = lambda x: F.linear(x, _dequant8(mod.qweight, s_bf16, torch.bfloat16))   # noqa: E731
    fused = lambda x: op(x, mod.qweight, mod.scale)                                 # noqa: E731
    for m in (1, 4):
        x = _bf16_rows(m, K, dev)
        rel, _ = _rel_err(fused(x), naive(x))
        if not rel < _LINEAR_CHECK_REL:
            _log(f"[int8] hip w8a16 self-check rel={rel:.3f} at M={m} -> naive")
            return None
    x1 = _bf16_rows(1, K, dev)
    t_fused, t_naive = _time_cuda(lambda: fused(x1), dev), _time_cuda(lambda: naive(x1), dev)
    if not t_fused < t_naive:
        _log(f"[int8] hip w8a16 {t_fused:.3f} ms vs dequant + F.linear {t_naive:.3f} ms -> naive")
        return None
    xp = _bf16_rows(_W8_PROBE_M, K, dev)
    p_fused = _time_cuda(lambda: fused(xp), dev, iters=6, warmup=2)
    p_naive = _time_cuda(lambda: naive(xp), dev, iters=6, warmup=2)
    return op, (0 if p_fused < p_naive else 1)


def _make_int8_linear_cls():
    import torch
    from torch import nn
    import torch.nn.functional as F

    class QuantLinear(nn.Module):
        def __init__(self, qweight, scale, bias):
            super().__init__()
            self.register_buffer("qweight", qweight)   # int8 [out, in]
            self.register_buffer("scale", scale)        # [out, 1]
            self.bias = bias
            # bound to the HIP op for every M, the packed weight may be line-tiled (_line_tiled);
            # state_dict and load_state_dict keep the reference's row layout
            self._line_tiled = False
            self.register_state_dict_post_hook(_untile_on_save)
            self.register_load_state_dict_pre_hook(_tile_on_load)

        def _row_qweight(self):
            """The packed weight in the row layout (a converted copy while line-tiled)."""
            if not self._line_tiled:
                return self.qweight
            if self.qweight.is_cuda:
                from . import ops
                return ops.line_untile(self.qweight)
            return _line_untile_torch(self.qweight)

        def _dequant(self, dtype):
            return _dequant8(self._row_qweight(), self.scale, dtype)

        def _kernel_serves(self, x) -> bool:
            if getattr(self, "_w8", None) is None or x.dtype is not torch.bfloat16:
                return False
            m_max = getattr(self, "_w8_m_max", 0)
            return not m_max or _rows(x) <= m_max

        def forward(self, x):
            if _cpu_fp32_worth(x):
                b = None if self.bias is None else self.bias.float()
                w = self.qweight.float() * self.scale.float()
                return F.linear(x.float(), w, b).to(x.dtype)
            if self._kernel_serves(x):
                y = self._w8(x.reshape(-1, x.shape[-1]), self.qweight, self.scale)
                y = y.reshape(*x.shape[:-1], y.shape[-1])
                return y if self.bias is None else y + self.bias
            return F.linear(x, self._dequant(x.dtype), self.bias)

        def prepare_fused(self):
            """Bind the HIP int8 op when ``_w8_binding`` accepts it (``_w8``, ``_w8_m_max``).
            ROCm only; idempotent; never raises."""
            if getattr(self, "_fused_tried", False) or not _FUSED_W8A16:
                return
            self._fused_tried = True
            if not _is_rocm_device(self.qweight.device):
                return
            try:
                bound = _w8_binding(self)
            except Exception as exc:
                _log(f"[int8] hip w8a16 bind failed on {self.qweight.device} ({exc!r}) -> naive")
                bound = None
            if bound is not None:
                self._w8, self._w8_m_max = bound
                if self._w8_m_max == 0:
                    try:
                        _tile_w8(self)
                    except Exception as exc:
                        _log(f"[int8] line-tiled bind failed ({exc!r}) -> row layout")

    return QuantLinear


def _tile_w8(mod) -> None:
    """A QuantLinear whose HIP op serves every M takes the line-tiled layout (rows a multiple of
    16, dense rows of a multiple of 128 bytes): the tiled op is checked against the bf16 dequant at
    M 1 and 4 (and 32, a prefill row count), then ``qweight`` is replaced by the tiled copy. A module
    that serves prefill through the naive path keeps the row layout, which that path reads."""
    import torch
    from . import ops
    q = mod.qweight
    if not (_LINE_TILED and q.shape[0] % 16 == 0 and q.shape[1] % 128 == 0 and q.is_contiguous()):
        return
    op = _w8a16_tiled_hip_op()
    if op is None:
        return
    tiled = ops.line_tile(q.view(torch.uint8)).view(torch.int8)
    ref_w = _dequant8(q, mod.scale.to(torch.bfloat16), torch.bfloat16)
    for m in (1, 4, 32):
        x = _bf16_rows(m, q.shape[1], q.device)
        rel, _ = _rel_err(op(x, tiled, mod.scale), torch.nn.functional.linear(x, ref_w))
        if not rel < _LINEAR_CHECK_REL:
            _log(f"[int8] hip w8a16 (line-tiled) self-check rel={rel:.3f} at M={m} -> row layout")
            return
    mod.qweight = tiled
    mod._line_tiled = True
    mod._w8 = op


def _quant_linear_cls():
    """QuantLinear(qweight int8[N,K], scale[N,1], bias) (worker_quant.py:391-508)."""
    return _lazy_class("QuantLinear", _make_int8_linear_cls)


# ---- one expert's packed weight as a tensor subclass -----------------------------------------
# The eager experts loop calls ``F.linear(x, self.gate_up_proj[e])``; the holders hand it a tensor
# subclass whose ``F.linear`` runs the fused kernel on the packed bytes and whose every other use
# sees the dequantized weight (worker_quant.py:1501-1585, 2734-2806).
def _make_packed_weight_cls(name: str, layout, kernel, materialize, accepts):
    """A wrapper tensor class: ``layout(*parts) -> (shape, dtype, device)`` describes the logical
    weight, ``kernel(x, parts) -> y`` is its F.linear, ``materialize(parts)`` its dense value,
    ``accepts(x)`` gates the kernel on the activation."""
    import torch
    import torch.nn.functional as F
    from torch.utils._pytree import tree_map

    linear_funcs = {F.linear, torch._C._nn.linear}

    def linear_call(args, kwargs):
        names = ("input", "weight", "bias")
        vals = list(args) + [None] * (3 - len(args))
        for i, n in enumerate(names):
            if n in kwargs:
                vals[i] = kwargs[n]
        return vals[0], vals[1], vals[2]

    class PackedWeight(torch.Tensor):
        @staticmethod
        def __new__(cls, *parts):
            shape, dtype, device = layout(*parts)
            t = torch.Tensor._make_wrapper_subclass(cls, shape, dtype=dtype, device=device, requires_grad=False)
            t._parts = parts
            return t

        def _materialize(self):
            return materialize(self._parts)

        @classmethod
        def _dense(cls, tree):
            return tree_map(lambda a: a._materialize() if isinstance(a, cls) else a, tree)

        @classmethod
        def __torch_function__(cls, func, types, args=(), kwargs=None):
            kwargs = kwargs or {}
            if func in linear_funcs:
                x, w, bias = linear_call(args, kwargs)
                if isinstance(w, cls) and accepts(x):
                    y = kernel(x, w._parts)
                    y = y.reshape(*x.shape[:-1], y.shape[-1])
                    return y if bias is None else y + bias.to(y.dtype)
            dargs, dkwargs = cls._dense((args, kwargs))
            return func(*dargs, **dkwargs)

        @classmethod
        def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
            dargs, dkwargs = cls._dense((args, kwargs or {}))
            return func(*dargs, **dkwargs)

    PackedWeight.__name__ = PackedWeight.__qualname__ = name
    return PackedWeight


def _w4a16_expert_cls():
    """Tensor subclass ``(packed u8 [N, K_pad/2], scale, zero, group, in_features)`` of one
    expert's int4 weight: ``F.linear`` runs the HIP fused op. None when libimq is unavailable."""
    def make():
        op = _w4a16_hip_op()
        if op is None:
            return None
        return _make_packed_weight_cls(
            "_W4A16Weight",
            layout=lambda q, s, z, g, k: ((q.shape[0], k), s.dtype, q.device),
            kernel=lambda x, p: op(x.reshape(-1, x.shape[-1]), p[0], p[3], (p[1], p[2])),
            materialize=lambda p: _dequant_g(p[0], p[1], p[2], p[4], p[3], p[1].dtype, 4),
            accepts=lambda x: True)
    return _lazy_class("_W4A16Weight", make)


def _w8a16_expert_cls():
    """Tensor subclass ``(packed int8 [N, K], scale [N, 1])`` of one expert's int8 weight:
    ``F.linear`` of a bf16 activation runs the HIP w8a16 op (the dense int8 path's dtype gate,
    worker_quant.py:2770-2774); any other use materializes ``q.to(scale.dtype) * scale``."""
    def make():
        import torch
        op = _w8a16_hip_op()
        if op is None:
            return None
        return _make_packed_weight_cls(
            "_W8A16Weight",
            layout=lambda q, s: (tuple(q.shape), s.dtype, q.device),
            kernel=lambda x, p: op(x.reshape(-1, x.shape[-1]), p[0], p[1]),
            materialize=lambda p: (p[0].to(p[1].dtype) * p[1]).contiguous(),
            accepts=lambda x: getattr(x, "dtype", None) is torch.bfloat16)
    return _lazy_class("_W8A16Weight", make)


def _expert_kernel_check(holder, weight_cls, make_weight, tag: str) -> bool:
    """One-time check of a holder's packed-weight subclass on expert 0 against the dequant it
    replaces, at M 1 and 8 (mean rel < 0.05)."""
    import torch.nn.functional as F
    if weight_cls is None:
        return False
    w0 = make_weight(0)
    dense = w0._materialize()
    for m in (1, 8):
        x = _bf16_rows(m, holder.in_features, holder.qweight.device)
        rel, _ = _rel_err(F.linear(x, w0), F.linear(x, dense))
        if not rel < _LINEAR_CHECK_REL:
            _log(f"[{tag}] expert kernel self-check rel={rel:.3f} at M={m} -> dequantized experts")
            return False
    return True


# ---- fused 3D int4 experts (worker_quant.py:1967-2125) ---------------------------------------
def _make_packed4_3d_cls():
    import torch
    from torch import nn

    class Packed4Tensor3D(nn.Module):
        _pad_choice: dict = {}     # (E, N, rs) -> padded rows win, one measurement per shape

        def __init__(self, qweight, scale, zero, in_features, group_size):
            super().__init__()
            self.register_buffer("qweight", qweight)   # uint8 [E, out, in_pad//2]
            self.register_buffer("scale", scale)        # [E, out, ng]
            self.register_buffer("zero", zero)          # [E, out, ng]
            self.in_features = in_features
            self.group_size = group_size
            self._expert_kernel = None                  # None: not decided yet

        def _expert_weight(self, e: int):
            return _w4a16_expert_cls()(self.qweight[e], self.scale[e], self.zero[e], self.group_size,
                                       self.in_features)

        def _expert_dense(self, e: int):
            return _dequant_g(self.qweight[e], self.scale[e], self.zero[e], self.in_features, self.group_size,
                              self.scale.dtype, 4)

        def __getitem__(self, e):
            """Expert e's weight for ``F.linear(bf16_x, w)``: the fused-op subclass on a ROCm
            device once it self-checks, else the dequant in the scale dtype."""
            e = int(e)
            if self._expert_kernel is None:
                self._expert_kernel = False
                with contextlib.suppress(Exception):
                    if _is_rocm_device(self.qweight.device):
                        self._expert_kernel = _expert_kernel_check(self, _w4a16_expert_cls(), self._expert_weight,
                                                                   "int4")
            return self._expert_weight(e) if self._expert_kernel else self._expert_dense(e)

        def _kernel_tensors(self):
            """(qweight, scale, zero) in the fused kernels' layout: K padded to a multiple of
            256 with zero codes and zero scales, so every row is whole 128-byte lines and an
            even number of groups (gpt-oss-20b's 2880 columns pad to 3072). The module's own
            buffers become views of the padded storage -- same shapes and values, no second
            copy. Idempotent; call on the final device."""
            qw, sc, ze = self.qweight, self.scale, self.zero
            kt = self.__dict__.get("_kt")
            if kt is not None and kt[3] is qw:
                return kt[:3]
            E, N, rs = qw.shape
            G = int(self.group_size)
            ng = int(sc.shape[2])
            kpad = rs * 2
            if (kpad % 256 == 0 and (ng * sc.element_size()) % 4 == 0) or 256 % G != 0:
                kt = (qw, sc, ze, qw)
            else:
                k2 = -(-kpad // 256) * 256
                q2 = torch.zeros((E, N, k2 // 2), dtype=torch.uint8, device=qw.device)
                q2[:, :, :rs].copy_(qw)
                s2 = torch.zeros((E, N, k2 // G), dtype=sc.dtype, device=sc.device)
                s2[:, :, :ng].copy_(sc)
                z2 = torch.zeros((E, N, k2 // G), dtype=ze.dtype, device=ze.device)
                z2[:, :, :ng].copy_(ze)
                self.qweight, self.scale, self.zero = q2[:, :, :rs], s2[:, :, :ng], z2[:, :, :ng]
                kt = (q2, s2, z2, self.qweight)
            self._kt = kt
            return kt[:3]

        def _decode_ms(self, op, q, sc, ze, reps: int = 25) -> float:
            """Device time of the per-row expert op at a decode shape (8 routed rows over fresh
            random experts per call), in ms."""
            E = q.shape[0]
            B = min(8, E)
            x = _bf16_rows(B, self.in_features, q.device, 0.1)
            picks = [torch.randperm(E, device=q.device)[:B].to(torch.int32) for _ in range(reps + 3)]
            it = iter(picks)
            return _device_ms(lambda: op(x, next(it), q, sc, ze, self.group_size, self.in_features), q.device,
                              iters=reps, warmup=3)

        def prepare_fused(self):
            """Kernel layout (``_kernel_tensors``), then the measured expert-row de-alias: keep
            ``[E, N, rs+64]`` padded rows only when they run the per-row op >= 13% faster
            (worker_quant.py:2045-2122); one measurement per (E, N, rs). Idempotent; never
            raises."""
            if getattr(self, "_dealiased", False):
                return
            self._dealiased = True
            qw = self.qweight
            if qw is None or qw.dim() != 3 or not _is_rocm_device(qw.device):
                return
            try:
                kq, ks, kz = self._kernel_tensors()
                E, N, rs = kq.shape
                op = _w4a16_moe_hip_op()
                if op is None or rs % 128 != 0 or kq.stride(2) != 1 or kq.stride(1) != rs:
                    return

                def padded():
                    buf = torch.zeros((E, N, rs + 64), dtype=torch.uint8, device=kq.device)
                    buf[:, :, :rs].copy_(kq)
                    return buf

                key = (E, N, rs)
                buf = None
                if key not in Packed4Tensor3D._pad_choice:
                    buf = padded()
                    t_flat = self._decode_ms(op, kq, ks, kz)
                    t_pad = self._decode_ms(op, buf[:, :, :rs], ks, kz)
                    Packed4Tensor3D._pad_choice[key] = t_pad < _NAIVE_MARGIN * t_flat
                    _log(f"[int4] moe row de-alias E={E} N={N} rs={rs}: {t_flat:.3f} ms -> padded {t_pad:.3f} ms "
                         f"({'padded' if Packed4Tensor3D._pad_choice[key] else 'kept'})")
                if Packed4Tensor3D._pad_choice[key]:
                    buf = buf if buf is not None else padded()
                    self.qweight = buf[:, :, :self.qweight.shape[2]]
                    self._kt = (buf[:, :, :rs], ks, kz, self.qweight)
            except Exception as exc:
                _log(f"[int4] moe kernel layout / de-alias skipped ({exc!r})")

    return Packed4Tensor3D


def _packed4_3d_cls():
    """Packed4Tensor3D(qweight u8[E,N,K_pad/2], scale[E,N,ng], zero[E,N,ng], in_features,
    group_size)."""
    return _lazy_class("Packed4Tensor3D", _make_packed4_3d_cls)


# ---- fused MoE experts forward (worker_quant.py:2131-2248) -----------------------------------
def _moe_fused_compute(experts_mod, hidden_states, top_k_index, top_k_weights):
    """All routed experts of one layer in one libimq call: the decode line kernels, token-sorted
    line kernels or grouped expert GEMMs for gate_up and down, SwiGLU between them, and the
    weighted combine into ``[T, H]``."""
    from . import ops
    gu, dn = experts_mod.gate_up_proj, experts_mod.down_proj
    # no host-side id check: the router's top-k ids lie in [0, E) by construction, the reference's
    # fused compute (worker_quant.py:2167-2191) checks none, and the kernels clamp any id outside
    # [0, E) to expert 0, so the layer never waits on a device-to-host read
    out = ops.moe_experts_w4(hidden_states, top_k_index, top_k_weights,
                             (*gu._kernel_tensors(), int(gu.in_features)),
                             (*dn._kernel_tensors(), int(dn.in_features)), int(gu.group_size),
                             check_ids=False)
    return out.to(hidden_states.dtype)


def _act_is_silu(act) -> bool:
    import torch
    if isinstance(act, torch.nn.SiLU):
        return True
    name = getattr(act, "__name__", "") or type(act).__name__
    return name.lower() in ("silu", "siluactivation", "silu_")


@contextlib.contextmanager
def _dense_experts(*holders):
    """Within the block the holders hand out dequantized experts (the reference's eager math)."""
    saved = [h._expert_kernel for h in holders]
    for h in holders:
        h._expert_kernel = False
    try:
        yield
    finally:
        for h, s in zip(holders, saved):
            h._expert_kernel = s


def _fused_moe_selfcheck(experts_mod, eager_forward) -> bool:
    """Fused experts forward against the module's original eager forward over dequantized experts,
    on random routings at T = 2 and 1 (8 of E experts, bf16 weights in [0.1, 1.1)); accepted when
    the mean rel < 0.03 and max rel < 0.1 (worker_quant.py:2193-2231)."""
    import torch
    gu, dn = experts_mod.gate_up_proj, experts_mod.down_proj
    dev = gu.qweight.device
    if not _is_rocm_device(dev):
        return False
    E, H = int(gu.qweight.shape[0]), int(gu.in_features)
    k = min(8, E)
    mean_worst = max_worst = 0.0
    for T in (2, 1):
        x = _bf16_rows(T, H, dev, 0.1)
        idx = torch.stack([torch.randperm(E, device=dev)[:k] for _ in range(T)])
        wts = torch.rand(T, k, device=dev, dtype=torch.bfloat16) + 0.1
        with _dense_experts(gu, dn):
            ref = eager_forward(x, idx, wts)
        mean_rel, max_rel = _rel_err(_moe_fused_compute(experts_mod, x, idx, wts), ref)
        mean_worst, max_worst = max(mean_worst, mean_rel), max(max_worst, max_rel)
    ok = mean_worst < _MOE_CHECK_MEAN and max_worst < _MOE_CHECK_MAX
    _log(f"[int4] fused-MoE self-check mean rel {mean_worst:.4f}, max rel {max_worst:.4f} -> "
         f"{'fused' if ok else 'eager per-expert loop'}")
    return ok


def _install_fused_moe_forward(experts_mod) -> None:
    """Patch a fused-3D int4 experts module (``gate_up_proj``/``down_proj`` Packed4Tensor3D +
    SiLU ``act_fn``) so token counts up to ``_FUSED_MOE_T_MAX`` run the fused HIP path, gated once
    by ``_fused_moe_selfcheck``; any exception falls back to the original forward.
    INFINITEMODEL_NO_FUSED_MOE disables it."""
    import types
    if os.environ.get("INFINITEMODEL_NO_FUSED_MOE") or getattr(experts_mod, "_fused_moe_installed", False):
        return
    PT = _packed4_3d_cls()
    holders = (getattr(experts_mod, "gate_up_proj", None), getattr(experts_mod, "down_proj", None))
    if not all(isinstance(h, PT) for h in holders) or not hasattr(experts_mod, "act_fn"):
        return
    if not _act_is_silu(experts_mod.act_fn) or _w4a16_moe_hip_op() is None:
        return                      # the fused kernels implement SiLU-GLU only
    eager_forward = experts_mod.forward

    def forward(self, hidden_states, top_k_index, top_k_weights):
        if hidden_states.shape[0] <= _FUSED_MOE_T_MAX:
            if self._fused_moe_ok is None:
                try:
                    self._fused_moe_ok = _fused_moe_selfcheck(self, eager_forward)
                except Exception as exc:
                    _log(f"[int4] fused-MoE self-check failed ({exc!r}) -> eager per-expert loop")
                    self._fused_moe_ok = False
            if self._fused_moe_ok:
                with contextlib.suppress(Exception):
                    return _moe_fused_compute(self, hidden_states, top_k_index, top_k_weights)
        return eager_forward(hidden_states, top_k_index, top_k_weights)

    experts_mod._fused_moe_ok = None
    experts_mod._fused_moe_installed = True
    experts_mod.forward = types.MethodType(forward, experts_mod)


# ---- gpt-oss fused experts (worker_quant.py:2250-2314) ---------------------------------------
def _is_gptoss_experts(module) -> bool:
    """A gpt-oss fused-expert block: interleaved clamped SwiGLU with per-expert biases
    (worker_quant.py:2257-2262)."""
    if type(module).__name__ == "GptOssExperts":
        return True
    return all(hasattr(module, a) for a in ("gate_up_proj_bias", "down_proj_bias", "alpha", "limit"))


def _gptoss_fused_ok() -> bool:
    """gpt-oss int4 needs the fused MoE kernel: its experts are transpose-packed, so there is no
    eager host path to fall back to (worker_quant.py:2265-2276). True when libimq loads, unless
    INFINITEMODEL_NO_FUSED_MOE is set."""
    return not os.environ.get("INFINITEMODEL_NO_FUSED_MOE") and _w4a16_moe_hip_op() is not None


def _gptoss_fused_compute(experts_mod, hidden_states, router_indices, routing_weights):
    """gpt-oss experts forward in one libimq call: transpose-packed gate_up (interleaved gate /
    up rows) + bias, clamped GLU, down + bias, routing-weighted combine."""
    from . import ops
    gu, dn = experts_mod.gate_up_proj, experts_mod.down_proj
    out = ops.moe_experts_w4(hidden_states, router_indices, routing_weights,
                             (*gu._kernel_tensors(), int(gu.in_features)),
                             (*dn._kernel_tensors(), int(dn.in_features)), int(gu.group_size),
                             act="gptoss", gu_bias=experts_mod.gate_up_proj_bias,
                             dn_bias=experts_mod.down_proj_bias,
                             alpha=float(getattr(experts_mod, "alpha", 1.702)),
                             limit=float(getattr(experts_mod, "limit", 7.0)), check_ids=False)
    return out.to(hidden_states.dtype)


def _install_gptoss_fused_forward(experts_mod) -> None:
    """Install gpt-oss's int4 fused-expert forward (worker_quant.py:2280-2314) for every token
    count: once the experts are transpose-packed there is no eager fallback. The caller has
    transpose-packed the experts and checked ``_gptoss_fused_ok()``."""
    import types

    def forward(self, hidden_states, router_indices=None, routing_weights=None):
        return _gptoss_fused_compute(self, hidden_states, router_indices, routing_weights)

    experts_mod._gptoss_fused_installed = True
    experts_mod.forward = types.MethodType(forward, experts_mod)
    _log("[int4] gpt-oss fused experts active (transpose-packed w4a16 + interleaved SwiGLU)")


# ---- int8 fused 3D experts (worker_quant.py:2707-2990) ---------------------------------------
def _w8a16_experts_ok(dev) -> bool:
    """Should Packed8Tensor3D hand the eager MoE loop the w8a16 expert subclass instead of a
    dequantized weight (worker_quant.py:2711-2731)? On a ROCm device unless IM_W8A16_EXPERTS=0 or
    IM_FUSED_W8A16=0; never on the CPU."""
    if os.environ.get("IM_W8A16_EXPERTS", "") == "0" or not _FUSED_W8A16:
        return False
    return _is_rocm_device(dev)


def _make_packed8_3d_cls():
    import torch
    from torch import nn

    class Packed8Tensor3D(nn.Module):
        def __init__(self, qweight, scale, in_features):
            super().__init__()
            self.register_buffer("qweight", qweight)   # int8 [E, out, in]
            self.register_buffer("scale", scale)        # [E, out, 1]
            self.in_features = in_features
            self._expert_kernel = None

        def _expert_weight(self, e: int):
            return _w8a16_expert_cls()(self.qweight[e], self.scale[e])

        def __getitem__(self, e):
            """Expert e's weight for ``F.linear(bf16_x, w)``: the w8a16 subclass on a ROCm device
            with a bf16 scale once it self-checks, else ``q.to(scale.dtype) * scale``."""
            e = int(e)
            if self._expert_kernel is None:
                self._expert_kernel = False
                with contextlib.suppress(Exception):
                    if _w8a16_experts_ok(self.qweight.device) and self.scale.dtype is torch.bfloat16:
                        self._expert_kernel = _expert_kernel_check(self, _w8a16_expert_cls(), self._expert_weight,
                                                                   "int8")
            if self._expert_kernel:
                return self._expert_weight(e)
            return (self.qweight[e].to(self.scale.dtype) * self.scale[e]).contiguous()

    return Packed8Tensor3D


def _packed8_3d_cls():
    """Packed8Tensor3D(qweight int8 [E, out, in], scale [E, out, 1], in_features)
    (worker_quant.py:2813-2897): all of one projection's experts at int8 behind the eager
    experts loop's ``self.gate_up_proj[e]`` indexing."""
    return _lazy_class("Packed8Tensor3D", _make_packed8_3d_cls)


def _pack8_3d(W3):
    """Fused expert tensor [E, out, in] -> Packed8Tensor3D through the 2D int8 packer per expert
    (worker_quant.py:2900-2921): per-row scales never cross an expert."""
    import torch
    E, out, in_f = W3.shape
    q = torch.empty((E, out, in_f), dtype=torch.int8, device=W3.device)
    sc = torch.empty((E, out, 1), dtype=W3.dtype, device=W3.device)
    for e in range(E):
        q[e], sc[e] = _pack8_expert(W3[e])
    return _packed8_3d_cls()(q, sc, in_f)


def apply_head_quant(model, head, head_quant: str, head_device=None):
    """The ``head_quant`` load option (client.py:799-840): ``"int8"`` packs a GPU-resident
    ``nn.Linear`` lm_head to an int8 QuantLinear (kept bf16 on the CPU, when tied to the
    embedding, or when the load tier already packed it); ``"bf16"`` keeps the head. Returns the
    head to use (also set as ``model.lm_head`` when replaced). Any failure keeps the head as built."""
    import torch
    hq = (head_quant or "").strip().lower()
    if not hq or head is None:
        return head
    try:
        if hq not in ("int8", "bf16"):
            raise ValueError(f"head_quant={hq!r} unsupported (int8 | bf16); int4 on the lm_head was "
                             "measured and rejected")
        dev = torch.device(head_device if head_device is not None else next(head.parameters()).device)
        is_linear = isinstance(head, torch.nn.Linear)
        tied = bool(getattr(getattr(model, "config", None), "tie_word_embeddings", False))
        if hq == "bf16":
            if not is_linear:
                _log("[head-quant] bf16 head requested but the load tier already quantized the head -- "
                     "leaving it")
            return head
        skip = ("the lm_head is on {} and the w8a16 kernel is GPU-only -- bf16 is faster there".format(dev)
                if dev.type != "cuda" else
                f"already packed by the load tier ({type(head).__name__})" if not is_linear else
                "tie_word_embeddings: lm_head aliases embed_tokens, so packing it adds a copy" if tied else None)
        if skip is not None:
            _log(f"[head-quant] int8 head skipped: {skip}")
            return head
        bf16_bytes = head.weight.numel() * head.weight.element_size()
        packed = _quantize_linear(head.to("cpu")).to(dev)
        if hasattr(model, "lm_head"):
            model.lm_head = packed
        pk = packed.qweight.numel() + packed.scale.numel() * packed.scale.element_size()
        _log(f"[head-quant] lm_head int8: {bf16_bytes / 2**30:.2f} GB bf16 -> {pk / 2**30:.2f} GB "
             f"({bf16_bytes / max(1, pk):.1f}x fewer bytes read per decoded token)")
        return packed
    except Exception as exc:
        _log(f"[head-quant] failed ({exc!r}) -> leaving the lm_head as built")
        return head


# ---- packers (worker_quant.py:511-536, 1588-1608, 1921-1944, 2394-2436) ---------------------
def _pack8_expert(W2d):
    """Per-row symmetric int8 of one ``[out, in]`` weight in W's own dtype -> (int8, scale)."""
    return _sc.pack_linear_int8(W2d)


def _quantize_linear(lin):
    """nn.Linear -> QuantLinear (int8 per-row)."""
    qW, scale = _pack8_expert(lin.weight.data)
    return _quant_linear_cls()(qW, scale, lin.bias)


def _quantize_linear4(lin, group_size: int = _INT4_GROUP):
    """nn.Linear -> QuantLinear4 (RTN asymmetric int4, 2 codes per byte)."""
    q, s, z, in_f = _sc.pack_linear_int4(lin.weight.data, group_size)
    return _quant4_linear_cls()(q, s, z, lin.bias, in_f, group_size)


def _quantize_linear2(lin, group_size: int = _INT2_GROUP):
    """nn.Linear -> QuantLinear2 (RTN asymmetric int2, 4 codes per byte)."""
    q, s, z, in_f = _sc.pack_linear_int2(lin.weight.data, group_size)
    return _quant2_linear_cls()(q, s, z, lin.bias, in_f, group_size)


def _pack4_expert(We, ng: int, G: int, in_pad: int, in_f: int, dt):
    """One expert ``[out, in]`` -> (qpacked [out, in_pad/2], scale [out, ng], zero [out, ng])."""
    q, s, z, _ = _sc.pack_linear_int4(We, G)
    if q.shape[1] * 2 != in_pad or s.shape[1] != ng:
        raise ValueError("expert shape does not match (ng, in_pad)")
    return q, s.to(dt), z.to(dt)


def _pack4_3d(W3, group_size: int = _INT4_GROUP):
    """Fused expert tensor ``[E, out, in]`` -> Packed4Tensor3D, one expert at a time."""
    q, s, z, in_f, _ng = _sc.pack_linear_int4_3d(W3, group_size)
    return _packed4_3d_cls()(q, s, z, in_f, group_size)


# ---- scope walkers ---------------------------------------------------------------------------
def _is_router_scope(module) -> bool:
    return type(module).__name__.endswith(("Router", "Gate"))


def _linear_targets(module):
    """(parent, attribute, nn.Linear) of every Linear under ``module`` that the quantizers replace:
    all but MoE routers -- a leaf named gate / router / wg, or anything inside a module whose
    class name ends in Router / Gate (worker_quant.py:539-575, 3051)."""
    from torch import nn
    found, stack = [], [module]
    while stack:
        parent = stack.pop()
        for name, child in parent.named_children():
            if isinstance(child, nn.Linear):
                if name not in _ROUTER_LEAF_NAMES:
                    found.append((parent, name, child))
            elif not _is_router_scope(child):
                stack.append(child)
    return found


def _quantize_linears_(module, convert) -> None:
    """Replace every quantizable nn.Linear under ``module`` with ``convert(lin)``."""
    for parent, name, lin in _linear_targets(module):
        setattr(parent, name, convert(lin))


def _quantize_int4_(module) -> None:
    _quantize_linears_(module, _quantize_linear4)


def _quantize_int2_(module) -> None:
    _quantize_linears_(module, _quantize_linear2)


def _quantize_int8_linears_(module) -> None:
    _quantize_linears_(module, _quantize_linear)


def _expert_params(module, meta=None):
    """(block, attribute, 3D Parameter, is_gptoss) of every fused ``gate_up_proj`` / ``down_proj``
    expert tensor under ``module``; ``meta`` True / False keeps only meta / materialized ones."""
    from torch import nn
    out = []
    for block in module.modules():
        gptoss = _is_gptoss_experts(block)
        for attr in ("gate_up_proj", "down_proj"):
            p = block._parameters.get(attr)
            if isinstance(p, nn.Parameter) and p.dim() == 3 and (meta is None or bool(p.is_meta) == meta):
                out.append((block, attr, p, gptoss))
    return out


def _finish_expert_blocks(blocks, install: bool) -> None:
    """After packing: force the eager experts implementation on every non-gpt-oss block's config
    (the packed holders serve it) and, with ``install``, put the fused forwards on."""
    configs = set()
    for block, gptoss in blocks.values():
        cfg = getattr(block, "config", None)
        if not gptoss and cfg is not None and hasattr(cfg, "_experts_implementation") and id(cfg) not in configs:
            cfg._experts_implementation = "eager"
            configs.add(id(cfg))
    if install:
        for block, gptoss in blocks.values():
            (_install_gptoss_fused_forward if gptoss else _install_fused_moe_forward)(block)


def _require_gptoss_kernel(targets) -> None:
    if any(t[3] for t in targets) and not _gptoss_fused_ok():
        raise RuntimeError("gpt-oss int4 requires the fused w4a16 MoE kernel (libimq on a ROCm "
                           "device) -- load gpt-oss at quant=none (bf16) here")


def _quantize_experts4_(module) -> None:
    """Replace 3D ``gate_up_proj``/``down_proj`` expert Parameters with Packed4Tensor3D
    (worker_quant.py:2439-2483). gpt-oss blocks store their experts in-major [E, in, out] and are
    transposed to [E, out, in] before packing; they get the dedicated fused forward (and need it:
    RuntimeError when it is unavailable). Every other block gets the eager experts implementation
    on its config and the fused-MoE forward."""
    targets = _expert_params(module)
    _require_gptoss_kernel(targets)
    blocks = {}
    for block, attr, p, gptoss in targets:
        w = p.data.transpose(1, 2).contiguous() if gptoss else p.data
        delattr(block, attr)
        setattr(block, attr, _pack4_3d(w))
        blocks[id(block)] = (block, gptoss)
    _finish_expert_blocks(blocks, install=True)


def _quantize_experts8_(module) -> None:
    """int8 twin of ``_quantize_experts4_`` (worker_quant.py:2924-2987): 3D ``gate_up_proj`` /
    ``down_proj`` Parameters -> Packed8Tensor3D and the eager experts implementation. Refuses
    gpt-oss (no int8 form of its transpose-packed fused forward) and meta experts (streaming is
    int4-only). No fused-MoE forward is installed: int8 experts run the eager loop, each routed
    expert through the w8a16 subclass."""
    targets = _expert_params(module)
    if any(t[3] for t in targets):
        raise RuntimeError("gpt-oss fused experts have no int8 path (in-major transpose-packed "
                           "weights need the fused w4a16 MoE forward) -- load gpt-oss at int4")
    meta = [f"{type(b).__name__}.{a}" for b, a, p, _ in targets if p.is_meta]
    if meta:
        raise RuntimeError(f"int8 MoE: {', '.join(meta)} still META -- per-expert expert streaming "
                           "is int4-only; load this model at int4")
    blocks = {}
    for block, attr, p, _gptoss in targets:
        delattr(block, attr)
        setattr(block, attr, _pack8_3d(p.data))
        blocks[id(block)] = (block, False)
    _finish_expert_blocks(blocks, install=False)


def _quantize_int8_(module) -> None:
    """int8 a decoder layer (worker_quant.py:578-596): every nn.Linear except routers, then the
    fused 3D routed experts."""
    _quantize_int8_linears_(module)
    _quantize_experts8_(module)


# ---- streamed expert builds (worker_quant.py:2486-2700) --------------------------------------
# A layer whose experts were left META by the loader is built expert by expert: the caller's
# ``fetch_experts(layer_idx, e0, k)`` returns experts e0 .. e0+k-1 either fused
# ({'gate_up_proj': [k, out, in], 'down_proj': [k, out, in]}) or per expert
# ({'<local e>.<proj>': [out, in]}, gate w1 / gate_proj, up w3 / up_proj, down w2 / down_proj),
# and each expert is int4-packed into its slot as it arrives, so at most one chunk of bf16 experts
# is ever resident.
_GATE_NAMES, _UP_NAMES, _DOWN_NAMES = ("w1", "gate_proj"), ("w3", "up_proj"), ("w2", "down_proj")


def _chunk_experts(per_expert_bytes: int) -> int:
    """Experts per fetch: as many as fit the chunk byte budget, 1 .. 64."""
    return max(1, min(_STREAM_CHUNK_MAX, _STREAM_CHUNK_BYTES // max(1, per_expert_bytes)))


def _oriented(w, rows: int, cols: int, force_t: bool = False):
    """``w`` as ``[rows, cols]``: transposed when ``force_t`` (in-major gpt-oss experts) or when
    only its transpose has that shape."""
    if force_t or (tuple(w.shape) != (rows, cols) and tuple(w.shape) == (cols, rows)):
        w = w.t()
    return w.contiguous()


def _per_expert_blob(blob, layer_idx: int) -> dict:
    """{local expert: {proj: tensor}} of a per-expert blob; a key without '<e>.' is a layout
    mismatch between the server and this worker."""
    grouped: dict = {}
    for key, t in blob.items():
        e_s, dot, proj = key.partition(".")
        if not dot or not e_s.isdigit():
            raise RuntimeError(f"L{layer_idx}: expert blob key {key!r} is not '<expert>.<proj>' -- "
                               "server and worker disagree on the expert layout")
        grouped.setdefault(int(e_s), {})[proj] = t
    return grouped


def _first_of(projs: dict, names):
    return next((projs[n] for n in names if n in projs), None)


class _StreamSlot:
    """Packed storage of one streamed fused expert tensor, filled expert by expert."""

    def __init__(self, block, attr, p, gptoss: bool, dt):
        import torch
        E, d1, d2 = (int(v) for v in p.shape)
        self.block, self.attr, self.gptoss, self.dt = block, attr, gptoss, dt
        self.E = E
        self.out, self.in_f = (d2, d1) if gptoss else (d1, d2)
        self.ng = -(-self.in_f // _INT4_GROUP)
        self.in_pad = self.ng * _INT4_GROUP
        self.q = torch.empty((E, self.out, self.in_pad // 2), dtype=torch.uint8)
        self.s = torch.empty((E, self.out, self.ng), dtype=dt)
        self.z = torch.empty((E, self.out, self.ng), dtype=dt)

    def put(self, e: int, w, in_major: bool = False) -> None:
        w = _oriented(w, self.out, self.in_f, force_t=in_major)
        self.q[e], self.s[e], self.z[e] = _pack4_expert(w.to(self.dt), self.ng, _INT4_GROUP, self.in_pad, self.in_f,
                                                        self.dt)

    def holder(self):
        return _packed4_3d_cls()(self.q, self.s, self.z, self.in_f, _INT4_GROUP)


def _quantize_experts4_streamed(module, layer_idx: int, fetch_experts, dt) -> None:
    """Build a layer's META fused 3D experts from ``fetch_experts`` (see above) into
    Packed4Tensor3D holders, then install the fused forwards as ``_quantize_experts4_`` does.
    Fused gpt-oss slices are in-major [k, in, out] and are transposed before packing."""
    import torch
    targets = _expert_params(module)
    if not targets:
        return
    _require_gptoss_kernel(targets)
    slots = {attr: _StreamSlot(block, attr, p, gptoss, dt) for block, attr, p, gptoss in targets}
    E = next(iter(slots.values())).E
    gu = slots.get("gate_up_proj")
    chunk = _chunk_experts(gu.out * gu.in_f * 2 if gu is not None else 1)
    for e0 in range(0, E, chunk):
        k = min(chunk, E - e0)
        blob = fetch_experts(layer_idx, e0, k)
        if "gate_up_proj" in blob and "down_proj" in blob:          # fused slices [k, out, in]
            for attr, slot in slots.items():
                for j in range(blob[attr].shape[0]):
                    slot.put(e0 + j, blob[attr][j], in_major=slot.gptoss)
            continue
        grouped = _per_expert_blob(blob, layer_idx)
        for j in range(k):
            projs = grouped.get(j, {})
            if "gate_up_proj" in slots:
                gate, up = _first_of(projs, _GATE_NAMES), _first_of(projs, _UP_NAMES)
                if gate is None or up is None:
                    raise RuntimeError(f"L{layer_idx} expert {e0 + j}: no gate / up among {sorted(projs)}")
                slot = slots["gate_up_proj"]
                both = (gate, up) if gate.shape[1] == slot.in_f else (gate.t(), up.t())
                slot.put(e0 + j, torch.cat(both, dim=0))        # [gate | up] rows
            if "down_proj" in slots:
                down = _first_of(projs, _DOWN_NAMES)
                if down is None:
                    raise RuntimeError(f"L{layer_idx} expert {e0 + j}: no down among {sorted(projs)}")
                slots["down_proj"].put(e0 + j, down)
        del blob, grouped
    blocks = {}
    for attr, slot in slots.items():
        delattr(slot.block, attr)
        setattr(slot.block, attr, slot.holder())
        blocks[id(slot.block)] = (slot.block, slot.gptoss)
    _finish_expert_blocks(blocks, install=True)
    _log(f"[load] L{layer_idx}: {E} experts built from the stream (int4, {chunk} per fetch)")


def _nonfused_expert_lists(module):
    """Every ``experts`` nn.ModuleList under ``module`` whose experts hold nn.Linear children."""
    from torch import nn
    lists = []
    for sub in module.modules():
        ex = getattr(sub, "experts", None)
        if isinstance(ex, nn.ModuleList) and len(ex) and any(isinstance(m, nn.Linear) for m in ex[0].modules()):
            lists.append(ex)
    return lists


def _quantize_experts4_streamed_nonfused(module, layer_idx: int, fetch_experts, dt) -> None:
    """Build a layer's META per-expert Linears (``experts[e].<proj>``, e.g. w1 / w3 / w2) from
    ``fetch_experts`` into QuantLinear4 modules in place -- the same holders the in-memory int4
    walker makes, so the result equals a full load. Runs before ``_quantize_int4_`` walks the layer."""
    from torch import nn
    QL = _quant4_linear_cls()
    for experts in _nonfused_expert_lists(module):
        projs = [n for n, ch in experts[0].named_children() if isinstance(ch, nn.Linear)]
        if not projs:
            continue
        per_expert = sum(int(getattr(experts[0], n).weight.numel()) * 2 for n in projs)
        chunk = _chunk_experts(per_expert)
        for e0 in range(0, len(experts), chunk):
            k = min(chunk, len(experts) - e0)
            for j, tensors in _per_expert_blob(fetch_experts(layer_idx, e0, k), layer_idx).items():
                if e0 + j >= len(experts):
                    continue
                expert = experts[e0 + j]
                for proj, w in tensors.items():
                    lin = getattr(expert, proj, None)
                    if not isinstance(lin, nn.Linear):
                        continue
                    out, in_f = int(lin.weight.shape[0]), int(lin.weight.shape[1])
                    w = _oriented(w, out, in_f)
                    ng = -(-in_f // _INT4_GROUP)
                    q, s, z = _pack4_expert(w.to(dt), ng, _INT4_GROUP, ng * _INT4_GROUP, in_f, dt)
                    setattr(expert, proj, QL(q, s, z, lin.bias, in_f, _INT4_GROUP))
        _log(f"[load] L{layer_idx}: {len(experts)} per-expert Linears ({'/'.join(projs)}) built from the "
             f"stream (int4, {chunk} per fetch)")


# ---- MoE layer structure helpers (worker_quant.py:2316-2392, 2983-3140) -----------------------
def _holds_fused_experts(module) -> bool:
    """True if ``module`` or a descendant carries fused 3D experts (a packed holder or a 3D
    gate_up_proj / down_proj tensor)."""
    holders = (_packed4_3d_cls(), _packed8_3d_cls())
    for sub in module.modules():
        for attr in ("gate_up_proj", "down_proj"):
            a = getattr(sub, attr, None)
            if isinstance(a, holders) or (a is not None and getattr(a, "dim", None) is not None and a.dim() == 3):
                return True
    return False


def _find_moe_block(layer):
    """(attribute, block) of the direct child of a decoder layer that holds its routed experts (an
    ``experts`` attribute, or fused 3D experts anywhere below it); (None, None) for a dense layer."""
    for name, child in layer.named_children():
        if getattr(child, "experts", None) is not None or _holds_fused_experts(child):
            return name, child
    return None, None


def _model_has_fused_experts(model) -> bool:
    """True if the model stores fused 3D expert Parameters (the streamed fused build's layout)."""
    return bool(_expert_params(model))


def _model_has_nonfused_experts(model) -> bool:
    """True if the model stores its experts as ``experts`` ModuleLists of Linears."""
    return bool(_nonfused_expert_lists(model))


def _layer_has_meta_experts(lyr) -> bool:
    """True if the layer's fused 3D experts are still META (to be built from the stream)."""
    return bool(_expert_params(lyr, meta=True))


def _layer_has_meta_experts_nonfused(lyr) -> bool:
    """True if a per-expert ``experts`` ModuleList of the layer still has META Linear weights."""
    from torch import nn
    return any(isinstance(m, nn.Linear) and m.weight.is_meta
               for ex in _nonfused_expert_lists(lyr) for m in ex[0].modules())


def _make_moe_bridge_cls():
    import torch
    from torch import nn
    from torch.utils._pytree import tree_map

    class _MoEDeviceBridge(nn.Module):
        """Runs a wrapped MoE block on the device its weights live on (the CPU) inside a layer that
        runs on the GPU: tensor arguments go to the block's device, tensor results come back to
        the device of ``hidden_states``."""

        def __init__(self, block, cpu_dev):
            super().__init__()
            self.block = block
            self._cpu = cpu_dev

        def forward(self, hidden_states, *args, **kwargs):
            home = hidden_states.device
            there = lambda t: t.to(self._cpu) if torch.is_tensor(t) else t     # noqa: E731
            back = lambda t: t.to(home) if torch.is_tensor(t) else t           # noqa: E731
            out = self.block(there(hidden_states), *tree_map(there, args), **tree_map(there, kwargs))
            return tree_map(back, out)

    return _MoEDeviceBridge


def _moe_bridge_cls():
    """The module that keeps a layer's MoE block (router + experts) in CPU memory while the rest of
    the layer runs on the GPU (worker_quant.py:2316-2361)."""
    return _lazy_class("_MoEDeviceBridge", _make_moe_bridge_cls)


def _resolve(model, dotted: str):
    """(parent, leaf, current value or None) of a dotted state-dict name; (None, leaf, None)
    when the path does not exist in the module tree."""
    *path, leaf = dotted.split(".")
    node = model
    for part in path:
        try:
            node = node[int(part)] if part.isdigit() else getattr(node, part)
        except (AttributeError, IndexError, KeyError, TypeError):
            return None, leaf, None
    return node, leaf, getattr(node, leaf, None)


def _meta_sibling(model, dotted: str, t):
    """For a name that is not in the module tree: a still-meta tensor of the same leaf name and
    shape on a sibling module under the same grandparent (transformers moves some checkpoint
    tensors, e.g. a router bias, onto another child while building). (parent, leaf, tensor)."""
    parts = dotted.split(".")
    if len(parts) < 3:
        return None
    grand, _, _ = _resolve(model, ".".join(parts[:-1]))
    if grand is None:
        return None
    for child in grand.children():
        cur = getattr(child, parts[-1], None)
        if cur is not None and getattr(cur, "is_meta", False) and tuple(cur.shape) == tuple(t.shape):
            return child, parts[-1], cur
    return None


def _assign_meta_from_sd(model, sd) -> int:
    """Give every tensor of ``sd`` whose model attribute is still META its data (what
    ``load_state_dict(assign=True)`` leaves out: non-persistent buffers, and names transformers
    moved onto a sibling module). Parameters stay Parameters (no grad); buffers are registered
    non-persistent. Tensors absent from ``sd`` stay META. Returns the number assigned."""
    import torch
    n = 0
    for name, t in sd.items():
        parent, leaf, cur = _resolve(model, name)
        if cur is None:
            hit = _meta_sibling(model, name, t)
            if hit is None:
                continue
            parent, leaf, cur = hit
        if not getattr(cur, "is_meta", False):
            continue
        val = t.detach().to(cur.dtype).clone()
        if isinstance(cur, torch.nn.Parameter):
            setattr(parent, leaf, torch.nn.Parameter(val, requires_grad=False))
        else:
            parent.register_buffer(leaf, val, persistent=False)
        n += 1
    return n


# ---- CPU path (worker_quant.py:201-237, 283-380) ---------------------------------------------
def _cpu_bf16_gemm_ok() -> bool:
    """Whether this CPU's bf16 Linear can be trusted (probed once): a decode-shaped biased bf16
    linear must not raise, must not fall back with a oneDNN / bf16 warning, and must agree with
    the fp32 product (max rel <= 0.05)."""
    global _CPU_BF16_GEMM_OK
    if _CPU_BF16_GEMM_OK is not None:
        return _CPU_BF16_GEMM_OK
    ok = True
    try:
        import warnings
        import torch
        import torch.nn.functional as F
        g = torch.Generator().manual_seed(0)
        x, w, b = torch.randn(1, 512, generator=g), torch.randn(512, 512, generator=g), torch.randn(512, generator=g)
        want = F.linear(x, w, b)
        with warnings.catch_warnings(record=True) as caught:
            warnings.simplefilter("always")
            got = F.linear(x.bfloat16(), w.bfloat16(), b.bfloat16()).float()
        noisy = any(s in str(c.message).lower() for c in caught for s in ("mkldnn", "bf16"))
        err = (got - want).abs().max().item() / (want.abs().max().item() + 1e-6)
        ok = not noisy and bool(torch.isfinite(got).all()) and err <= 0.05
        _log(f"[cpu] bf16 GEMM probe: ok={ok} (warning={noisy}, max rel {err:.4f})")
    except Exception as exc:
        ok = False
        _log(f"[cpu] bf16 GEMM probe raised ({type(exc).__name__}) -> fp32 for every CPU matmul")
    _CPU_BF16_GEMM_OK = ok
    return ok


def _env_threads():
    for var in ("OMP_NUM_THREADS", "MKL_NUM_THREADS", "TORCH_NUM_THREADS"):
        v = (os.environ.get(var) or "").strip()
        if v.isdigit() and int(v) > 0:
            return int(v)
    return None


def _physical_cores() -> int:
    try:
        import psutil
        n = psutil.cpu_count(logical=False)
    except Exception:
        n = None
    return n or os.cpu_count() or 1


def tune_cpu_threads() -> None:
    """Set torch's CPU intra-op threads once per process (worker_quant.py:283-330): an explicit
    OMP_NUM_THREADS / MKL_NUM_THREADS / TORCH_NUM_THREADS wins, else the physical core count,
    clamped to 1 .. 128; inter-op threads min(2, n). On a CPU whose bf16 GEMM is unusable every
    CPU matmul is upcast to fp32 (``_CPU_FP32_MIN_ROWS`` 1). No-op without torch."""
    global _CPU_FP32_MIN_ROWS
    try:
        import torch
    except Exception:
        return
    env = _env_threads()
    n = max(1, min(128, env or _physical_cores()))
    with contextlib.suppress(Exception):
        torch.set_num_threads(n)
    with contextlib.suppress(Exception):
        torch.set_num_interop_threads(min(2, n))
    if _CPU_FP32_GEMM and not _cpu_bf16_gemm_ok():
        _CPU_FP32_MIN_ROWS = 1
    _log(f"[cpu] torch intra-op threads {torch.get_num_threads()} ({'environment' if env else 'physical cores'}); "
         f"fp32 CPU GEMM {'on from ' + str(_CPU_FP32_MIN_ROWS) + ' rows' if _CPU_FP32_GEMM else 'off'}")


def _accelerate_cpu_linears(module) -> None:
    """Route every CPU-resident plain nn.Linear under ``module`` through an fp32 GEMM for calls
    of at least ``_CPU_FP32_MIN_ROWS`` rows (worker_quant.py:333-380); GPU-resident Linears and
    the quantized modules (their own CPU rule) are left alone. Idempotent."""
    if module is None:
        return
    import torch.nn.functional as F
    from torch import nn
    for lin in module.modules():
        if not isinstance(lin, nn.Linear) or getattr(lin, "_im_fp32_wrapped", False):
            continue
        if getattr(lin.weight, "device", None) is None or lin.weight.device.type != "cpu":
            continue
        native = lin.forward

        def forward(x, lin=lin, native=native):
            if _cpu_fp32_worth(x) and lin.weight.device.type == "cpu":
                b = None if lin.bias is None else lin.bias.float()
                return F.linear(x.float(), lin.weight.float(), b).to(x.dtype)
            return native(x)

        lin.forward = forward
        lin._im_fp32_wrapped = True


# ---- placement sweep ------------------------------------------------------------------------
def finalize_placement(model) -> int:
    """Call ``prepare_fused`` on every submodule that has it (after the model reached its final
    device) and return how many ended with a bound fused op (client.py:852-864)."""
    bound = 0
    for sub in model.modules():
        if hasattr(sub, "prepare_fused"):
            sub.prepare_fused()
            bound += int(getattr(sub, "_fused", None) is not None or getattr(sub, "_w8", None) is not None)
    return bound
