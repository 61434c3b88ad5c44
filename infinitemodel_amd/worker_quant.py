"""Reference-compatible quantized Linear modules, backed by the gfx950 kernels of libimq.

This module keeps the plugin boundary of the reference's worker_quant.py so a caller switches by
import: the same lazy class factories, constructors, buffer names (``qweight``/``scale``/``zero``
are state_dict keys), attributes (``in_features``, ``group_size``, ``bias``, ``_fused``,
``_fused_tried``, ``_naive_m_min``), methods (``forward``, ``_dequant``, ``prepare_fused``), op
builders with the reference's call signatures, packers and scope walkers.

Device behaviour:

* ROCm device: every kernel is a hand-written HIP kernel of libimq. ``prepare_fused`` binds the
  fused op after a self-check (never raises; on failure the module keeps the naive path). The naive
  path is ``F.linear(x, _dequant(dtype))`` where ``_dequant`` is libimq's bit-exact dequant
  kernel, so a missing library raises ``ImqUnavailable`` from forward instead of silently running
  a torch substitute.
* CPU device: the reference's CPU semantics, in torch (dequant in ``dtype``; rows >= 16 take the
  fp32 dequant + fp32 GEMM of worker_quant.py:847-852).

Op builder names: the reference names its builders after Triton (``_w4a16_triton_op`` ...). Those
names are kept as aliases because other code reads them; the callables they return launch HIP
kernels (``_w4a16_hip_op`` ...). There is no Triton anywhere in this package.
"""
from __future__ import annotations

import contextlib
import os
import threading
import time

from . import shard_compile as _sc

# ---- flags (worker_quant.py:97-115; same environment switches) ------------------------------
_FUSED_INT4 = os.environ.get("IM_FUSED_INT4", "1") != "0"
_FUSED_W8A16 = os.environ.get("IM_FUSED_W8A16", "1") != "0"
_FUSED_INT2 = os.environ.get("IM_FUSED_INT2", "1") != "0"
_LARGE_M_NAIVE = os.environ.get("IM_LARGE_M_NAIVE", "1") != "0"

# CPU fp32-GEMM rule for CPU-resident modules (worker_quant.py:183-198).
_CPU_FP32_MIN_ROWS = 16
_CPU_FP32_GEMM = True

_INT4_GROUP = _sc.INT4_GROUP
_INT2_GROUP = _sc.INT2_GROUP
_W8_PROBE_M = 256            # prefill-shaped probe of the int8 bind decision (worker_quant.py:885)

# Leaf names of MoE routers that are bare nn.Linear modules; never quantized (worker_quant.py:3051).
_ROUTER_LEAF_NAMES = frozenset({"gate", "router", "wg"})

# Token counts up to this take the fused MoE path; larger ones the eager per-expert loop. The
# reference fuses only T <= 8 because its kernel re-reads each expert's weight once per routed
# row; the HIP path groups rows by expert, so prefill-sized T stays on it.
_FUSED_MOE_T_MAX = int(os.environ.get("IM_FUSED_MOE_T_MAX", "4096"))

_BUILD_LOCK = threading.RLock()


def _log(msg: str) -> None:
    print(msg, flush=True)


# ---- dispatch helpers (worker_quant.py:240-263, 888-899, 1235-1335) --------------------------
def _rows(x) -> int:
    """Flattened row count of an activation ``[*, in_features]``."""
    n = 1
    for d in x.shape[:-1]:
        n *= int(d)
    return n


def _m_bucket(m: int) -> int:
    """Next power of two for m >= 2 (0 and 1 pass through), the reference's row bucket."""
    if m <= 1:
        return m
    b = 2
    while b < m:
        b <<= 1
    return b


def _cpu_fp32_worth(x) -> bool:
    import torch
    return (_CPU_FP32_GEMM and x.device.type == "cpu" and x.dtype != torch.float32
            and _rows(x) >= _CPU_FP32_MIN_ROWS)


def _time_cuda(fn, dev, iters: int = 30, warmup: int = 8) -> float:
    """Wall time per call in ms with the device synchronized (worker_quant.py:888-899)."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for _ in range(iters):
        fn()
    torch.cuda.synchronize(dev)
    return (time.perf_counter() - t0) / iters * 1e3


_LARGE_M_CHOICE: dict = {}


def _prefill_bench_m() -> int:
    """Row bucket of the production prefill chunk (INFINITEMODEL_PREFILL_CHUNK, default 2048)."""
    try:
        c = int(os.environ.get("INFINITEMODEL_PREFILL_CHUNK", "2048") or "2048")
    except (TypeError, ValueError):
        c = 2048
    if c <= 1:
        c = 2048
    return _m_bucket(c)


def _bench_large_m_naive(mod, tag: str) -> int:
    """Measured prefill dispatch threshold of a fused quant linear (worker_quant.py:1252-1335).

    Times the fused op and the naive dequant-once + BLAS GEMM at the prefill bucket; returns that
    bucket when naive wins by >= 13% (then descends to the smallest bucket where naive still wins,
    extrapolating the fused time linearly in rows), else 0 = fused for every M. Cached per
    (tag, N, in_pad, group). A failing bench returns 0 and is not cached."""
    if not _LARGE_M_NAIVE:
        return 0
    try:
        import torch
        import torch.nn.functional as F
        qw, szt, op, in_pad = mod._fused
        key = (tag, qw.shape[0], in_pad, mod.group_size)
        hit = _LARGE_M_CHOICE.get(key)
        if hit is not None:
            return hit
        dev = qw.device

        def _ms(fn, iters=2):
            fn()
            torch.cuda.synchronize(dev)
            t0 = time.perf_counter()
            for _ in range(iters):
                fn()
            torch.cuda.synchronize(dev)
            return (time.perf_counter() - t0) / iters * 1e3

        M = _prefill_bench_m()
        xt = torch.randn(M, mod.in_features, device=dev, dtype=torch.bfloat16)
        xk = xt if in_pad == mod.in_features else F.pad(xt, (0, in_pad - mod.in_features))
        xk = xk.contiguous()
        if tag == "int8":
            t_f = _ms(lambda: op(xk, qw, szt))
        else:
            t_f = _ms(lambda: op(xk, qw, mod.group_size, szt))
        t_n = _ms(lambda: F.linear(xt, mod._dequant(torch.bfloat16)))
        thr = M if t_n < t_f * 0.87 else 0
        if thr:
            f_per_row = t_f / max(1, M)
            b = M
            while b > 16:
                nb = b >> 1
                xt2 = torch.randn(nb, mod.in_features, device=dev, dtype=torch.bfloat16)
                t_n2 = _ms(lambda: F.linear(xt2, mod._dequant(torch.bfloat16)))
                if t_n2 >= f_per_row * nb * 0.87:
                    break
                b = nb
                thr = nb
        _LARGE_M_CHOICE[key] = thr
        _log(f"[{tag}] large-M dispatch [N={qw.shape[0]},Kpad={in_pad}]: M={M} fused={t_f:.2f}ms "
             f"naive={t_n:.2f}ms -> {f'naive at row-bucket>={thr}' if thr else 'fused for all M'}")
        return thr
    except Exception as exc:
        _log(f"[{tag}] large-M bench skipped ({exc!r})")
        return 0


def _is_rocm_device(dev) -> bool:
    import torch
    return dev.type == "cuda" and getattr(torch.version, "hip", None) is not None


# ---- op builders (worker_quant.py:926-1225, 1342-1495): HIP kernels behind the same signatures --
_OPS: dict = {}


def _build_op(name: str, make):
    """Thread-safe lazy build; None (and one log line) when libimq cannot be loaded."""
    if name in _OPS:
        return _OPS[name]
    with _BUILD_LOCK:
        if name in _OPS:
            return _OPS[name]
        try:
            from . import _lib
            _lib.lib()
            op = make()
        except Exception as exc:
            _log(f"[imq] {name} unavailable ({exc!r})")
            op = None
        _OPS[name] = op
        return op


def _w4a16_hip_op():
    """``op(x[M,Kpad] bf16, qweight u8[N,Kpad/2], group, (scale, zero) [N,ng]) -> y[M,N] bf16``."""
    def make():
        from . import ops
        return ops.linear_w4
    return _build_op("w4a16", make)


def _w2a16_hip_op():
    """``op(x[M,Kpad] bf16, qweight u8[N,Kpad/4], group, (scale, zero) [N,ng]) -> y[M,N] bf16``."""
    def make():
        from . import ops
        return ops.linear_w2
    return _build_op("w2a16", make)


def _w8a16_hip_op():
    """``op(x[M,K] bf16, qweight int8[N,K], scale[N,1]) -> y[M,N] bf16``."""
    def make():
        from . import ops
        return ops.linear_w8
    return _build_op("w8a16", make)


def _w4a16_moe_hip_op():
    """``op(x[B,Kin] bf16, eid[B], q u8[E,N,Kpad/2], scale, zero [E,N,ng], group, in_features)
    -> y[B,N] bf16``: each row b against expert eid[b]."""
    def make():
        from . import ops
        return ops.moe_rows_w4
    return _build_op("w4a16_moe", make)


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
    if bits == 4:
        parts = ((qweight & 0x0F), (qweight >> 4))
    else:
        parts = tuple(((qweight >> (2 * i)) & 0x3) for i in range(4))
    q = torch.stack([p.to(torch.int16) for p in parts], dim=2).reshape(out, -1)
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
    """Mean relative error of the fused op against ``F.linear(x, ref_w)`` at each M; returns
    (worst_rel, failing_M or 0) with the reference's rel < 0.05 rule."""
    import torch
    import torch.nn.functional as F
    rel = 0.0
    for M in Ms:
        xt = torch.randn(M, in_features, device=dev, dtype=torch.bfloat16)
        xk = xt if in_pad == in_features else F.pad(xt, (0, in_pad - in_features))
        yf = op_call(xk.contiguous()).float()
        yn = F.linear(xt, ref_w).float()
        rel = ((yf - yn).abs().mean() / (yn.abs().mean() + 1e-6)).item()
        if not (rel < 0.05):
            return rel, M
    return rel, 0


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

        def _dequant(self, dtype):
            """The dequantized weight ``[out, in_features]`` in ``dtype``, bit-exact to the
            reference dequant (libimq kernel on a ROCm device, torch on CPU)."""
            return _dequant_g(self.qweight, self.scale, self.zero, self.in_features, self.group_size,
                              dtype, bits)

        def prepare_fused(self):
            """Bind the HIP fused op after final device placement: de-alias the packed rows,
            self-check the op against ``F.linear(x, _dequant(bf16))`` at M=1 and M=8 (mean rel
            < 0.05), then measure the prefill dispatch threshold. Idempotent; never raises; any
            failure keeps the naive path (worker_quant.py:650-724, 1666-1722)."""
            enabled = _FUSED_INT4 if bits == 4 else _FUSED_INT2
            if not enabled or getattr(self, "_fused", None) is not None \
                    or getattr(self, "_fused_tried", False) or self.qweight is None:
                return
            self._fused_tried = True
            dev = self.qweight.device
            if not _is_rocm_device(dev):
                return
            op = _w4a16_hip_op() if bits == 4 else _w2a16_hip_op()
            if op is None:
                return
            try:
                G = self.group_size
                ng = self.scale.shape[1]
                in_pad = ng * G
                self.qweight = _dealias_rows(self.qweight)
                sz = (self.scale, self.zero)
                wref = self._dequant(torch.bfloat16)
                rel, bad_m = _selfcheck_rel(lambda xk: op(xk, self.qweight, G, sz), wref,
                                            self.in_features, in_pad, dev)
                del wref
                if not bad_m:
                    self._fused = (self.qweight, sz, op, in_pad)
                    self._naive_m_min = _bench_large_m_naive(self, tag)
                else:
                    _log(f"[{tag}] hip w{bits}a16 self-check rel={rel:.3f} at M={bad_m} on {dev} -> naive")
            except Exception as exc:
                _log(f"[{tag}] hip w{bits}a16 prepare failed on {dev} ({exc!r}) -> naive")

        def forward(self, x):
            fz = getattr(self, "_fused", None)
            nm = getattr(self, "_naive_m_min", 0)
            if fz is not None and nm and self.qweight is not None and _m_bucket(_rows(x)) >= nm:
                fz = None
            if fz is not None:
                qw, sz, op, in_pad = fz
                xq = x.reshape(-1, self.in_features)
                if xq.dtype != torch.bfloat16:
                    xq = xq.to(torch.bfloat16)
                if in_pad != self.in_features:
                    xq = F.pad(xq, (0, in_pad - self.in_features))
                y = op(xq.contiguous(), qw, self.group_size, sz).reshape(*x.shape[:-1], -1)
                y = y.to(x.dtype)
                return y if self.bias is None else y + self.bias.to(y.dtype)
            if _cpu_fp32_worth(x):
                b = self.bias
                y = F.linear(x.to(torch.float32), self._dequant(torch.float32),
                             None if b is None else b.to(torch.float32))
                return y.to(x.dtype)
            return F.linear(x, self._dequant(x.dtype), self.bias)

    _GroupQuantLinear.__name__ = _GroupQuantLinear.__qualname__ = \
        "QuantLinear4" if bits == 4 else "QuantLinear2"
    return _GroupQuantLinear


_QUANT_LINEAR4 = None
_QUANT_LINEAR2 = None
_QUANT_LINEAR = None
_PACKED4_3D = None
_W4A16_EXPERT = None
_PACKED8_3D = None
_W8A16_EXPERT = None


def _quant4_linear_cls():
    """QuantLinear4(qweight u8[N,K_pad/2], scale[N,ng], zero[N,ng], bias, in_features,
    group_size) (worker_quant.py:621-856)."""
    global _QUANT_LINEAR4
    if _QUANT_LINEAR4 is None:
        with _BUILD_LOCK:
            if _QUANT_LINEAR4 is None:
                _QUANT_LINEAR4 = _make_group_linear_cls(4)
    return _QUANT_LINEAR4


def _quant2_linear_cls():
    """QuantLinear2(qweight u8[N,K_pad/4], scale, zero, bias, in_features, group_size)
    (worker_quant.py:1635-1761)."""
    global _QUANT_LINEAR2
    if _QUANT_LINEAR2 is None:
        with _BUILD_LOCK:
            if _QUANT_LINEAR2 is None:
                _QUANT_LINEAR2 = _make_group_linear_cls(2)
    return _QUANT_LINEAR2


# ---- int8 per-row linear ---------------------------------------------------------------------
def _dequant8(qweight, scale, dtype):
    """``qweight.to(dtype) * scale`` with torch's promotion (worker_quant.py:439)."""
    if qweight.device.type == "cuda":
        from . import ops
        return ops.dequant_w8(qweight, scale, dtype)
    return qweight.to(dtype) * scale


def _quant_linear_cls():
    """QuantLinear(qweight int8[N,K], scale[N,1], bias) (worker_quant.py:391-508)."""
    global _QUANT_LINEAR
    if _QUANT_LINEAR is not None:
        return _QUANT_LINEAR
    with _BUILD_LOCK:
        if _QUANT_LINEAR is not None:
            return _QUANT_LINEAR
        import torch
        from torch import nn
        import torch.nn.functional as F

        class QuantLinear(nn.Module):
            def __init__(self, qweight, scale, bias):
                super().__init__()
                self.register_buffer("qweight", qweight)   # int8 [out, in]
                self.register_buffer("scale", scale)        # [out, 1]
                self.bias = bias

            def _dequant(self, dtype):
                return _dequant8(self.qweight, self.scale, dtype)

            def forward(self, x):
                if _cpu_fp32_worth(x):
                    w = self.qweight.to(torch.float32) * self.scale.to(torch.float32)
                    b = self.bias
                    y = F.linear(x.to(torch.float32), w, None if b is None else b.to(torch.float32))
                    return y.to(x.dtype)
                op = getattr(self, "_w8", None)
                if op is not None and x.dtype == torch.bfloat16:
                    mx = getattr(self, "_w8_m_max", 0)
                    if not mx or _rows(x) <= mx:
                        shape = x.shape
                        y = op(x.reshape(-1, shape[-1]), self.qweight, self.scale)
                        y = y.reshape(*shape[:-1], y.shape[-1])
                        return y if self.bias is None else y + self.bias
                return F.linear(x, self._dequant(x.dtype), self.bias)

            def prepare_fused(self):
                """Bind the HIP int8 op when it self-checks at M=1 and M=4 and beats the naive
                path at decode; a prefill probe (M=256) decides whether it also serves prefill
                (``_w8_m_max`` 0) or decode only (1). Never raises (worker_quant.py:442-505)."""
                if getattr(self, "_fused_tried", False) or not _FUSED_W8A16:
                    return
                self._fused_tried = True
                dev = self.qweight.device
                if not _is_rocm_device(dev):
                    return
                op = _w8a16_hip_op()
                if op is None:
                    return
                try:
                    K = int(self.qweight.shape[1])
                    # reference check weight: qweight.to(bf16) * scale.to(bf16), in bf16
                    wref = _dequant8(self.qweight, self.scale.to(torch.bfloat16), torch.bfloat16)
                    for M in (1, 4):
                        xt = torch.randn(M, K, device=dev, dtype=torch.bfloat16)
                        yf = op(xt, self.qweight, self.scale).float()
                        yn = F.linear(xt, wref).float()
                        rel = ((yf - yn).abs().mean() / (yn.abs().mean() + 1e-6)).item()
                        if not (rel < 0.05):
                            _log(f"[int8] hip w8a16 self-check rel={rel:.3f} at M={M} on {dev} -> naive")
                            return
                    sb = self.scale.to(torch.bfloat16)
                    x1 = torch.randn(1, K, device=dev, dtype=torch.bfloat16)
                    t_f = _time_cuda(lambda: op(x1, self.qweight, self.scale), dev)
                    t_n = _time_cuda(lambda: F.linear(x1, _dequant8(self.qweight, sb, torch.bfloat16)), dev)
                    del wref
                    if not (t_f < t_n):
                        _log(f"[int8] hip w8a16 {t_f:.3f}ms vs dequant+F.linear {t_n:.3f}ms on {dev} -> naive")
                        return
                    self._w8 = op
                    xp = torch.randn(_W8_PROBE_M, K, device=dev, dtype=torch.bfloat16)
                    p_f = _time_cuda(lambda: op(xp, self.qweight, self.scale), dev, iters=6, warmup=2)
                    p_n = _time_cuda(lambda: F.linear(xp, _dequant8(self.qweight, sb, torch.bfloat16)),
                                     dev, iters=6, warmup=2)
                    self._w8_m_max = 0 if p_f < p_n else 1
                except Exception as exc:
                    _log(f"[int8] hip w8a16 prepare failed on {dev} ({exc!r}) -> naive")

        _QUANT_LINEAR = QuantLinear
    return _QUANT_LINEAR


# ---- one expert's int4 weight as a tensor subclass (worker_quant.py:1501-1585) ----------------
def _w4a16_expert_cls():
    """Tensor subclass for one expert's packed int4 weight: ``F.linear(x, w)`` runs the HIP
    fused op on the packed bytes; any other op materializes the bf16 dequant. None when libimq
    is unavailable."""
    global _W4A16_EXPERT
    if _W4A16_EXPERT is not None:
        return _W4A16_EXPERT
    with _BUILD_LOCK:
        if _W4A16_EXPERT is not None:
            return _W4A16_EXPERT
        op = _w4a16_hip_op()
        if op is None:
            return None
        import torch
        import torch.nn.functional as F

        class _W4A16Weight(torch.Tensor):
            @staticmethod
            def __new__(cls, packed, scale, zero, group, in_features):
                t = torch.Tensor._make_wrapper_subclass(
                    cls, (packed.shape[0], in_features), dtype=scale.dtype, device=packed.device,
                    requires_grad=False)
                t._packed = packed
                t._scale = scale
                t._zero = zero
                t._group = group
                t._infeat = in_features
                return t

            def _materialize(self):
                return _dequant_g(self._packed, self._scale, self._zero, self._infeat, self._group,
                                  self._scale.dtype, 4)

            @classmethod
            def __torch_function__(cls, func, types, args=(), kwargs=None):
                kwargs = kwargs or {}
                if func is F.linear or getattr(func, "__name__", "") == "linear":
                    inp = args[0]
                    w = args[1] if len(args) > 1 else kwargs.get("weight")
                    bias = args[2] if len(args) > 2 else kwargs.get("bias")
                    if isinstance(w, cls):
                        y = op(inp, w._packed, w._group, (w._scale, w._zero))
                        if inp.dim() > 2:
                            y = y.reshape(*inp.shape[:-1], y.shape[-1])
                        return y if bias is None else y + bias.to(y.dtype)
                mat = [a._materialize() if isinstance(a, cls) else a for a in args]
                mkw = {k: (v._materialize() if isinstance(v, cls) else v) for k, v in kwargs.items()}
                return func(*mat, **mkw)

            @classmethod
            def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
                kwargs = kwargs or {}
                mat = [a._materialize() if isinstance(a, cls) else a for a in args]
                mkw = {k: (v._materialize() if isinstance(v, cls) else v) for k, v in kwargs.items()}
                return func(*mat, **mkw)

        _W4A16_EXPERT = _W4A16Weight
    return _W4A16_EXPERT


# ---- fused 3D int4 experts (worker_quant.py:1967-2125) ---------------------------------------
def _packed4_3d_cls():
    """Packed4Tensor3D(qweight u8[E,N,K_pad/2], scale[E,N,ng], zero[E,N,ng], in_features,
    group_size)."""
    global _PACKED4_3D
    if _PACKED4_3D is not None:
        return _PACKED4_3D
    with _BUILD_LOCK:
        if _PACKED4_3D is not None:
            return _PACKED4_3D
        import torch
        from torch import nn

        class Packed4Tensor3D(nn.Module):
            _pad_choice: dict = {}     # (E, N, rs) -> bool, one measurement per shape

            def __init__(self, qweight, scale, zero, in_features, group_size):
                super().__init__()
                self.register_buffer("qweight", qweight)   # uint8 [E, out, in_pad//2]
                self.register_buffer("scale", scale)        # [E, out, ng]
                self.register_buffer("zero", zero)          # [E, out, ng]
                self.in_features = in_features
                self.group_size = group_size
                self._expert_triton = None                  # fused-expert weights enabled (lazy)

            def _expert_selfcheck(self) -> bool:
                wc = _w4a16_expert_cls()
                if wc is None:
                    return False
                import torch.nn.functional as F
                w0 = wc(self.qweight[0], self.scale[0], self.zero[0], self.group_size, self.in_features)
                wref = w0._materialize()
                for M in (1, 8):
                    xt = torch.randn(M, self.in_features, device=self.qweight.device, dtype=torch.bfloat16)
                    yn = F.linear(xt, wref).float()
                    yf = F.linear(xt, w0).float()
                    rel = ((yf - yn).abs().mean() / (yn.abs().mean() + 1e-6)).item()
                    if not (rel < 0.05):
                        _log(f"[int4] hip w4a16 experts self-check rel={rel:.3f} at M={M} -> bf16 dequant")
                        return False
                return True

            def __getitem__(self, e):
                """Expert e's weight for ``F.linear(bf16_x, w)``: the fused-op subclass on a ROCm
                device once it self-checks, else the bf16 dequant."""
                e = int(e)
                if self._expert_triton is None:
                    self._expert_triton = False
                    with contextlib.suppress(Exception):
                        if _is_rocm_device(self.qweight.device):
                            self._expert_triton = self._expert_selfcheck()
                if self._expert_triton:
                    return _w4a16_expert_cls()(self.qweight[e], self.scale[e], self.zero[e],
                                               self.group_size, self.in_features)
                return _dequant_g(self.qweight[e], self.scale[e], self.zero[e], self.in_features,
                                  self.group_size, self.scale.dtype, 4)

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

            def _dealias_ms(self, op, q, sc, ze, iters=25):
                """Fused expert GEMV time on ``q`` at a decode shape over fresh random expert
                subsets, in ms."""
                E = q.shape[0]
                B = min(8, E)
                x = torch.randn(B, self.in_features, device=q.device, dtype=torch.bfloat16) * 0.1
                eids = [torch.randperm(E, device=q.device)[:B].to(torch.int32) for _ in range(iters + 3)]
                for i in range(3):
                    op(x, eids[i], q, sc, ze, self.group_size, self.in_features)
                torch.cuda.synchronize(q.device)
                t0 = time.perf_counter()
                for i in range(iters):
                    op(x, eids[3 + i], q, sc, ze, self.group_size, self.in_features)
                torch.cuda.synchronize(q.device)
                return (time.perf_counter() - t0) / iters * 1e3

            def prepare_fused(self):
                """Kernel layout (``_kernel_tensors``), then the measured expert-row de-alias:
                keep ``[E, N, rs+64]`` padded rows only when the fused op runs >= 15% faster on
                them; decision cached per (E, N, rs). Idempotent; never raises
                (worker_quant.py:2067-2122)."""
                if getattr(self, "_dealiased", False):
                    return
                self._dealiased = True
                qw = self.qweight
                if qw is None or qw.dim() != 3 or not _is_rocm_device(qw.device):
                    return
                try:
                    kq, ks, kz = self._kernel_tensors()
                except Exception as exc:
                    _log(f"[int4] moe kernel layout skipped ({exc!r})")
                    return
                E, N, rs = kq.shape
                if rs % 128 != 0 or kq.stride(2) != 1 or kq.stride(1) != rs:
                    return
                op = _w4a16_moe_hip_op()
                if op is None:
                    return
                try:
                    choice = Packed4Tensor3D._pad_choice.get((E, N, rs))
                    buf = None
                    if choice is None:
                        buf = torch.zeros((E, N, rs + 64), dtype=torch.uint8, device=kq.device)
                        buf[:, :, :rs].copy_(kq)
                        t_un = self._dealias_ms(op, kq, ks, kz)
                        t_pad = self._dealias_ms(op, buf[:, :, :rs], ks, kz)
                        choice = t_pad < t_un * 0.87
                        Packed4Tensor3D._pad_choice[(E, N, rs)] = choice
                        _log(f"[int4] moe row de-alias [E={E},N={N},rs={rs}]: unpadded={t_un:.3f}ms "
                             f"padded={t_pad:.3f}ms -> {'PAD' if choice else 'keep unpadded'}")
                    if choice:
                        if buf is None:
                            buf = torch.zeros((E, N, rs + 64), dtype=torch.uint8, device=kq.device)
                            buf[:, :, :rs].copy_(kq)
                        self.qweight = buf[:, :, :self.qweight.shape[2]]
                        self._kt = (buf[:, :, :rs], ks, kz, self.qweight)
                except Exception as exc:
                    _log(f"[int4] moe row de-alias skipped ({exc!r})")

        _PACKED4_3D = Packed4Tensor3D
    return _PACKED4_3D


# ---- fused MoE experts forward (worker_quant.py:2131-2248) -----------------------------------
def _moe_fused_compute(experts_mod, hidden_states, top_k_index, top_k_weights):
    """All routed experts of one layer in one libimq call: token-sorted grouped expert GEMMs for
    gate_up and down, SwiGLU between them, and the weighted combine into ``[T, H]``."""
    from . import ops
    gu, dn = experts_mod.gate_up_proj, experts_mod.down_proj
    I = int(dn.in_features)
    out = ops.moe_experts_w4(hidden_states, top_k_index, top_k_weights,
                             (*gu._kernel_tensors(), int(gu.in_features)),
                             (*dn._kernel_tensors(), I), int(gu.group_size))
    return out.to(hidden_states.dtype)


def _act_is_silu(act) -> bool:
    import torch
    if isinstance(act, torch.nn.SiLU):
        return True
    name = getattr(act, "__name__", "") or type(act).__name__
    return name.lower() in ("silu", "siluactivation", "silu_")


def _install_fused_moe_forward(experts_mod) -> None:
    """Patch a fused-3D int4 experts module (``gate_up_proj``/``down_proj`` Packed4Tensor3D +
    ``act_fn``) so small and medium token counts run the fused HIP path; a one-time self-check
    against the original eager forward (T=2 and T=1, mean rel < 0.03, max rel < 0.1) gates it,
    and any exception falls back to the original forward. INFINITEMODEL_NO_FUSED_MOE disables it."""
    import types
    if os.environ.get("INFINITEMODEL_NO_FUSED_MOE"):
        return
    PT = _packed4_3d_cls()
    gu = getattr(experts_mod, "gate_up_proj", None)
    dn = getattr(experts_mod, "down_proj", None)
    if not (isinstance(gu, PT) and isinstance(dn, PT) and hasattr(experts_mod, "act_fn")):
        return
    if getattr(experts_mod, "_fused_moe_installed", False):
        return
    if not _act_is_silu(experts_mod.act_fn):
        return                      # the fused kernel implements SiLU-GLU only
    if _w4a16_moe_hip_op() is None:
        return
    orig_forward = experts_mod.forward

    def _selfcheck(self):
        import torch
        try:
            gu_h, dn_h = self.gate_up_proj, self.down_proj
            if not _is_rocm_device(gu_h.qweight.device):
                return False
            E = int(gu_h.qweight.shape[0])
            H = int(gu_h.in_features)
            dev = gu_h.qweight.device
            k = min(8, E)
            worst = worst_max = 0.0
            for T in (2, 1):
                x = torch.randn(T, H, device=dev, dtype=torch.bfloat16) * 0.1
                idx = torch.stack([torch.randperm(E, device=dev)[:k] for _ in range(T)])
                wts = torch.rand(T, k, device=dev, dtype=torch.bfloat16) + 0.1
                sv = (gu_h._expert_triton, dn_h._expert_triton)
                gu_h._expert_triton = dn_h._expert_triton = False
                try:
                    ref = orig_forward(x, idx, wts).float()
                finally:
                    gu_h._expert_triton, dn_h._expert_triton = sv
                out = _moe_fused_compute(self, x, idx, wts).float()
                worst = max(worst, ((out - ref).abs().mean() / (ref.abs().mean() + 1e-6)).item())
                worst_max = max(worst_max, ((out - ref).abs().max() / (ref.abs().max() + 1e-6)).item())
            ok = worst < 0.03 and worst_max < 0.1
            _log(f"[int4] fused-MoE self-check rel={worst:.4f} max={worst_max:.4f} -> "
                 f"{'ACTIVE' if ok else 'fallback (per-expert)'}")
            return ok
        except Exception as exc:
            _log(f"[int4] fused-MoE self-check failed ({exc!r}) -> per-expert")
            return False

    def _fused_forward(self, hidden_states, top_k_index, top_k_weights):
        if hidden_states.shape[0] <= _FUSED_MOE_T_MAX:
            if self._fused_moe_ok is None:
                self._fused_moe_ok = _selfcheck(self)
            if self._fused_moe_ok:
                try:
                    return _moe_fused_compute(self, hidden_states, top_k_index, top_k_weights)
                except Exception:
                    pass
        return orig_forward(hidden_states, top_k_index, top_k_weights)

    experts_mod._fused_moe_ok = None
    experts_mod._fused_moe_installed = True
    experts_mod.forward = types.MethodType(_fused_forward, experts_mod)


# ---- gpt-oss fused experts (worker_quant.py:2250-2314) ---------------------------------------
def _is_gptoss_experts(module) -> bool:
    """A gpt-oss fused-expert block: interleaved clamped SwiGLU with per-expert biases
    (worker_quant.py:2257-2262)."""
    if type(module).__name__ == "GptOssExperts":
        return True
    return (hasattr(module, "gate_up_proj_bias") and hasattr(module, "down_proj_bias")
            and hasattr(module, "alpha") and hasattr(module, "limit"))


def _gptoss_fused_ok() -> bool:
    """gpt-oss int4 needs the fused MoE kernel: its experts are transpose-packed, so there is no
    eager host path to fall back to (worker_quant.py:2265-2276). True when libimq loads, unless
    INFINITEMODEL_NO_FUSED_MOE is set."""
    if os.environ.get("INFINITEMODEL_NO_FUSED_MOE"):
        return False
    return _w4a16_moe_hip_op() is not None


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
                             limit=float(getattr(experts_mod, "limit", 7.0)))
    return out.to(hidden_states.dtype)


def _install_gptoss_fused_forward(experts_mod) -> None:
    """Install gpt-oss's int4 fused-expert forward (worker_quant.py:2280-2314) for every token
    count: once the experts are transpose-packed there is no eager fallback. The caller has
    transpose-packed the experts and checked ``_gptoss_fused_ok()``."""
    import types

    def _forward(self, hidden_states, router_indices=None, routing_weights=None):
        return _gptoss_fused_compute(self, hidden_states, router_indices, routing_weights)

    experts_mod._gptoss_fused_installed = True
    experts_mod.forward = types.MethodType(_forward, experts_mod)
    _log("[int4] gpt-oss fused experts active (transpose-packed w4a16 + interleaved SwiGLU)")


# ---- int8 fused 3D experts (worker_quant.py:2707-2990) ---------------------------------------
def _w8a16_experts_ok(dev) -> bool:
    """Should Packed8Tensor3D hand the eager MoE loop the w8a16 expert subclass instead of a
    dequantized weight (worker_quant.py:2711-2731)? On a ROCm device unless IM_W8A16_EXPERTS=0 or
    IM_FUSED_W8A16=0; never on the CPU."""
    if os.environ.get("IM_W8A16_EXPERTS", "") == "0" or not _FUSED_W8A16:
        return False
    return _is_rocm_device(dev)


def _w8a16_expert_cls():
    """Tensor subclass for one expert's int8 weight (worker_quant.py:2734-2806): ``F.linear`` of
    a bf16 activation runs the HIP w8a16 op on the int8 bytes; every other op materializes
    ``qweight.to(scale.dtype) * scale``. None when libimq is unavailable."""
    global _W8A16_EXPERT
    if _W8A16_EXPERT is not None:
        return _W8A16_EXPERT
    with _BUILD_LOCK:
        if _W8A16_EXPERT is not None:
            return _W8A16_EXPERT
        op = _w8a16_hip_op()
        if op is None:
            return None
        import torch
        import torch.nn.functional as F

        class _W8A16Weight(torch.Tensor):
            @staticmethod
            def __new__(cls, packed, scale):
                out, in_f = packed.shape
                t = torch.Tensor._make_wrapper_subclass(cls, (out, in_f), dtype=scale.dtype,
                                                        device=packed.device, requires_grad=False)
                t._packed = packed          # int8 [out, in]
                t._scale = scale            # [out, 1]
                return t

            def _materialize(self):
                return (self._packed.to(self._scale.dtype) * self._scale).contiguous()

            @classmethod
            def __torch_function__(cls, func, types, args=(), kwargs=None):
                kwargs = kwargs or {}
                if func is F.linear or getattr(func, "__name__", "") == "linear":
                    inp = args[0]
                    w = args[1] if len(args) > 1 else kwargs.get("weight")
                    bias = args[2] if len(args) > 2 else kwargs.get("bias")
                    # bf16 activations only, as the dense int8 path gates (worker_quant.py:2770-2774)
                    if isinstance(w, cls) and getattr(inp, "dtype", None) is torch.bfloat16:
                        y = op(inp, w._packed, w._scale)
                        if inp.dim() > 2:
                            y = y.reshape(*inp.shape[:-1], y.shape[-1])
                        return y if bias is None else y + bias.to(y.dtype)
                mat = [a._materialize() if isinstance(a, cls) else a for a in args]
                mkw = {k: (v._materialize() if isinstance(v, cls) else v) for k, v in kwargs.items()}
                return func(*mat, **mkw)

            @classmethod
            def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
                kwargs = kwargs or {}
                mat = [a._materialize() if isinstance(a, cls) else a for a in args]
                mkw = {k: (v._materialize() if isinstance(v, cls) else v) for k, v in kwargs.items()}
                return func(*mat, **mkw)

        _W8A16_EXPERT = _W8A16Weight
    return _W8A16_EXPERT


def _packed8_3d_cls():
    """Packed8Tensor3D(qweight int8 [E, out, in], scale [E, out, 1], in_features)
    (worker_quant.py:2813-2897): all of one projection's experts at int8 behind the eager
    experts loop's ``self.gate_up_proj[e]`` indexing."""
    global _PACKED8_3D
    if _PACKED8_3D is not None:
        return _PACKED8_3D
    with _BUILD_LOCK:
        if _PACKED8_3D is not None:
            return _PACKED8_3D
        import torch
        from torch import nn

        class Packed8Tensor3D(nn.Module):
            def __init__(self, qweight, scale, in_features):
                super().__init__()
                self.register_buffer("qweight", qweight)   # int8 [E, out, in]
                self.register_buffer("scale", scale)        # [E, out, 1]
                self.in_features = in_features
                self._expert_triton = None                  # fused-expert weights enabled (lazy)

            def _expert_selfcheck(self) -> bool:
                """One-time check of the w8a16 expert subclass against the dequant it replaces,
                at M = 1 and M = 8 (mean rel < 0.05)."""
                import torch.nn.functional as F
                wc = _w8a16_expert_cls()
                if wc is None:
                    return False
                w0 = wc(self.qweight[0], self.scale[0])
                wref = w0._materialize()
                for M in (1, 8):
                    xt = torch.randn(M, self.in_features, device=self.qweight.device, dtype=torch.bfloat16)
                    yn = F.linear(xt, wref).float()
                    yf = F.linear(xt, w0).float()
                    rel = ((yf - yn).abs().mean() / (yn.abs().mean() + 1e-6)).item()
                    if not (rel < 0.05):
                        _log(f"[int8] hip w8a16 experts self-check rel={rel:.3f} at M={M} -> dequant")
                        return False
                _log(f"[int8] hip w8a16 experts active (rel={rel:.4f})")
                return True

            def __getitem__(self, e):
                """Expert e's weight for ``F.linear(bf16_x, w)``: the w8a16 subclass on a ROCm
                device with a bf16 scale once it self-checks, else ``q.to(dt) * scale``."""
                e = int(e)
                if self._expert_triton is None:
                    self._expert_triton = False
                    with contextlib.suppress(Exception):
                        if _w8a16_experts_ok(self.qweight.device) and self.scale.dtype is torch.bfloat16:
                            self._expert_triton = self._expert_selfcheck()
                if self._expert_triton:
                    return _w8a16_expert_cls()(self.qweight[e], self.scale[e])
                return (self.qweight[e].to(self.scale.dtype) * self.scale[e]).contiguous()

        _PACKED8_3D = Packed8Tensor3D
    return _PACKED8_3D


def _pack8_3d(W3):
    """Fused expert tensor [E, out, in] -> Packed8Tensor3D, one expert at a time through the 2D
    int8 packer (worker_quant.py:2900-2921): per-row scales never cross an expert, so this equals
    the 2D packer on every expert slice."""
    import torch
    E, out, in_f = W3.shape
    q = torch.empty((E, out, in_f), dtype=torch.int8, device=W3.device)
    sc = torch.empty((E, out, 1), dtype=W3.dtype, device=W3.device)
    for e in range(E):
        qe, se = _pack8_expert(W3[e])
        q[e] = qe
        sc[e] = se
    return _packed8_3d_cls()(q, sc, in_f)


def _quantize_experts8_(module) -> None:
    """int8 twin of ``_quantize_experts4_`` (worker_quant.py:2924-2987): 3D ``gate_up_proj`` /
    ``down_proj`` Parameters -> Packed8Tensor3D and the eager experts implementation. Refuses
    gpt-oss (no int8 form of its transpose-packed fused forward) and meta experts (streaming is
    int4-only). No fused-MoE forward is installed: int8 experts run the eager loop, each routed
    expert through the w8a16 subclass."""
    from torch import nn
    targets = []
    for sub in module.modules():
        is_go = _is_gptoss_experts(sub)
        for attr in ("gate_up_proj", "down_proj"):
            p = sub._parameters.get(attr)
            if isinstance(p, nn.Parameter) and p.dim() == 3:
                targets.append((sub, attr, is_go))
    if not targets:
        return
    if any(is_go for _s, _a, is_go in targets):
        raise RuntimeError("gpt-oss fused experts have no int8 path (in-major transpose-packed "
                           "weights need the fused w4a16 MoE forward) -- load gpt-oss at int4")
    for sub, attr, _is_go in targets:
        p = getattr(sub, attr)
        if getattr(p, "is_meta", False):
            raise RuntimeError(f"int8 MoE: {type(sub).__name__}.{attr} is META -- per-expert "
                               "expert streaming is int4-only; load this model at int4")
        delattr(sub, attr)
        setattr(sub, attr, _pack8_3d(p.data))
    seen = set()
    for sub, _attr, _is_go in targets:
        cfg = getattr(sub, "config", None)
        if cfg is not None and hasattr(cfg, "_experts_implementation") and id(cfg) not in seen:
            cfg._experts_implementation = "eager"
            seen.add(id(cfg))


def _quantize_int8_(module) -> None:
    """int8 a decoder layer (worker_quant.py:578-596): every nn.Linear except routers, then the
    fused 3D routed experts."""
    _quantize_int8_linears_(module)
    _quantize_experts8_(module)


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
        dev = head_device if head_device is not None else next(head.parameters()).device
        dev = torch.device(dev)
        tied = bool(getattr(getattr(model, "config", None), "tie_word_embeddings", False))
        if hq == "int8" and dev.type != "cuda":
            _log(f"[head-quant] int8 head SKIPPED: lm_head is on {dev} and the w8a16 kernel is "
                 "GPU-only -- bf16 is faster there")
        elif hq == "int8" and not isinstance(head, torch.nn.Linear):
            _log(f"[head-quant] int8 head already packed by the load tier ({type(head).__name__})")
        elif hq == "int8" and tied:
            _log("[head-quant] int8 head SKIPPED: tie_word_embeddings -- lm_head aliases "
                 "embed_tokens, so packing it would add a copy, not replace one")
        elif hq == "int8":
            nbytes = head.weight.numel() * head.weight.element_size()
            q = _quantize_linear(head.to("cpu")).to(dev)
            head = q
            if hasattr(model, "lm_head"):
                model.lm_head = q
            pk = q.qweight.numel() + q.scale.numel() * q.scale.element_size()
            _log(f"[head-quant] lm_head int8: {nbytes / 2**30:.2f} GB bf16 -> {pk / 2**30:.2f} GB "
                 f"({nbytes / max(1, pk):.1f}x fewer bytes read per decoded token)")
        elif hq == "bf16" and not isinstance(head, torch.nn.Linear):
            _log("[head-quant] bf16 head requested but the head is already quantized by the load "
                 "tier -- leaving it")
    except Exception as exc:
        _log(f"[head-quant] FAILED ({exc!r}) -> leaving the lm_head as built")
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


def _quantize_linears_(module, convert) -> None:
    """Replace every nn.Linear under ``module`` with ``convert(lin)``, except MoE routers: leaf
    names in _ROUTER_LEAF_NAMES and whole subtrees whose class name ends in Router/Gate."""
    from torch import nn
    for name, child in list(module.named_children()):
        if isinstance(child, nn.Linear):
            if name in _ROUTER_LEAF_NAMES:
                continue
            setattr(module, name, convert(child))
        elif type(child).__name__.endswith(("Router", "Gate")):
            continue
        else:
            _quantize_linears_(child, convert)


def _quantize_int4_(module) -> None:
    _quantize_linears_(module, _quantize_linear4)


def _quantize_int2_(module) -> None:
    _quantize_linears_(module, _quantize_linear2)


def _quantize_int8_linears_(module) -> None:
    _quantize_linears_(module, _quantize_linear)


def _quantize_experts4_(module) -> None:
    """Replace 3D ``gate_up_proj``/``down_proj`` expert Parameters with Packed4Tensor3D
    (worker_quant.py:2439-2483). gpt-oss blocks store their experts in-major [E, in, out] and are
    transposed to [E, out, in] before packing; they get the dedicated fused forward (and need it:
    RuntimeError when it is unavailable). Every other block gets the eager experts implementation
    on its config and the fused-MoE forward."""
    from torch import nn
    targets = []
    for sub in module.modules():
        is_go = _is_gptoss_experts(sub)
        for attr in ("gate_up_proj", "down_proj"):
            p = sub._parameters.get(attr)
            if isinstance(p, nn.Parameter) and p.dim() == 3:
                targets.append((sub, attr, is_go))
    if any(is_go for _s, _a, is_go in targets) and not _gptoss_fused_ok():
        raise RuntimeError("gpt-oss int4 requires the fused w4a16 MoE kernel (libimq on a ROCm "
                           "device) -- load gpt-oss at quant=none (bf16) here")
    for sub, attr, is_go in targets:
        p = getattr(sub, attr)
        delattr(sub, attr)
        w = p.data.transpose(1, 2).contiguous() if is_go else p.data
        setattr(sub, attr, _pack4_3d(w))
    seen = set()
    for sub, _attr, is_go in targets:
        if is_go:
            continue
        cfg = getattr(sub, "config", None)
        if cfg is not None and hasattr(cfg, "_experts_implementation") and id(cfg) not in seen:
            cfg._experts_implementation = "eager"
            seen.add(id(cfg))
    done = set()
    for sub, _attr, is_go in targets:
        if id(sub) not in done:
            done.add(id(sub))
            if is_go:
                _install_gptoss_fused_forward(sub)
            else:
                _install_fused_moe_forward(sub)


def finalize_placement(model) -> int:
    """Call ``prepare_fused`` on every submodule that has it (after the model reached its final
    device) and return how many ended with a bound fused op (client.py:852-864)."""
    n = 0
    for sub in model.modules():
        if hasattr(sub, "prepare_fused"):
            sub.prepare_fused()
            if getattr(sub, "_fused", None) is not None or getattr(sub, "_w8", None) is not None:
                n += 1
    return n
