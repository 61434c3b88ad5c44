"""torch-facing wrappers of the libimq kernels.

Every function takes/returns torch tensors on a ROCm device, checks shapes/strides on the host,
and launches on torch's current stream for that device. Outputs are allocated with torch (so
they come from the caching allocator, and from the graph pool under stream capture). Nothing
here synchronizes except the MoE ops' routing-id check, which is skipped under stream capture,
so these calls are capturable into HIP graphs.

These are the product path: they never fall back to a CPU/torch computation. A missing library
raises ``ImqUnavailable``, a rejected call raises ``ImqError``.
"""
from __future__ import annotations

import torch

from . import _lib
from ._lib import call, dtype_code


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _check_dev(*ts):
    dev = ts[0].device
    if dev.type != "cuda":
        raise ValueError("libimq ops need tensors on a ROCm device")
    for t in ts[1:]:
        if t is not None and t.device != dev:
            raise ValueError(f"device mismatch: {t.device} vs {dev}")
    return dev


def _rows2d(x: torch.Tensor) -> torch.Tensor:
    if x.dim() != 2:
        x = x.reshape(-1, x.shape[-1])
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    if x.stride(1) != 1 or (x.stride(0) % 8) != 0 or (x.data_ptr() % 16) != 0:
        x = x.contiguous()
    return x


# Workspaces (split-K / K-split partials of the fused linears, MoE intermediates), one per
# (device, stream): calls sharing one are ordered by that stream, and their contents need no
# initialization. A workspace is never freed once handed out, because a HIP graph captured with it
# keeps its address: when a call needs more, the old buffer is retired (kept alive for the life of
# the process) and one at least twice its size takes its place, so at most log2(largest need)
# buffers are ever retired per stream.
_WS: dict = {}
_WS_RETIRED: list = []


def _scratch(dev: torch.device, need: int):
    """The (device, current stream) workspace of at least ``need`` bytes, or None if need <= 0."""
    if need <= 0:
        return None
    key = (dev.index, torch.cuda.current_stream(dev).cuda_stream)
    ws = _WS.get(key)
    if ws is None or ws.numel() < need:
        size = need
        if ws is not None:
            _WS_RETIRED.append(ws)
            size = max(need, 2 * ws.numel())
        ws = torch.empty(size, dtype=torch.uint8, device=dev)
        _WS[key] = ws
    return ws


def _workspace(dev: torch.device, M: int, N: int, K: int):
    ws = _scratch(dev, int(_lib.lib().imq_linear_workspace_bytes(M, N, K)))
    if ws is None:
        return 0, 0
    return ws.data_ptr(), ws.numel()


def _check_expert_ids(idx: torch.Tensor, E: int) -> None:
    """Refuse routing ids outside [0, E), as the reference's eager experts loop does (its
    ``one_hot(num_classes=E)`` raises). One device-to-host read, so it is skipped while a HIP graph
    is being captured (the kernels then only keep out-of-range ids' loads in bounds)."""
    if idx.numel() == 0 or (idx.is_cuda and torch.cuda.is_current_stream_capturing()):
        return
    lo, hi = (int(v) for v in torch.aminmax(idx))
    if lo < 0 or hi >= E:
        raise ValueError(f"expert ids must lie in [0, {E}); got ids in [{lo}, {hi}]")


def _check_packed(q: torch.Tensor, dt=torch.uint8):
    if q.dtype != dt or q.dim() < 2 or q.stride(-1) != 1:
        raise ValueError(f"packed weight must be {dt} with a unit last stride, got {q.dtype} {tuple(q.stride())}")


# ---------------------------------------------------------------------------------------------
# dequant (bit-exact reference dequant)
# ---------------------------------------------------------------------------------------------
def _dequant_g(fn: str, bits: int, qweight, scale, zero, in_features: int, group_size: int, dtype):
    dev = _check_dev(qweight, scale, zero)
    _check_packed(qweight)
    N = qweight.shape[0]
    out = torch.empty((N, in_features), dtype=dtype, device=dev)
    with torch.cuda.device(dev):
        call(fn, _ptr(qweight), qweight.stride(0), _ptr(scale), scale.stride(0), scale.stride(1),
             dtype_code(scale.dtype), _ptr(zero), zero.stride(0), zero.stride(1), dtype_code(zero.dtype),
             N, in_features, group_size, _ptr(out), out.stride(0), dtype_code(dtype), _stream(dev))
    return out


def dequant_w4(qweight, scale, zero, in_features: int, group_size: int, dtype=torch.bfloat16):
    """QuantLinear4._dequant(dtype) on the GPU (worker_quant.py:638-648), bit-exact."""
    return _dequant_g("imq_dequant_w4", 4, qweight, scale, zero, in_features, group_size, dtype)


def dequant_w2(qweight, scale, zero, in_features: int, group_size: int, dtype=torch.bfloat16):
    """QuantLinear2._dequant(dtype) on the GPU (worker_quant.py:1652-1664), bit-exact."""
    return _dequant_g("imq_dequant_w2", 2, qweight, scale, zero, in_features, group_size, dtype)


def dequant_w8(qweight, scale, dtype):
    """``qweight.to(x_dtype) * scale`` (worker_quant.py:439) with torch's dtype promotion: the
    result dtype is ``torch.promote_types(dtype, scale.dtype)``."""
    dev = _check_dev(qweight, scale)
    _check_packed(qweight, torch.int8)
    res = torch.promote_types(dtype, scale.dtype)
    N, K = qweight.shape
    out = torch.empty((N, K), dtype=res, device=dev)
    with torch.cuda.device(dev):
        call("imq_dequant_w8", _ptr(qweight), qweight.stride(0), _ptr(scale), scale.stride(0),
             dtype_code(scale.dtype), N, K, _ptr(out), out.stride(0), dtype_code(res), _stream(dev))
    return out


# ---------------------------------------------------------------------------------------------
# RTN packers on the device (bit-identical to shard_compile.pack_linear_int4 / int2 / int8)
# ---------------------------------------------------------------------------------------------
def _pack_g(fn: str, bits: int, W, group_size: int):
    dev = _check_dev(W)
    if W.dim() != 2 or W.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError(f"W must be a 2D bf16 / fp16 / fp32 tensor, got {W.dtype} {tuple(W.shape)}")
    if W.stride(1) != 1:
        W = W.contiguous()
    N, in_f = W.shape
    ng = -(-in_f // group_size)
    q = torch.empty((N, ng * group_size * bits // 8), dtype=torch.uint8, device=dev)
    scale = torch.empty((N, ng), dtype=W.dtype, device=dev)
    zero = torch.empty((N, ng), dtype=W.dtype, device=dev)
    with torch.cuda.device(dev):
        call(fn, _ptr(W), W.stride(0), dtype_code(W.dtype), N, in_f, group_size, _ptr(q), q.stride(0),
             _ptr(scale), _ptr(zero), scale.stride(0), _stream(dev))
    return q, scale, zero, in_f


def pack_w4(W, group_size: int = 128):
    """``pack_linear_int4`` on the device: (qweight u8 [N, K_pad/2], scale, zero, in_features)
    (shard_compile.py:74-94)."""
    return _pack_g("imq_pack_w4", 4, W, group_size)


def pack_w2(W, group_size: int = 64):
    """``pack_linear_int2`` on the device: (qweight u8 [N, K_pad/4], scale, zero, in_features)
    (shard_compile.py:50-71)."""
    return _pack_g("imq_pack_w2", 2, W, group_size)


def pack_w8(W):
    """``pack_linear_int8`` on the device: (qweight int8 [N, K], scale [N, 1] in W's dtype)
    (shard_compile.py:170-178)."""
    dev = _check_dev(W)
    if W.dim() != 2 or W.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError(f"W must be a 2D bf16 / fp16 / fp32 tensor, got {W.dtype} {tuple(W.shape)}")
    if W.stride(1) != 1:
        W = W.contiguous()
    N, K = W.shape
    q = torch.empty((N, K), dtype=torch.int8, device=dev)
    scale = torch.empty((N, 1), dtype=W.dtype, device=dev)
    with torch.cuda.device(dev):
        call("imq_pack_w8", _ptr(W), W.stride(0), dtype_code(W.dtype), N, K, _ptr(q), q.stride(0), _ptr(scale),
             scale.stride(0), _stream(dev))
    return q, scale


# ---------------------------------------------------------------------------------------------
# fused dequant linears
# ---------------------------------------------------------------------------------------------
def _linear_g(fn: str, codes_per_byte: int, x, qweight, group_size: int, sz, out=None):
    scale, zero = sz
    dev = _check_dev(x, qweight, scale, zero)
    _check_packed(qweight)
    x = _rows2d(x)
    Kpad = qweight.shape[1] * codes_per_byte
    if x.shape[1] != Kpad:
        x = torch.nn.functional.pad(x, (0, Kpad - x.shape[1])).contiguous()
    M = x.shape[0]
    N = qweight.shape[0]
    ng = Kpad // group_size
    if Kpad % group_size or tuple(scale.shape) != (N, ng) or tuple(zero.shape) != (N, ng):
        raise ValueError(f"scale/zero must be [{N}, {ng}] for K_pad={Kpad}, group={group_size}; "
                         f"got {tuple(scale.shape)} / {tuple(zero.shape)}")
    if out is not None and (tuple(out.shape) != (M, N) or out.dtype != torch.bfloat16 or out.stride(1) != 1):
        raise ValueError("out must be a bf16 [M, N] tensor with unit column stride")
    y = out if out is not None else torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    with torch.cuda.device(dev):
        if fn == "imq_linear_w4":
            # this call's own need (0 for the decode kernels that keep their partials in the
            # workgroup), not the shape-only bound over all formats
            need = int(_lib.lib().imq_linear_w4_workspace_bytes(
                M, Kpad, N, group_size, qweight.stride(0), x.stride(0), scale.stride(0), scale.stride(1),
                dtype_code(scale.dtype), zero.stride(0), zero.stride(1), dtype_code(zero.dtype)))
            w = _scratch(dev, need)
            ws, wsb = (0, 0) if w is None else (w.data_ptr(), w.numel())
        else:
            ws, wsb = _workspace(dev, M, N, Kpad)
        call(fn, _ptr(x), x.stride(0), M, Kpad, _ptr(qweight), qweight.stride(0), _ptr(scale), scale.stride(0),
             scale.stride(1), dtype_code(scale.dtype), _ptr(zero), zero.stride(0), zero.stride(1),
             dtype_code(zero.dtype), N, group_size, _ptr(y), y.stride(0), ws, wsb, _stream(dev))
    return y


def linear_w4(x, qweight, group_size: int, sz, out=None):
    """``op(x[M,Kpad] bf16, qweight u8[N,Kpad/2], group, (scale, zero)) -> y[M,N] bf16``: the
    signature of the op returned by the reference's _w4a16_triton_op (worker_quant.py:1180-1217)."""
    return _linear_g("imq_linear_w4", 2, x, qweight, group_size, sz, out)


def linear_w4_tiled(x, qweight_tiled, group_size: int, sz, out=None):
    """``linear_w4`` on int4 weights in the line-tiled layout (``line_tile``): the same results
    bit for bit. ``qweight_tiled`` is the dense u8 [N, Kpad/2] tiled array (N a multiple of 16,
    Kpad of 256, groups of 128); shapes no tiled-layout kernel takes raise ImqError."""
    if group_size != 128:
        raise ValueError("line-tiled int4 weights take groups of 128")
    if not qweight_tiled.is_contiguous():
        raise ValueError("the line-tiled weight array must be dense")
    return _linear_g("imq_linear_w4_tiled", 2, x, qweight_tiled, group_size, sz, out)


def linear_w2_tiled(x, qweight_tiled, group_size: int, sz, out=None):
    """``linear_w2`` on int2 weights in the line-tiled layout (``line_tile``): the dense u8
    [N, Kpad/4] tiled array (N a multiple of 16, Kpad of 512, groups of 64)."""
    if group_size != 64:
        raise ValueError("line-tiled int2 weights take groups of 64")
    if not qweight_tiled.is_contiguous():
        raise ValueError("the line-tiled weight array must be dense")
    return _linear_g("imq_linear_w2_tiled", 4, x, qweight_tiled, group_size, sz, out)


def _tile_shape_check(N: int, row_bytes: int):
    if N % 16 or row_bytes % 128:
        raise ValueError(f"the line-tiled layout needs N % 16 == 0 and row bytes % 128 == 0, got N={N}, "
                         f"row bytes={row_bytes}")


def line_tile(qweight, out=None):
    """Row-layout packed weight [N, row_bytes] (u8 int4 / int2 codes, or int8) -> the line-tiled
    layout of the same dtype (a new dense array, or ``out``): in 16-row tile t the 2 KiB block of
    line-step l holds, in slot 64 h + s, 16-byte piece 4 (((s >> 3) & 1) ^ h) + (s >> 4) of tile
    row 8 h + (s & 7). No counterpart in the reference."""
    if qweight.dtype == torch.int8:
        return line_tile(qweight.view(torch.uint8), None if out is None else out.view(torch.uint8)).view(torch.int8)
    dev = _check_dev(qweight)
    _check_packed(qweight)
    N, KB = qweight.shape
    _tile_shape_check(N, KB)
    t = out if out is not None else torch.empty((N, KB), dtype=torch.uint8, device=dev)
    if tuple(t.shape) != (N, KB) or t.dtype != torch.uint8 or not t.is_contiguous():
        raise ValueError("out must be a dense u8 array of qweight's shape")
    with torch.cuda.device(dev):
        call("imq_line_tile", _ptr(qweight), qweight.stride(0), N, KB, _ptr(t), _stream(dev))
    return t


def line_untile(qweight_tiled, out=None):
    """Inverse of ``line_tile``: the row-layout [N, row_bytes] array (new, or ``out``)."""
    if qweight_tiled.dtype == torch.int8:
        return line_untile(qweight_tiled.view(torch.uint8),
                           None if out is None else out.view(torch.uint8)).view(torch.int8)
    dev = _check_dev(qweight_tiled)
    _check_packed(qweight_tiled)
    if not qweight_tiled.is_contiguous():
        raise ValueError("the line-tiled weight array must be dense")
    N, KB = qweight_tiled.shape
    _tile_shape_check(N, KB)
    r = out if out is not None else torch.empty((N, KB), dtype=torch.uint8, device=dev)
    if tuple(r.shape) != (N, KB) or r.dtype != torch.uint8 or r.stride(1) != 1:
        raise ValueError("out must be a u8 array of qweight's shape with unit column stride")
    with torch.cuda.device(dev):
        call("imq_line_untile", _ptr(qweight_tiled), N, KB, _ptr(r), r.stride(0), _stream(dev))
    return r


def linear_w8_tiled(x, qweight_tiled, scale, out=None):
    """``linear_w8`` on int8 weights in the line-tiled layout (``line_tile``): the dense int8 [N, K]
    tiled array (N a multiple of 16, K of 128); the same results bit for bit."""
    dev = _check_dev(x, qweight_tiled, scale)
    _check_packed(qweight_tiled, torch.int8)
    if not qweight_tiled.is_contiguous():
        raise ValueError("the line-tiled weight array must be dense")
    x = _rows2d(x)
    M, K = x.shape
    N = qweight_tiled.shape[0]
    if qweight_tiled.shape[1] != K:
        raise ValueError(f"x has {K} columns, qweight {qweight_tiled.shape[1]}")
    y = out if out is not None else torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    with torch.cuda.device(dev):
        ws, wsb = _workspace(dev, M, N, K)
        call("imq_linear_w8_tiled", _ptr(x), x.stride(0), M, K, _ptr(qweight_tiled), qweight_tiled.stride(0),
             _ptr(scale), scale.stride(0), dtype_code(scale.dtype), N, _ptr(y), y.stride(0), ws, wsb, _stream(dev))
    return y


def linear_w2(x, qweight, group_size: int, sz, out=None):
    """int2 twin (worker_quant.py:1876-1910): qweight u8 [N, Kpad/4]."""
    return _linear_g("imq_linear_w2", 4, x, qweight, group_size, sz, out)


def linear_w8(x, qweight, scale, out=None):
    """``op(x, qweight int8[N,K], scale[N,1]) -> y bf16 [M,N]`` (worker_quant.py:1022-1048)."""
    dev = _check_dev(x, qweight, scale)
    _check_packed(qweight, torch.int8)
    x = _rows2d(x)
    M, K = x.shape
    N = qweight.shape[0]
    if qweight.shape[1] != K:
        raise ValueError(f"x has {K} columns, qweight {qweight.shape[1]}")
    y = out if out is not None else torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    with torch.cuda.device(dev):
        ws, wsb = _workspace(dev, M, N, K)
        call("imq_linear_w8", _ptr(x), x.stride(0), M, K, _ptr(qweight), qweight.stride(0), _ptr(scale),
             scale.stride(0), dtype_code(scale.dtype), N, _ptr(y), y.stride(0), ws, wsb, _stream(dev))
    return y


# ---------------------------------------------------------------------------------------------
# fused MoE experts
# ---------------------------------------------------------------------------------------------
def moe_rows_w4(x, eid, q, scale, zero, group_size: int, in_features: int, *, check_ids: bool = True):
    """``op(x[B,Kin], eid[B], q[E,N,Kpad/2], scale, zero, group, in_features) -> y[B,N] bf16``:
    the op returned by the reference's _w4a16_moe_op (worker_quant.py:1452-1487). Expert ids
    outside [0, E) raise ValueError (``check_ids``; not checked under graph capture)."""
    dev = _check_dev(x, eid, q, scale, zero)
    _check_packed(q)
    if scale.dtype != zero.dtype:
        zero = zero.to(scale.dtype)
    x = _rows2d(x)
    Kpad = q.shape[2] * 2
    if x.shape[1] != Kpad:
        x = torch.nn.functional.pad(x, (0, Kpad - x.shape[1])).contiguous()
    eid = eid.to(torch.int32).contiguous()
    B = x.shape[0]
    E, N = q.shape[0], q.shape[1]
    if check_ids:
        _check_expert_ids(eid, E)
    ng = Kpad // group_size
    if tuple(scale.shape) != (E, N, ng) or tuple(zero.shape) != (E, N, ng) or eid.numel() != B:
        raise ValueError("scale/zero must be [E, N, K_pad/group] and eid [B]")
    y = torch.empty((B, N), dtype=torch.bfloat16, device=dev)
    with torch.cuda.device(dev):
        call("imq_moe_rows_w4", _ptr(x), x.stride(0), B, Kpad, _ptr(eid), E, _ptr(q), q.stride(0), q.stride(1),
             _ptr(scale), scale.stride(0), scale.stride(1), scale.stride(2), _ptr(zero), zero.stride(0),
             zero.stride(1), zero.stride(2), dtype_code(scale.dtype), N, group_size, _ptr(y), y.stride(0),
             _stream(dev))
    return y


def moe_workspace_bytes(T: int, top_k: int, E: int, H: int, I: int, group_size: int) -> int:
    return int(_lib.lib().imq_moe_workspace_bytes(T, top_k, E, H, I, group_size))


_ACT = {"silu_glu": 0, "gptoss": 1}


def moe_experts_w4(hidden, topk_idx, topk_w, gu, dn, group_size: int, workspace=None, *, act: str = "silu_glu",
                   gu_bias=None, dn_bias=None, alpha: float = 1.702, limit: float = 7.0, check_ids: bool = True):
    """One MoE layer's experts forward: ``out[t] = sum_j w[t,j] * (down_e(act(gate_up_e(x_t))) + b_dn[e])``.

    ``gu`` / ``dn`` are (qweight, scale, zero, in_features) of the gate_up [E, 2I, K1/2] and down
    [E, H, K2/2] int4 stacks, K1 / K2 the kernel layout's padded K (any multiple of the group
    >= in_features; columns past in_features carry zero codes and zero scales).

    ``act="silu_glu"``: rows [gate | up], h = silu(gate) * up -- the transformers eager experts
    loop (modeling_olmoe.py:301-325) as fused by worker_quant.py:2167-2191. ``act="gptoss"``:
    rows interleaved (gate 2i, up 2i+1) with per-expert biases ``gu_bias`` [E, 2I] and ``dn_bias``
    [E, H] and gpt-oss's clamped GLU (worker_quant.py:2280-2314).

    Routing ids outside [0, E) raise ValueError, as the reference's eager loop does
    (``check_ids``: one device-to-host read per call, skipped under graph capture). Without a
    ``workspace`` the call uses the cached per-(device, stream) workspace."""
    gq, gs, gz, H = gu
    dq, ds, dz, I = dn
    dev = _check_dev(hidden, topk_idx, topk_w, gq, gs, gz, dq, ds, dz)
    for t in (gq, dq):
        _check_packed(t)
    if act not in _ACT:
        raise ValueError(f"act must be one of {sorted(_ACT)} (got {act!r})")
    T = hidden.shape[0]
    k = topk_idx.shape[1]
    E = gq.shape[0]
    if gq.shape[1] != 2 * I or dq.shape[1] != H:
        raise ValueError("gate_up must be [E, 2I, .] and down [E, H, .]")
    sdt = gs.dtype
    gz = gz if gz.dtype == sdt else gz.to(sdt)
    ds = ds if ds.dtype == sdt else ds.to(sdt)
    dz = dz if dz.dtype == sdt else dz.to(sdt)
    for t in (gs, gz, ds, dz):
        if t.stride(2) != 1:
            raise ValueError("scale/zero need a unit last stride")
    if gs.stride() != gz.stride() or ds.stride() != dz.stride():
        gs, gz = gs.contiguous(), gz.contiguous()
        ds, dz = ds.contiguous(), dz.contiguous()
    bdt = None
    biases = []
    for b, rows in ((gu_bias, 2 * I), (dn_bias, H)):
        if b is not None:
            _check_dev(hidden, b)
            if b.dim() != 2 or b.shape[0] != E or b.shape[1] != rows:
                raise ValueError(f"bias must be [E, {rows}] (got {tuple(b.shape)})")
            if b.stride(1) != 1:
                b = b.contiguous()
            if bdt is not None and b.dtype != bdt:
                b = b.to(bdt)
            bdt = b.dtype
        biases.append(b)
    gb, db = biases
    gK, dK = gq.shape[2] * 2, dq.shape[2] * 2
    x = _rows2d(hidden)
    if x.shape[1] != gK and (x.shape[1] != H or H % 8 or (T > 16 and (H % 64 or gK > 40 * 128))):
        # rows of exactly H columns (H % 8 == 0) are read as zero past H by the decode and line
        # kernels; past 16 tokens the register-B GEMM skips the K steps past H when H is a
        # multiple of its 64-column step (and K within its 40 groups): other rows get one
        # zero-padded copy, cheaper than every pass reading them clamped
        x = torch.nn.functional.pad(x[:, :H], (0, gK - H)).contiguous()
    # int64 ids (torch's top-k) and int32 ids are read by the kernels as they are
    idx = topk_idx if topk_idx.dtype in (torch.int64, torch.int32) else topk_idx.to(torch.int64)
    idx = idx.contiguous()
    if check_ids:
        _check_expert_ids(idx, E)
    w = topk_w.to(torch.bfloat16).contiguous()
    need = moe_workspace_bytes(T, k, E, H, I, group_size)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = _scratch(dev, max(need, 1))
    out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    with torch.cuda.device(dev):
        call("imq_moe_experts_w4_ex", _ptr(x), x.stride(0), T, H, k, _ptr(idx),
             _lib.IMQ_DT_I64 if idx.dtype == torch.int64 else _lib.IMQ_DT_I32, _ptr(w), E,
             _ptr(gq), gq.stride(0), gq.stride(1), gK, _ptr(gs), _ptr(gz), gs.stride(0), gs.stride(1), I,
             _ptr(dq), dq.stride(0), dq.stride(1), dK, _ptr(ds), _ptr(dz), ds.stride(0), ds.stride(1),
             dtype_code(sdt), group_size,
             _ptr(gb) if gb is not None else None, gb.stride(0) if gb is not None else 0,
             _ptr(db) if db is not None else None, db.stride(0) if db is not None else 0,
             dtype_code(bdt) if bdt is not None else 0, _ACT[act], float(alpha), float(limit),
             _ptr(out), out.stride(0), _ptr(workspace), workspace.numel() * workspace.element_size(),
             _stream(dev))
    return out
