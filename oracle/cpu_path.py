"""The reference's CPU execution path for the quantized linears, restated in torch
(TEST / BENCH BASELINE ONLY -- the timed ``cpu_baseline`` comparator, never the product path).

* int4 fused CPU op: torch tinygemm ``_convert_weight_to_int4pack_for_cpu(q.int32 [N, K_pad], 8)``
  once, then ``_weight_int4pack_mm_for_cpu(x_bf16, mat2, G, sz)`` with
  ``sz = stack(S, (8 - z) * S)`` -> ``[ng, N, 2]`` bf16 (worker_quant.py:732-759).
* naive rule: rows < 16 -> ``F.linear(x, _dequant(x.dtype))``; rows >= 16 -> fp32 dequant +
  fp32 GEMM (worker_quant.py:847-853; int8 411-417).
* threads: physical cores clamped to [1, 128], interop min(2, n) (tune_cpu_threads,
  worker_quant.py:283-330).
The tinygemm dequant is (q - 8) * S + bf16((8 - z) * S), not (q - z) * S: third-party op, parity
unpinned beyond the reference's own rel < 0.05 self-check (worker_quant.py:760-767); it is only a
timing comparator here.

Pins (tests/test_oracle.py): ``dequant_g`` is bit-identical to oracle.quant's dequant for int4 /
int2 in bf16 / fp16 / fp32; ``naive_linear`` (both row branches), ``naive_linear_int8`` and
``moe_eager_cpu`` agree with the oracle's pinned products and eager MoE loop within their bf16
roundings.
"""
from __future__ import annotations

import contextlib
import os


def tune_cpu_threads() -> int:
    import torch
    n = 0
    for ev in ("OMP_NUM_THREADS", "MKL_NUM_THREADS", "TORCH_NUM_THREADS"):
        v = os.environ.get(ev)
        if v and v.strip().isdigit():
            n = int(v.strip())
            break
    if not n:
        try:
            import psutil
            n = psutil.cpu_count(logical=False) or 0
        except Exception:
            n = 0
        if not n:
            n = os.cpu_count() or 1
    n = max(1, min(int(n), 128))
    torch.set_num_threads(n)
    with contextlib.suppress(Exception):
        torch.set_num_interop_threads(min(2, n))
    return torch.get_num_threads()


def _codes_int4(qweight):
    import torch
    lo = (qweight & 0x0F)
    hi = (qweight >> 4)
    return torch.stack((lo, hi), dim=2).reshape(qweight.shape[0], -1)


def tinygemm_prepare(qweight, scale, zero, group_size: int):
    """(mat2, sz) for the CPU tinygemm op, built from the group-wise asymmetric int4 format with no
    re-quantization (worker_quant.py:743-759)."""
    import torch
    aten = torch.ops.aten
    out = qweight.shape[0]
    q = _codes_int4(qweight)
    ng = scale.shape[1]
    S = scale.float()
    Z = (8.0 - zero.float()) * S
    sz = torch.cat([S.reshape(out, ng, 1), Z.reshape(out, ng, 1)], dim=2)
    sz = sz.transpose(0, 1).contiguous().to(torch.bfloat16)
    mat2 = aten._convert_weight_to_int4pack_for_cpu(q.to(torch.int32).contiguous(), 8)
    return mat2, sz


def tinygemm_linear(x, mat2, group_size: int, sz):
    import torch
    return torch.ops.aten._weight_int4pack_mm_for_cpu(x, mat2, group_size, sz)


def dequant_g(qweight, scale, zero, in_features: int, group_size: int, dtype, bits: int):
    """The reference `_dequant(dtype)` in torch (worker_quant.py:638-648, 1652-1664)."""
    import torch
    out = qweight.shape[0]
    if bits == 4:
        q = _codes_int4(qweight).to(torch.int16)
    else:
        q = torch.stack([((qweight >> (2 * i)) & 0x3) for i in range(4)], dim=2).reshape(out, -1).to(torch.int16)
    ng = scale.shape[1]
    qf = q.reshape(out, ng, group_size).to(dtype)
    w = (qf - zero.to(dtype).unsqueeze(2)) * scale.to(dtype).unsqueeze(2)
    return w.reshape(out, ng * group_size)[:, :in_features].contiguous()


def naive_linear(x, qweight, scale, zero, in_features: int, group_size: int, bits: int = 4):
    """The naive forward tail of QuantLinear4/2 on CPU (worker_quant.py:847-853)."""
    import torch
    import torch.nn.functional as F
    rows = x.numel() // x.shape[-1]
    if rows >= 16:
        y = F.linear(x.to(torch.float32), dequant_g(qweight, scale, zero, in_features, group_size,
                                                    torch.float32, bits))
        return y.to(x.dtype)
    return F.linear(x, dequant_g(qweight, scale, zero, in_features, group_size, x.dtype, bits))


def naive_linear_int8(x, qweight, scale):
    """QuantLinear.forward CPU tail (worker_quant.py:411-417 rows >= 16; 439-440 otherwise)."""
    import torch
    import torch.nn.functional as F
    rows = x.numel() // x.shape[-1]
    if rows >= 16:
        w = qweight.to(torch.float32) * scale.to(torch.float32)
        return F.linear(x.to(torch.float32), w).to(x.dtype)
    return F.linear(x, qweight.to(x.dtype) * scale)


def moe_eager_cpu(hidden, topk_idx, topk_w, gu, dn, group_size: int):
    """transformers eager experts loop over per-expert bf16 dequant (modeling_olmoe.py:301-325 over
    Packed4Tensor3D.__getitem__, worker_quant.py:2033-2043). gu/dn = (q, s, z, in_features)."""
    import torch
    import torch.nn.functional as F
    gq, gs, gz, H = gu
    dq, ds, dz, I = dn
    E = gq.shape[0]
    final = torch.zeros_like(hidden)
    mask = F.one_hot(topk_idx, num_classes=E).permute(2, 1, 0)
    hit = torch.greater(mask.sum(dim=(-1, -2)), 0).nonzero()
    for e in hit:
        e = int(e[0])
        pos, tok = torch.where(mask[e])
        cur = hidden[tok]
        wg = dequant_g(gq[e], gs[e], gz[e], H, group_size, hidden.dtype, 4)
        gate, up = F.linear(cur, wg).chunk(2, dim=-1)
        h = F.silu(gate) * up
        wd = dequant_g(dq[e], ds[e], dz[e], I, group_size, hidden.dtype, 4)
        o = F.linear(h, wd) * topk_w[tok, pos, None]
        final.index_add_(0, tok, o.to(final.dtype))
    return final
