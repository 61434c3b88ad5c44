"""Reference MoE-expert semantics (TEST ORACLE ONLY).

Follows the transformers eager experts loop that the reference falls back to and self-checks
against (container transformers 5.15.0 ``models/olmoe/modeling_olmoe.py:301-325``; restated by
the reference in bench_moe_w4a16.py:132-149) and the reference's fused decode form
(worker_quant.py:2167-2191: ``repeat_interleave`` -> gate_up -> ``chunk(2)`` -> ``act(gate)*up``
-> down -> T==1 matvec ``w @ zb`` / T>1 ``index_add_``).

Pins: ``moe_eager_bf16`` is checked against a live ``OlmoeExperts`` module from the installed
transformers (a third-party implementation) fed the oracle's dequantized weights;
``moe_exact`` against ``moe_eager_bf16`` (agreement to bf16 noise) and a brute-force single-token
case; ``moe_exact_grouped`` against ``moe_exact``; ``route_topk`` against ``OlmoeTopKRouter``;
``gptoss_exact`` against a live ``GptOssExperts`` module (float64, in-major weights = the
transpose of the oracle's) and against hand-evaluated activation cases (clamp on and off).
"""
from __future__ import annotations

import numpy as np

from .quant import round_to

F32 = np.float32


def silu64(v):
    v = np.asarray(v, np.float64)
    return v / (1.0 + np.exp(-v))


def moe_exact(x, idx, wts, Wgu, Wdn) -> np.ndarray:
    """float64 ``out[t] = sum_j w[t,j] * Wdn[e] @ (silu(gate) * up)`` with ``[gate | up] = Wgu[e] @ x[t]``,
    e = idx[t,j] (worker_quant.py:2175 gate-then-up order). Wgu [E, 2I, H], Wdn [E, H, I] are the
    dequantized bf16 expert weights; no intermediate rounding."""
    x = np.asarray(x, np.float64)
    T, H = x.shape
    I = Wgu.shape[1] // 2
    out = np.zeros((T, Wdn.shape[1]), np.float64)
    for t in range(T):
        for j in range(idx.shape[1]):
            e = int(idx[t, j])
            g = np.asarray(Wgu[e], np.float64) @ x[t]
            h = silu64(g[:I]) * g[I:]
            out[t] += float(wts[t, j]) * (np.asarray(Wdn[e], np.float64) @ h)
    return out


def moe_exact_grouped(x, idx, wts, Wgu, Wdn) -> np.ndarray:
    """``moe_exact`` evaluated expert by expert (one float64 product per hit expert over all its
    routed tokens) -- the same sum, reordered; fast enough for T in the hundreds."""
    x = np.asarray(x, np.float64)
    T, H = x.shape
    I = Wgu.shape[1] // 2
    idx = np.asarray(idx)
    w = np.asarray(wts, np.float64)
    out = np.zeros((T, Wdn.shape[1]), np.float64)
    for e in np.unique(idx):
        tok, slot = np.nonzero(idx == e)
        g = x[tok] @ np.asarray(Wgu[e], np.float64).T
        h = silu64(g[:, :I]) * g[:, I:]
        y = h @ np.asarray(Wdn[e], np.float64).T
        np.add.at(out, tok, w[tok, slot][:, None] * y)
    return out


def moe_eager_bf16(x, idx, wts, Wgu, Wdn) -> np.ndarray:
    """The eager experts loop with its bf16 roundings (modeling_olmoe.py:301-325): experts in
    ascending id order; per expert, its (slot, token) pairs in ``torch.where`` order; each
    F.linear result rounded to bf16 (the fp32-accumulated GEMM is modelled exactly), ``silu`` and
    ``*`` rounded to bf16, the routing weight product rounded to bf16, and ``index_add_`` adding
    into the bf16 output one contribution at a time."""
    x = np.asarray(x, F32)
    T, H = x.shape
    E = Wgu.shape[0]
    I = Wgu.shape[1] // 2
    k = idx.shape[1]
    final = np.zeros((T, Wdn.shape[1]), F32)
    for e in range(E):
        pos, tok = np.nonzero((np.asarray(idx) == e).T)   # expert_mask[e] is [k, T]
        if pos.size == 0:
            continue
        order = np.lexsort((tok, pos))
        pos, tok = pos[order], tok[order]
        cur = x[tok].astype(np.float64)
        gu = round_to(cur @ np.asarray(Wgu[e], np.float64).T, "bf16")
        gate, up = gu[:, :I], gu[:, I:]
        act = round_to(silu64(gate), "bf16")
        h = round_to(act.astype(np.float64) * up, "bf16")
        dn = round_to(h.astype(np.float64) @ np.asarray(Wdn[e], np.float64).T, "bf16")
        w = np.asarray(wts, F32)[tok, pos][:, None]
        dn = round_to(dn.astype(np.float64) * w, "bf16")
        for r in range(tok.size):
            final[tok[r]] = round_to(final[tok[r]] + dn[r], "bf16")
    return final


def route_topk(logits, k: int, out_dt: str = "bf16"):
    """OLMoE router on given logits (modeling_olmoe.py:336-346): softmax in fp32, top-k,
    renormalize (norm_topk_prob), cast to the logits dtype (bf16 for a bf16 model). Returns
    (idx int64 [T,k], weights as out_dt values [T,k])."""
    lg = np.asarray(logits, F32)
    m = lg.max(axis=1, keepdims=True)
    p = np.exp((lg - m).astype(np.float64))
    p = (p / p.sum(axis=1, keepdims=True)).astype(F32)
    idx = np.argsort(-p, axis=1, kind="stable")[:, :k]
    top = np.take_along_axis(p, idx, axis=1)
    top = (top / top.sum(axis=1, keepdims=True)).astype(F32)
    return idx.astype(np.int64), round_to(top, out_dt)


def gptoss_glu64(gate, up, alpha: float = 1.702, limit: float = 7.0):
    """gpt-oss's clamped GLU in float64 (worker_quant.py:2301-2303): gate <= limit, up in
    [-limit, limit], (up + 1) * gate * sigmoid(alpha * gate)."""
    g = np.minimum(np.asarray(gate, np.float64), limit)
    u = np.clip(np.asarray(up, np.float64), -limit, limit)
    return (u + 1.0) * (g / (1.0 + np.exp(-alpha * g)))


def gptoss_exact(x, idx, wts, Wgu, bgu, Wdn, bdn, alpha: float = 1.702, limit: float = 7.0) -> np.ndarray:
    """float64 gpt-oss experts forward (worker_quant.py:2292-2309) over transpose-packed weights:
    ``gu = Wgu[e] @ x[t] + bgu[e]`` with Wgu [E, 2I, H] (rows interleaved gate 2i / up 2i+1),
    ``h = glu(gu[::2], gu[1::2])``, ``out[t] += w[t,j] * (Wdn[e] @ h + bdn[e])`` with Wdn [E, H, I],
    evaluated expert by expert; no intermediate rounding."""
    x = np.asarray(x, np.float64)
    T, H = x.shape
    idx = np.asarray(idx)
    w = np.asarray(wts, np.float64)
    out = np.zeros((T, np.asarray(Wdn).shape[1]), np.float64)
    for e in np.unique(idx):
        tok, slot = np.nonzero(idx == e)
        gu = x[tok] @ np.asarray(Wgu[e], np.float64).T + np.asarray(bgu[e], np.float64)
        h = gptoss_glu64(gu[:, 0::2], gu[:, 1::2], alpha, limit)
        y = h @ np.asarray(Wdn[e], np.float64).T + np.asarray(bdn[e], np.float64)
        np.add.at(out, tok, w[tok, slot][:, None] * y)
    return out
