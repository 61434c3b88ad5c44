"""GPTQ-calibrated int2 packing on the GPU: the per-Linear pieces of the reference's calibrated
int2 packer (gptq_pack.py:57-189), with the column-by-column solve on this library's HIP solver.

Names and semantics follow the reference:

* ``_STAGES`` -- the sub-layer order the Hessians are collected in (gptq_pack.py:57);
* ``_find_params(Wg, grid, maxshrink)`` -- the group search: scale / zero on the asymmetric
  0..3 grid, best of ``int(maxshrink * grid)`` range-shrink candidates by sum |dq - w|^2.4
  (gptq_pack.py:78-100), one HIP thread per row;
* ``_GPTQ(linear, device)`` with ``add_batch(x)`` (gptq_pack.py:110-118: the running Hessian
  H = 2 / n sum x x^T, a plain GEMM in torch) and ``solve(group_size, grid, maxshrink, percdamp,
  blocksize=128)`` (gptq_pack.py:120-189): the Cholesky stage in torch.linalg (dead columns,
  damping, cholesky -> cholesky_inverse -> upper factor), then imq_gptq_int2_solve; the
  dequantized weight is written back into the Linear and (qweight crumbs, scale, zero) are
  returned in the RTN int2 packer's format, scale / zero in the weight's dtype.

The solver's arithmetic is float32 with every operation rounded on its own and sums in a fixed
order, so its output is identical to the host restatement of the same algorithm; against the
reference's own GPU run (torch reductions, torch.pow) a few codes can differ where two candidates
or two rounding sides tie within float error -- the reference likewise notes that its caches are
not byte-identical across boxes (gptq_pack.py:23-24). There is no CPU fallback: the solve needs
the HIP library (the reference's CPU branch is its own fp32 torch loop).

The calibrated compile driver (compile_int2_gptq: model streaming, calibration corpus, layer
forwards) stays in the reference; it calls exactly these pieces per Linear.
"""
from __future__ import annotations

from . import _lib
from .ops import _ptr, _stream, call

# gptq_pack.py:57, kept as data: each stage's Hessian is collected with the earlier stages of the
# layer already quantized.
_STAGES = (("q_proj", "k_proj", "v_proj"), ("o_proj",), ("gate_proj", "up_proj"), ("down_proj",))


def _need_gpu(t, what: str):
    if not t.is_cuda:
        raise RuntimeError(f"{what} runs on the HIP GPTQ solver: the tensor must be on a GPU (got {t.device})")


def _find_params(Wg, grid: int, maxshrink: float):
    """Group scale / zero of each row of Wg [out, g] (gptq_pack.py:78-100) -> fp32 (scale [out],
    zero [out]) on Wg's device."""
    import torch
    _need_gpu(Wg, "_find_params")
    W = Wg.detach().to(torch.float32).contiguous()
    rows, cols = W.shape
    s = torch.empty(rows, dtype=torch.float32, device=W.device)
    z = torch.empty_like(s)
    with torch.cuda.device(W.device):
        call("imq_gptq_int2_params", _ptr(W), W.stride(0), rows, cols, int(grid), float(maxshrink), _ptr(s), _ptr(z),
             _stream(W.device))
    return s, z


class _GPTQ:
    """One Linear's Hessian accumulator and solver (gptq_pack.py:103-189)."""

    def __init__(self, linear, device):
        import torch
        self.lin = linear
        self.dev = torch.device(device)
        self.in_f = int(linear.weight.shape[1])
        self.H = torch.zeros((self.in_f, self.in_f), dtype=torch.float32, device=self.dev)
        self.n = 0

    def add_batch(self, x) -> None:
        """H <- H n / (n + t) + (2 / (n + t)) x^T x for a batch of t rows (gptq_pack.py:110-118)."""
        import torch
        x = x.reshape(-1, self.in_f).to(self.dev, torch.float32)
        t = x.shape[0]
        self.H *= self.n / (self.n + t)
        self.n += t
        x = x * (2.0 / self.n) ** 0.5
        self.H += x.t() @ x

    def solve(self, group_size: int, grid: int, maxshrink: float, percdamp: float, blocksize: int = 128):
        """Quantize the Linear's weight against the collected Hessian. Returns (qweight uint8
        [out, in_pad / 4], scale [out, ng], zero [out, ng]) on the CPU, scale / zero in the weight
        dtype, and writes the dequantized weight back into the Linear (gptq_pack.py:120-189)."""
        import torch
        _need_gpu(self.H, "_GPTQ.solve")
        G = int(group_size)
        W = self.lin.weight.data.to(self.dev, torch.float32).clone()
        out, in_f = W.shape
        H = self.H
        self.H = None
        dead = torch.diag(H) == 0
        H[dead, dead] = 1.0
        W[:, dead] = 0.0
        damp = percdamp * torch.mean(torch.diag(H))
        idx = torch.arange(in_f, device=self.dev)
        H[idx, idx] += damp
        H = torch.linalg.cholesky(H)
        H = torch.cholesky_inverse(H)
        Hinv = torch.linalg.cholesky(H, upper=True).contiguous()
        del H
        ng = (in_f + G - 1) // G
        in_pad = ng * G
        q = torch.empty((out, in_pad // 4), dtype=torch.uint8, device=self.dev)
        scales = torch.empty((out, ng), dtype=torch.float32, device=self.dev)
        zeros = torch.empty_like(scales)
        DQ = torch.empty((out, in_f), dtype=torch.float32, device=self.dev)
        L = _lib.lib()
        nws = int(L.imq_gptq_int2_workspace_bytes(out, int(blocksize)))
        if nws < 0:
            raise ValueError(f"blocksize must lie in [1, 128] (got {blocksize})")
        ws = torch.empty(nws, dtype=torch.uint8, device=self.dev)
        with torch.cuda.device(self.dev):
            call("imq_gptq_int2_solve", _ptr(W), W.stride(0), out, in_f, _ptr(Hinv), Hinv.stride(0), G, int(grid),
                 float(maxshrink), int(blocksize), _ptr(q), q.stride(0), _ptr(scales), _ptr(zeros), scales.stride(0),
                 _ptr(DQ), DQ.stride(0), _ptr(ws), nws, _stream(self.dev))
        wdt = self.lin.weight.dtype
        self.lin.weight.data.copy_(DQ.to(wdt).to(self.lin.weight.device))
        del W, DQ, Hinv
        return q.cpu(), scales.to(wdt).cpu(), zeros.to(wdt).cpu()
