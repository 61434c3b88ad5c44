"""Synthetic workloads of the benchmark configurations (random weights of the named shapes,
RTN-packed with this package's packers; there is no network for checkpoints).

C1  single int4 g128 linear 1x4096 -> 4096
C2  Llama-3-8B decode stack: 32 layers x {qkv 4096->6144, o 4096->4096, gate_up 4096->28672,
    down 14336->4096}, int4 g128 asymmetric, bf16 scale/zero, M in {1, 4, 16}
C3  int2 g64 70B shapes 8192->28672 and 28672->8192, fp16 scale ~U(0.005,0.05), zero ~U(0,3)
C4  prefill int4 g128 / int8 per-row, 4096->14336 and 14336->4096, M in {512, 2048}
C5  OLMoE experts: E=64, top-8, H=2048, I=1024, int4 g128, T in {1, 16, 256}
"""
from __future__ import annotations

from dataclasses import dataclass

from .shard_compile import pack_linear_int4, pack_linear_int4_3d, pack_linear_int8

LLAMA8B_PROJ = (("qkv", 4096, 6144), ("o", 4096, 4096), ("gate_up", 4096, 28672), ("down", 14336, 4096))


@dataclass
class Linear4:
    name: str
    q: "object"
    s: "object"
    z: "object"
    K: int
    N: int
    G: int = 128

    def algorithmic_bytes(self, M: int) -> int:
        ng = self.s.shape[1]
        return (self.N * self.q.shape[1] + self.N * ng * (self.s.element_size() + self.z.element_size())
                + M * self.K * 2 + M * self.N * 2)


def _gen(seed: int, dev):
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return g


def rtn_int4_linear(N: int, K: int, seed: int, dev, G: int = 128, std: float = 0.02, name: str = "") -> Linear4:
    import torch
    W = (torch.randn(N, K, generator=_gen(seed, dev), device=dev) * std).to(torch.bfloat16)
    q, s, z, _ = pack_linear_int4(W, G)
    del W
    return Linear4(name, q, s, z, K, N, G)


def llama8b_stack(dev, layers: int = 32):
    """C2 weights: W ~ N(0, 0.02), seed 1000 + 4*l + p, RTN int4 g128, bf16 s/z."""
    out = []
    for l in range(layers):
        for p, (name, K, N) in enumerate(LLAMA8B_PROJ):
            out.append(rtn_int4_linear(N, K, 1000 + 4 * l + p, dev, name=f"L{l}.{name}"))
    return out


def activations(M: int, K: int, seed: int, dev):
    import torch
    return torch.randn(M, K, generator=_gen(seed, dev), device=dev).to(torch.bfloat16)


def int2_random_linear(N: int, K: int, seed: int, dev, G: int = 64):
    """C3: codes ~ U{0..3} packed 4/byte, fp16 scale ~ U(0.005, 0.05), fp16 zero ~ U(0, 3)."""
    import torch
    g = _gen(seed, dev)
    ng = (K + G - 1) // G
    q = torch.randint(0, 256, (N, ng * G // 4), generator=g, device=dev, dtype=torch.uint8)
    s = (torch.rand(N, ng, generator=g, device=dev) * 0.045 + 0.005).to(torch.float16)
    z = (torch.rand(N, ng, generator=g, device=dev) * 3.0).to(torch.float16)
    return q, s, z


def int8_linear(N: int, K: int, seed: int, dev, dtype=None, std: float = 0.02):
    """C4 int8: RTN per-row symmetric of fp16 W -> fp16 scale."""
    import torch
    dtype = dtype or torch.float16
    W = (torch.randn(N, K, generator=_gen(seed, dev), device=dev) * std).to(dtype)
    q, s = pack_linear_int8(W)
    return q, s


def olmoe_layer(dev, seed: int = 3000, E: int = 64, H: int = 2048, I: int = 1024, G: int = 128):
    """C5 experts: gate_up [E, 2I, H], down [E, H, I], RTN int4 g128 of N(0, 0.02), bf16 s/z."""
    import torch
    Wg = (torch.randn(E, 2 * I, H, generator=_gen(seed, dev), device=dev) * 0.02).to(torch.bfloat16)
    gq, gs, gz, _, _ = pack_linear_int4_3d(Wg, G)
    del Wg
    Wd = (torch.randn(E, H, I, generator=_gen(seed + 500, dev), device=dev) * 0.02).to(torch.bfloat16)
    dq, ds, dz, _, _ = pack_linear_int4_3d(Wd, G)
    del Wd
    return (gq, gs, gz, H), (dq, ds, dz, I)


def olmoe_routing(T: int, dev, E: int = 64, k: int = 8, seed: int = 4):
    """Router logits ~ N(0,1) [T, E] -> softmax(fp32) -> top-k -> renormalize -> bf16."""
    import torch
    logits = torch.randn(T, E, generator=_gen(seed, dev), device=dev)
    p = torch.softmax(logits, dim=-1, dtype=torch.float32)
    top, idx = torch.topk(p, k, dim=-1)
    top = top / top.sum(dim=-1, keepdim=True)
    return idx, top.to(torch.bfloat16)


def gptoss_layer(dev, seed: int = 5000, E: int = 32, H: int = 2880, I: int = 2880, G: int = 128):
    """gpt-oss-20b experts: gate_up / down transpose-packed to [E, 2I, H] / [E, H, I] (rows of
    gate_up interleaved gate / up), RTN int4 g128 of N(0, 0.02), bf16 s/z and per-expert bf16
    biases N(0, 0.02); returned in the fused kernels' layout (Packed4Tensor3D._kernel_tensors:
    K 2880 padded to 3072 with zero codes and scales)."""
    import torch
    from . import worker_quant as wq
    PT = wq._packed4_3d_cls()
    Wg = (torch.randn(E, 2 * I, H, generator=_gen(seed, dev), device=dev) * 0.02).to(torch.bfloat16)
    gq, gs, gz, _, _ = pack_linear_int4_3d(Wg, G)
    del Wg
    Wd = (torch.randn(E, H, I, generator=_gen(seed + 500, dev), device=dev) * 0.02).to(torch.bfloat16)
    dq, ds, dz, _, _ = pack_linear_int4_3d(Wd, G)
    del Wd
    gh, dh = PT(gq, gs, gz, H, G), PT(dq, ds, dz, I, G)
    g = _gen(seed + 900, dev)
    bgu = (torch.randn(E, 2 * I, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    bdn = (torch.randn(E, H, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    return (*gh._kernel_tensors(), H), (*dh._kernel_tensors(), I), bgu, bdn
