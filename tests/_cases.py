"""Seeded test-case builders shared by the CPU and GPU tests (inputs + oracle expectations)."""
from __future__ import annotations

import functools

import numpy as np

from oracle import quant as oq


def rng(seed: int):
    return np.random.default_rng(seed)


def bf16_normal(r, shape, std=1.0, dt="bf16"):
    return oq.round_to((r.standard_normal(shape) * std).astype(np.float32), dt)


@functools.lru_cache(maxsize=16)
def int4_case(N, K, G=128, seed=0, dt="bf16", wstd=0.02):
    """RTN int4 pack of W ~ N(0, wstd) (values in dtype dt), oracle dequant in bf16."""
    r = rng(seed)
    W = bf16_normal(r, (N, K), wstd, dt)
    q, s, z, in_f = oq.pack_linear_int4(W, G, dt)
    Wd = oq.dequant_int4(q, s, z, in_f, G, "bf16")
    return dict(W=W, q=q, s=s, z=z, in_f=in_f, G=G, dt=dt, Wd=Wd)


@functools.lru_cache(maxsize=16)
def int2_case(N, K, G=64, seed=0, dt="bf16", wstd=0.02):
    r = rng(seed)
    W = bf16_normal(r, (N, K), wstd, dt)
    q, s, z, in_f = oq.pack_linear_int2(W, G, dt)
    Wd = oq.dequant_int2(q, s, z, in_f, G, "bf16")
    return dict(W=W, q=q, s=s, z=z, in_f=in_f, G=G, dt=dt, Wd=Wd)


@functools.lru_cache(maxsize=16)
def int2_random_case(N, K, G=64, seed=2000, dt="fp16"):
    """BASELINE C3 generator: codes ~ U{0..3}, scale ~ U(0.005, 0.05), zero ~ U(0, 3) (non-integer),
    stored in dt."""
    r = rng(seed)
    ng = -(-K // G)
    codes = r.integers(0, 4, size=(N, ng * G), dtype=np.uint8)
    q = (codes[:, 0::4] | (codes[:, 1::4] << 2) | (codes[:, 2::4] << 4) | (codes[:, 3::4] << 6)).astype(np.uint8)
    s = oq.round_to(r.uniform(0.005, 0.05, size=(N, ng)).astype(np.float32), dt)
    z = oq.round_to(r.uniform(0.0, 3.0, size=(N, ng)).astype(np.float32), dt)
    Wd = oq.dequant_int2(q, s, z, K, G, "bf16")
    return dict(q=q, s=s, z=z, in_f=K, G=G, dt=dt, Wd=Wd)


@functools.lru_cache(maxsize=4)
def int4_random_case(N, K, G=128, seed=0, dt="bf16"):
    """Large-N int4 cases without the RTN search: codes ~ U{0..15}, scale ~ U(0.0005, 0.005),
    zero ~ U{0..15} (stored in dt). No bf16 oracle dequant (Wd None): the checks use the exact
    dequant, which is fast at these sizes."""
    r = rng(seed)
    ng = -(-K // G)
    q = r.integers(0, 256, size=(N, ng * G // 2), dtype=np.uint8)
    s = oq.round_to(r.uniform(0.0005, 0.005, size=(N, ng)).astype(np.float32), dt)
    z = r.integers(0, 16, size=(N, ng)).astype(np.float32)
    return dict(q=q, s=s, z=z, in_f=K, G=G, dt=dt, Wd=None)


@functools.lru_cache(maxsize=16)
def int8_case(N, K, seed=0, dt="bf16", wstd=0.02):
    r = rng(seed)
    W = bf16_normal(r, (N, K), wstd, dt)
    q, s = oq.pack_linear_int8(W, dt)
    return dict(W=W, q=q, s=s, dt=dt)


def to_torch(a, dt, device):
    """numpy float32 (dtype-representable values) / int arrays -> torch tensor of dtype name dt."""
    import torch
    tdt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[dt]
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(tdt).to(device)


def u8(a, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def t2np(t):
    import torch
    return t.detach().to(torch.float32).cpu().numpy()


def line_tile_np(q):
    """The line-tiled int4 layout of a row-layout qweight u8 [N, Kpad/2] (N % 16 == 0, Kpad % 256
    == 0), restated from its definition: in 16-row tile t the 2 KiB block of line-step l holds in
    16-byte slot 64 h + s piece 4 (((s >> 3) & 1) ^ h) + (s >> 4) of tile row 8 h + (s & 7)."""
    q = np.ascontiguousarray(q)
    N, KB = q.shape
    assert N % 16 == 0 and KB % 128 == 0
    KL = KB // 128
    pieces = q.reshape(N // 16, 16, KL, 8, 16)            # tile, row, line-step, piece, byte
    out = np.empty((N // 16, KL, 2, 64, 16), dtype=np.uint8)
    for h in range(2):
        for s in range(64):
            out[:, :, h, s] = pieces[:, 8 * h + (s & 7), :, 4 * (((s >> 3) & 1) ^ h) + (s >> 4)]
    return out.reshape(N, KB)
