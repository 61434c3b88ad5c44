"""The package's torch packers (shard_compile.py restatement, used by the module packers) are
byte-identical to the oracle's numpy packers, which tests/test_oracle.py pins against known
answers, closed forms and the reference quirks."""
import numpy as np
import pytest
import torch

from infinitemodel_amd import shard_compile as sc
from infinitemodel_amd import worker_quant as wq
from oracle import quant as oq

TDT = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


def _w(shape, dt, seed, std=0.02):
    r = np.random.default_rng(seed)
    W = oq.round_to((r.standard_normal(shape) * std).astype(np.float32), dt)
    # a constant group and an all-zero row exercise the clamp(min=1e-8) branches
    W[0, :] = 0.0
    if shape[1] >= 128:
        W[1, :128] = W[1, 0]
    return W


def _t(a, dt):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(TDT[dt])


@pytest.mark.parametrize("dt", ["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("N,K,G", [(64, 4096, 128), (33, 1000, 128), (16, 100, 128), (24, 448, 64)])
def test_int4_packer_matches_oracle(dt, N, K, G):
    W = _w((N, K), dt, N + K)
    q, s, z, in_f = sc.pack_linear_int4(_t(W, dt), G)
    oq_, os_, oz_, oin = oq.pack_linear_int4(W, G, dt)
    assert in_f == oin == K
    assert np.array_equal(q.numpy(), oq_)
    assert s.dtype == TDT[dt] and z.dtype == TDT[dt]
    assert np.array_equal(s.float().numpy(), os_) and np.array_equal(z.float().numpy(), oz_)


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("N,K,G", [(64, 1024, 64), (17, 200, 64)])
def test_int2_packer_matches_oracle(dt, N, K, G):
    W = _w((N, K), dt, 7 * N + K)
    q, s, z, in_f = sc.pack_linear_int2(_t(W, dt), G)
    oq_, os_, oz_, _ = oq.pack_linear_int2(W, G, dt)
    assert np.array_equal(q.numpy(), oq_)
    assert np.array_equal(s.float().numpy(), os_) and np.array_equal(z.float().numpy(), oz_)


@pytest.mark.parametrize("dt", ["bf16", "fp16", "fp32"])
def test_int8_packer_matches_oracle(dt):
    W = _w((48, 512), dt, 11)
    q, s = sc.pack_linear_int8(_t(W, dt))
    oq_, os_ = oq.pack_linear_int8(W, dt)
    assert q.dtype == torch.int8 and s.dtype == TDT[dt] and tuple(s.shape) == (48, 1)
    assert np.array_equal(q.numpy(), oq_)
    assert np.array_equal(s.float().numpy(), os_)


@pytest.mark.parametrize("in_major", [False, True])
def test_int4_3d_packer_matches_oracle(in_major):
    r = np.random.default_rng(5)
    shape = (4, 40, 256) if in_major else (4, 256, 40)
    W3 = oq.round_to((r.standard_normal(shape) * 0.02).astype(np.float32), "bf16")
    q, s, z, in_f, ng = sc.pack_linear_int4_3d(_t(W3, "bf16"), 128, in_major=in_major)
    oq_, os_, oz_, oin, ong = oq.pack_linear_int4_3d(W3, 128, "bf16", in_major=in_major)
    assert (in_f, ng) == (oin, ong)
    assert np.array_equal(q.numpy(), oq_)
    assert np.array_equal(s.float().numpy(), os_) and np.array_equal(z.float().numpy(), oz_)


def test_module_packers_use_the_same_bytes():
    W = _w((32, 300), "bf16", 3)
    lin = torch.nn.Linear(300, 32, bias=True).to(torch.bfloat16)
    lin.weight.data.copy_(_t(W, "bf16"))
    m4 = wq._quantize_linear4(lin)
    m2 = wq._quantize_linear2(lin)
    m8 = wq._quantize_linear(lin)
    assert np.array_equal(m4.qweight.numpy(), oq.pack_linear_int4(W, 128, "bf16")[0])
    assert (m4.in_features, m4.group_size) == (300, 128)
    assert np.array_equal(m2.qweight.numpy(), oq.pack_linear_int2(W, 64, "bf16")[0])
    assert (m2.in_features, m2.group_size) == (300, 64)
    assert np.array_equal(m8.qweight.numpy(), oq.pack_linear_int8(W, "bf16")[0])
    assert m4.bias is lin.bias and m8.bias is lin.bias
    # 3D experts: per-expert pack == the 2D packer on each slice
    W3 = np.stack([_w((16, 256), "bf16", 20 + e) for e in range(3)])
    p = wq._pack4_3d(_t(W3, "bf16"))
    for e in range(3):
        qe, se, ze, _ = sc.pack_linear_int4(_t(W3[e], "bf16"))
        assert torch.equal(p.qweight[e], qe) and torch.equal(p.scale[e], se) and torch.equal(p.zero[e], ze)
