"""Device RTN packers (imq_pack_w4 / w2 / w8) are bit-identical to the host packers the cache
compiler and the load-time quantizer share (shard_compile.pack_linear_int4 / int2 / int8 on the
CPU, pinned to the oracle in test_oracle / test_packers): codes byte for byte, scale and zero bit
for bit -- including zero-padded last groups, all-zero groups (a -0.0 zero point), constant groups
(scale 1e-8) and the fp16 int8 quirk (fp16(1e-8) == 0)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

DTS = ["bf16", "fp16", "fp32"]


def _tdt(dt):
    import torch
    return {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[dt]


def _bits(t):
    import torch
    t = t.detach().cpu()
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32).numpy()


def _weights(N, K, dt, seed, std=0.02):
    """N(0, std) rows plus the special rows: an all-zero row, a constant row, a row with one large
    outlier, a row of tiny values (scale clamped to 1e-8)."""
    import torch
    g = torch.Generator().manual_seed(seed)
    W = torch.randn(N, K, generator=g) * std
    if N >= 4:
        W[0] = 0.0
        W[1] = 0.5
        W[2, K // 3] = 7.0
        W[3] = 1e-10
    return W.to(_tdt(dt))


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("bits,G", [(4, 128), (4, 64), (4, 256), (2, 64), (2, 128)])
@pytest.mark.parametrize("N,K", [(64, 4096), (37, 300), (5, 64), (300, 1000)])
def test_group_packer_bit_identical(dev, dt, bits, G, N, K):
    from infinitemodel_amd import ops, shard_compile as sc
    W = _weights(N, K, dt, seed=N + K + G)
    host = (sc.pack_linear_int4 if bits == 4 else sc.pack_linear_int2)(W, G)
    devp = (ops.pack_w4 if bits == 4 else ops.pack_w2)(W.to(dev), G)
    assert devp[3] == host[3] == K
    assert np.array_equal(devp[0].cpu().numpy(), host[0].numpy())
    assert devp[1].dtype == host[1].dtype == W.dtype
    assert np.array_equal(_bits(devp[1]), _bits(host[1]))
    assert np.array_equal(_bits(devp[2]), _bits(host[2]))


@pytest.mark.parametrize("dt", DTS)
@pytest.mark.parametrize("N,K", [(64, 4096), (37, 300), (4, 14336)])
def test_int8_packer_bit_identical(dev, dt, N, K):
    from infinitemodel_amd import ops, shard_compile as sc
    W = _weights(N, K, dt, seed=N * K)
    qh, sh = sc.pack_linear_int8(W)
    qd, sd = ops.pack_w8(W.to(dev))
    assert np.array_equal(qd.cpu().numpy(), qh.numpy())
    assert np.array_equal(_bits(sd), _bits(sh))


def test_packers_dispatch_to_the_device_and_match_the_oracle(dev):
    """shard_compile's packers take the device path for a ROCm tensor and agree with the numpy
    oracle at the C2 gate_up shape slice."""
    import torch
    from infinitemodel_amd import shard_compile as sc
    from oracle import quant as oq
    W = _weights(512, 4096, "bf16", seed=7)
    q, s, z, in_f = sc.pack_linear_int4(W.to(dev), 128)
    assert q.is_cuda and s.is_cuda
    qo, so, zo, _ = oq.pack_linear_int4(W.float().numpy(), 128, "bf16")
    assert np.array_equal(q.cpu().numpy(), qo)
    assert np.array_equal(s.float().cpu().numpy(), so) and np.array_equal(z.float().cpu().numpy(), zo)
    q8, s8 = sc.pack_linear_int8(W.to(dev))
    qo8, so8 = oq.pack_linear_int8(W.float().numpy(), "bf16")
    assert np.array_equal(q8.cpu().numpy(), qo8) and np.array_equal(s8.float().cpu().numpy(), so8)
    assert torch.equal(sc.pack_linear_int2(W.to(dev), 64)[0].cpu(), sc.pack_linear_int2(W, 64)[0])
