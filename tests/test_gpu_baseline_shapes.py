"""GPU parity at the BASELINE configs' full shapes (C2 full-N decode linears, C3 int2 at 70B
widths, C4 prefill at M = 2048) and with outlier activation channels.

References are float64 products over the oracle's bit-exact weights:
  * decode kernels accumulate the un-rounded weight ``(q - bf16 z) * bf16 s`` (dequant_exact);
  * the prefill GEMM feeds MFMA the weight rounded once to bf16, which for the integer zeros of
    the reference packers is exactly the reference dequant;
  * int8: ``s * (x @ q.T)`` (int8_gemm_ref).
Bars: normwise max relative error <= 1e-2 and mean <= 5e-3 (north star), and per element
|y - ref| <= 2^-8 |ref| + 1e-5 max|ref| (the output's bf16 rounding plus fp32 accumulation noise).
"""
import functools

import numpy as np
import pytest

from oracle import quant as oq
from tests import _cases as C

pytestmark = pytest.mark.gpu

MAX_REL = 1e-2
MEAN_REL = 5e-3


def _assert_close(y, exact, what):
    assert y.shape == exact.shape and np.isfinite(y).all(), what
    mr, me = oq.max_rel(y, exact), oq.mean_rel(y, exact)
    assert mr <= MAX_REL and me <= MEAN_REL, (what, mr, me)
    tol = 2.0 ** -8 * np.abs(exact) + 1e-5 * np.abs(exact).max()
    bad = np.abs(y - exact) > tol
    assert not bad.any(), (what, int(bad.sum()), np.argwhere(bad)[:5].tolist())


def _x(M, K, seed, outliers=False):
    """x ~ N(0, 1) in bf16; with ``outliers`` 1% of the channels carry 50x larger values (the
    activation outliers of real LLM layers), which stress the kernels' folded zero-point term
    s * sum((128 + q) x) - s * (128 + z) * sum(x)."""
    r = C.rng(seed)
    x = r.standard_normal((M, K)).astype(np.float32)
    if outliers:
        ch = r.choice(K, size=max(1, K // 100), replace=False)
        x[:, ch] *= 50.0
    return oq.round_to(x, "bf16")


@functools.lru_cache(maxsize=1)
def _int4(N, K, seed):
    c = C.int4_case.__wrapped__(N, K, 128, seed=seed)
    codes = oq.unpack_int4(c["q"])
    c["Wx"] = oq.dequant_exact(codes, c["s"], c["z"], 128, c["in_f"])
    return c


def _run_w4(dev, c, x):
    import torch
    from infinitemodel_amd import ops
    q, s, z = C.u8(c["q"], dev), C.to_torch(c["s"], "bf16", dev), C.to_torch(c["z"], "bf16", dev)
    y = ops.linear_w4(C.to_torch(x, "bf16", dev), q, 128, (s, z))
    torch.cuda.synchronize()
    return C.t2np(y)


# ---- C2: full-N gate_up and down at the decode rows --------------------------------------------
@pytest.mark.parametrize("N,K", [(28672, 4096), (4096, 14336)])
def test_c2_full_width_decode(dev, N, K):
    """Llama-3-8B gate_up 4096 -> 28672 and down 14336 -> 4096 at M = 1 and 4 (line kernel) and 16
    (K-split kernel), over the whole weight."""
    c = _int4(N, K, 1000 + N + K)
    for M in (1, 4, 16):
        x = _x(M, K, seed=M)
        _assert_close(_run_w4(dev, c, x), oq.linear_ref(x, c["Wx"]), (N, K, M))


@pytest.mark.parametrize("M", [1, 4, 16])
def test_c2_outlier_activations(dev, M):
    """Outlier channels against the line (M 1, 4) and K-split (M 16) kernels' folded zero point."""
    c = _int4(6144, 4096, 7)
    x = _x(M, 4096, seed=50 + M, outliers=True)
    _assert_close(_run_w4(dev, c, x), oq.linear_ref(x, c["Wx"]), M)


# ---- C3: int2 g64 fp16 non-integer zeros at the 70B widths --------------------------------------
@functools.lru_cache(maxsize=1)
def _int2(N, K, seed):
    """C3 generator (codes ~ U{0..3}, fp16 scale ~ U(0.005, 0.05), fp16 zero ~ U(0, 3)) at full
    width. The reference dequant ``Wd`` comes from torch's CPU bf16 arithmetic
    (oracle.cpu_path.dequant_g, pinned bit-exact to oracle.quant's dequant in test_oracle) because
    the numpy bf16 emulation takes minutes over 235M weights."""
    import torch
    from oracle import cpu_path
    r = C.rng(seed)
    ng = K // 64
    codes = r.integers(0, 4, size=(N, K), dtype=np.uint8)
    q = (codes[:, 0::4] | (codes[:, 1::4] << 2) | (codes[:, 2::4] << 4) | (codes[:, 3::4] << 6)).astype(np.uint8)
    s = oq.round_to(r.uniform(0.005, 0.05, size=(N, ng)).astype(np.float32), "fp16")
    z = oq.round_to(r.uniform(0.0, 3.0, size=(N, ng)).astype(np.float32), "fp16")
    Wd = cpu_path.dequant_g(torch.from_numpy(q), torch.from_numpy(s).half(), torch.from_numpy(z).half(), K, 64,
                            torch.bfloat16, 2).float().numpy()
    sb = torch.from_numpy(oq.round_to(s, "bf16")).double()[:, :, None]
    zb = torch.from_numpy(oq.round_to(z, "bf16")).double()[:, :, None]
    Wx = ((torch.from_numpy(codes).reshape(N, ng, 64).double() - zb) * sb).reshape(N, K).numpy()
    return dict(q=q, s=s, z=z, Wd=Wd, Wx=Wx)


@pytest.mark.parametrize("N,K", [(28672, 8192), (8192, 28672)])
def test_c3_full_width(dev, N, K):
    """C3's 8192 -> 28672 and 28672 -> 8192 over the whole weight at M = 1 and 8 (and outlier
    activations at M = 1)."""
    import torch
    from infinitemodel_amd import ops
    c = _int2(N, K, 2000 if N > K else 2001)
    q, s, z = C.u8(c["q"], dev), C.to_torch(c["s"], "fp16", dev), C.to_torch(c["z"], "fp16", dev)
    for M, out in ((1, False), (8, False), (1, True)):
        x = _x(M, K, seed=60 + M, outliers=out)
        y = ops.linear_w2(C.to_torch(x, "bf16", dev), q, 64, (s, z))
        torch.cuda.synchronize()
        yn = C.t2np(y)
        _assert_close(yn, oq.linear_ref(x, c["Wx"]), (N, K, M, out))
        # and the north-star bar against the reference's own (two-rounding) dequant
        ref = oq.linear_ref(x, c["Wd"])
        assert oq.max_rel(yn, ref) <= MAX_REL and oq.mean_rel(yn, ref) <= MEAN_REL


# ---- C4: prefill at M = 2048 ---------------------------------------------------------------------
@pytest.mark.parametrize("N,K", [(14336, 4096), (4096, 14336)])
def test_c4_prefill_int4_m2048(dev, N, K):
    """The LDS-dequant MFMA GEMM at the C4 shapes and M = 2048 (and M = 512 with outliers)."""
    c = _int4(N, K, 3000 + N)
    Wb = oq.round_to(c["Wx"].astype(np.float32), "bf16")
    assert np.array_equal(Wb, c["Wd"])          # integer zeros: bf16-rounded exact == reference dequant
    for M, out in ((2048, False), (512, True)):
        x = _x(M, K, seed=70 + M, outliers=out)
        _assert_close(_run_w4(dev, c, x), oq.linear_ref(x, Wb), (N, K, M, out))


@pytest.mark.parametrize("bits", [4, 8])
def test_register_b_ragged_split_k(dev, bits):
    """The register-B GEMM with ragged rows and columns AND K splits: M = 600, N = 1000, K = 14336
    runs 128-row tiles with four K splits on 256 CUs (the plan the CPU bounds model restates), so
    partial stores of ragged tiles and the reduction's column tails are exercised; then twice in a
    row, bit-identical."""
    import torch
    from infinitemodel_amd import ops
    M, N, K = 600, 1000, 14336
    x = _x(M, K, seed=91)
    if bits == 4:
        c = C.int4_case.__wrapped__(N, K, 128, seed=92)
        Wb = oq.round_to(oq.dequant_exact(oq.unpack_int4(c["q"]), c["s"], c["z"], 128, c["in_f"]).astype(np.float32),
                         "bf16")
        q, s_, z = C.u8(c["q"], dev), C.to_torch(c["s"], "bf16", dev), C.to_torch(c["z"], "bf16", dev)
        run = lambda: ops.linear_w4(C.to_torch(x, "bf16", dev), q, 128, (s_, z))   # noqa: E731
        ref = oq.linear_ref(x, Wb)
    else:
        c = C.int8_case.__wrapped__(N, K, seed=93, dt="bf16")
        q, s_ = C.u8(c["q"], dev), C.to_torch(c["s"], "bf16", dev)
        run = lambda: ops.linear_w8(C.to_torch(x, "bf16", dev), q, s_)   # noqa: E731
        ref = oq.int8_gemm_ref(x, c["q"], c["s"])
    y1 = run()
    y2 = run()
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    _assert_close(C.t2np(y1), ref, (bits, M, N, K))


@pytest.mark.parametrize("N,K", [(14336, 4096), (4096, 14336)])
def test_c4_prefill_int8_fp16_scale_m2048(dev, N, K):
    """int8 per-row symmetric with fp16 scales (the C4 int8 weights) at M = 2048."""
    import torch
    from infinitemodel_amd import ops
    c = C.int8_case.__wrapped__(N, K, seed=3100 + N, dt="fp16")
    q, s = C.u8(c["q"], dev), C.to_torch(c["s"], "fp16", dev)
    for M, out in ((2048, False), (512, True)):
        x = _x(M, K, seed=80 + M, outliers=out)
        y = ops.linear_w8(C.to_torch(x, "bf16", dev), q, s)
        torch.cuda.synchronize()
        _assert_close(C.t2np(y), oq.int8_gemm_ref(x, c["q"], c["s"]), (N, K, M, out))


@pytest.mark.parametrize("M", [1, 4, 16])
def test_int8_outlier_activations(dev, M):
    """int8 decode kernels (line M <= 4, skinny M 16) with outlier channels: the kernel form
    s * (sum x (q + 128) - 128 sum x) cancels a large common term."""
    import torch
    from infinitemodel_amd import ops
    c = C.int8_case(1024, 4096, seed=90, dt="bf16")
    x = _x(M, 4096, seed=91 + M, outliers=True)
    y = ops.linear_w8(C.to_torch(x, "bf16", dev), C.u8(c["q"], dev), C.to_torch(c["s"], "bf16", dev))
    torch.cuda.synchronize()
    _assert_close(C.t2np(y), oq.int8_gemm_ref(x, c["q"], c["s"]), M)
