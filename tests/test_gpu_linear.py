"""GPU parity: HIP dequant (bit-exact) and fused dequant linears vs the CPU oracle.

Tolerances for the fused linears:
  * north star: normwise max relative error <= 1e-2 of the oracle's dequantize-then-matmul
    (bf16-rounded reference weights), and mean relative error <= 5e-3;
  * per element, against the exact fp64 product with the un-rounded weights (q - z) * s that the
    kernels accumulate with: |y - ref| <= 2^-8 |ref| + 1e-5 max|ref| -- i.e. only the final bf16
    rounding and fp32 accumulation noise; this catches any single wrong output element.
"""
import numpy as np
import pytest

from oracle import quant as oq
from tests import _cases as C

pytestmark = pytest.mark.gpu

MAX_REL = 1e-2
MEAN_REL = 5e-3


def _bits(t):
    import torch
    return t.view(torch.int16).cpu().numpy()


@pytest.mark.parametrize("N,K,G", [(4096, 4096, 128), (37, 384, 128), (64, 256, 64), (48, 200, 128)])
def test_dequant_w4_bitexact(dev, N, K, G):
    import torch
    from infinitemodel_amd import ops
    c = C.int4_case(N, K, G, seed=N + K)
    q = C.u8(c["q"], dev)
    s = C.to_torch(c["s"], "bf16", dev)
    z = C.to_torch(c["z"], "bf16", dev)
    out = ops.dequant_w4(q, s, z, c["in_f"], G, torch.bfloat16)
    torch.cuda.synchronize()
    ref = oq.f32_to_bf16_bits(c["Wd"]).view(np.int16)
    assert np.array_equal(_bits(out), ref)


@pytest.mark.parametrize("odt", ["fp16", "fp32"])
def test_dequant_w4_other_dtypes(dev, odt):
    import torch
    from infinitemodel_amd import ops
    c = C.int4_case(64, 256, 128, seed=3)
    q = C.u8(c["q"], dev)
    s = C.to_torch(c["s"], "bf16", dev)
    z = C.to_torch(c["z"], "bf16", dev)
    tdt = {"fp16": torch.float16, "fp32": torch.float32}[odt]
    out = ops.dequant_w4(q, s, z, c["in_f"], 128, tdt)
    ref = oq.dequant_int4(c["q"], c["s"], c["z"], c["in_f"], 128, odt)
    assert np.array_equal(C.t2np(out), ref)


def test_dequant_w2_bitexact_nonint_zero(dev):
    """BASELINE C3 style: fp16 non-integer zeros -> the two-rounding reference rule."""
    import torch
    from infinitemodel_amd import ops
    c = C.int2_random_case(128, 512, 64, seed=2000, dt="fp16")
    q = C.u8(c["q"], dev)
    s = C.to_torch(c["s"], "fp16", dev)
    z = C.to_torch(c["z"], "fp16", dev)
    out = ops.dequant_w2(q, s, z, c["in_f"], 64, torch.bfloat16)
    assert np.array_equal(_bits(out), oq.f32_to_bf16_bits(c["Wd"]).view(np.int16))


def test_dequant_w8_promotion(dev):
    import torch
    from infinitemodel_amd import ops
    c = C.int8_case(64, 999, seed=5, dt="fp16")
    q = C.u8(c["q"], dev)
    s = C.to_torch(c["s"], "fp16", dev)
    out = ops.dequant_w8(q, s, torch.bfloat16)          # bf16 x fp16 -> fp32 (torch promotion)
    assert out.dtype == torch.float32
    ref, res = oq.dequant_int8(c["q"], c["s"], "fp16", "bf16")
    assert res == "fp32"
    assert np.array_equal(C.t2np(out), ref)


def _uses_gemm(M, Kpad, G):
    """Rows > 16 with K_pad a multiple of 64 and a power-of-two group >= 32 take the tiled prefill
    GEMM (csrc/gemm.hip); the rest take the decode kernels, which keep the weights un-rounded."""
    return M > 16 and Kpad % 64 == 0 and G >= 32 and (G & (G - 1)) == 0


def _linear_check(dev, c, M, seed, bits=4, view_pad=0):
    import torch
    from infinitemodel_amd import ops
    r = C.rng(seed)
    Kpad = c["q"].shape[1] * (8 // bits)
    x = np.zeros((M, Kpad), np.float32)
    x[:, : c["in_f"]] = C.bf16_normal(r, (M, c["in_f"]))
    q = C.u8(c["q"], dev)
    if view_pad:
        buf = torch.zeros((q.shape[0], q.shape[1] + view_pad), dtype=torch.uint8, device=dev)
        buf[:, : q.shape[1]].copy_(q)
        q = buf[:, : q.shape[1]]
    s = C.to_torch(c["s"], c["dt"], dev)
    z = C.to_torch(c["z"], c["dt"], dev)
    xt = C.to_torch(x, "bf16", dev)
    fn = ops.linear_w4 if bits == 4 else ops.linear_w2
    y = fn(xt, q, c["G"], (s, z))
    yn = C.t2np(y)
    assert yn.shape == (M, q.shape[0])
    assert np.isfinite(yn).all()
    if c["Wd"] is not None:      # large random-code cases carry only the exact dequant check
        ref = oq.linear_ref(x[:, : c["in_f"]], c["Wd"])
        mr, me = oq.max_rel(yn, ref), oq.mean_rel(yn, ref)
        assert mr <= MAX_REL and me <= MEAN_REL, (M, mr, me)
    unpack = oq.unpack_int4 if bits == 4 else oq.unpack_int2
    w_exact = oq.dequant_exact(unpack(c["q"]), c["s"], c["z"], c["G"], c["in_f"])
    if _uses_gemm(M, Kpad, c["G"]):
        # the prefill GEMM feeds MFMA with bf16 weights rounded once from the exact (q - z) * s
        w_exact = oq.round_to(w_exact.astype(np.float32), "bf16")
    exact = oq.linear_ref(x[:, : c["in_f"]], w_exact)
    tol = 2.0 ** -8 * np.abs(exact) + 1e-5 * np.abs(exact).max()
    bad = np.abs(yn - exact) > tol
    assert not bad.any(), (M, int(bad.sum()), np.argwhere(bad)[:5].tolist())
    return y


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 16])
def test_linear_w4_c1_shape(dev, M):
    """BASELINE C1 shape 1x4096 -> 4096 (and the C2 M values)."""
    c = C.int4_case(4096, 4096, 128, seed=0)
    _linear_check(dev, c, M, seed=100 + M)


@pytest.mark.parametrize("N,K", [(37, 384), (1000, 256), (16, 128), (17, 1152), (6144, 4096)])
@pytest.mark.parametrize("M", [1, 4, 16])
def test_linear_w4_ragged(dev, N, K, M):
    c = C.int4_case(N, K, 128, seed=N * 7 + K)
    _linear_check(dev, c, M, seed=M)


@pytest.mark.parametrize("N,K", [(37, 512), (100, 768), (512, 14336), (48, 16384), (32, 16640)])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_linear_w4_line_kernel_shapes(dev, N, K, M):
    """Decode shapes of the int4 line kernel (M <= 4, G 128, K_pad % 256 == 0, K_pad <= 16384):
    a ragged last tile (N % 16), waves with unused line-steps (K 768), Llama down_proj K 14336,
    the largest K it takes (16384) and the first it leaves to the skinny kernel (16640)."""
    c = C.int4_case(N, K, 128, seed=N + K)
    _linear_check(dev, c, M, seed=M)


@pytest.mark.parametrize("sdt", ["fp16", "fp32"])
@pytest.mark.parametrize("M", [1, 3])
def test_linear_w4_line_kernel_scale_dtypes_dealias(dev, sdt, M):
    """The line kernel's fp16 / fp32 scale-zero words and the +64-byte de-alias row view."""
    c = dict(C.int4_case(96, 1024, 128, seed=5))
    c["s"] = oq.round_to(c["s"], sdt)
    c["z"] = oq.round_to(c["z"], sdt)
    c["dt"] = sdt
    c["Wd"] = oq.dequant_int4(c["q"], c["s"], c["z"], c["in_f"], 128, "bf16")
    _linear_check(dev, c, M, seed=M, view_pad=64)


@pytest.mark.parametrize("N,K", [(36, 768), (100, 1280), (20, 256), (4096, 14336), (6144, 4096), (28672, 4096)])
@pytest.mark.parametrize("M", [5, 8, 9, 16])
def test_linear_w4_ksplit_shapes(dev, N, K, M):
    """Decode rows 4 < M <= 16: Llama gate_up (N 28672, K 4096) takes the wave-split kernel, the
    others the K-split kernel (workspace from ops): a partial last row block (N % 64), splits with
    unused line-steps (K 768, 1280), Llama down_proj K 14336 (14 splits, 8-tile workgroups),
    both activation-row instantiations (M <= 8, <= 16)."""
    import torch
    from infinitemodel_amd import _lib
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    splits4 = -(-K // 1024)
    short = splits4 * -(-N // 128) < cus and splits4 * -(-N // 64) <= 2 * cus   # 512-code splits
    assert _lib.lib().imq_linear_workspace_bytes(M, N, K) == (-(-K // 512) if short else splits4) * M * N * 4
    c = C.int4_case(N, K, 128, seed=N + K + M)
    _linear_check(dev, c, M, seed=M)


@pytest.mark.parametrize("N,K,M", [(28672, 4096, 5), (28672, 4096, 16), (16400, 2048, 8), (16400, 2048, 12),
                                   (16392, 4096, 9)])
def test_linear_w4_wsplit_shapes(dev, N, K, M):
    """The wave-split kernel (K_pad 2048 / 4096, 4 < M <= 16, at least 4 row tiles per CU): one and
    two line-steps per wave, partial last tiles (N % 16), a persistent grid with uneven tiles per
    workgroup (N 16400, 16392: 1025 tiles), rows beyond M zero in the A operand."""
    c = C.int4_random_case(N, K, 128, seed=8000 + N + K + M)
    _linear_check(dev, c, M, seed=M + 1)


@pytest.mark.parametrize("sdt", ["fp16", "fp32"])
@pytest.mark.parametrize("K", [2048, 4096])
def test_linear_w4_wsplit_scale_dtypes_dealias(dev, sdt, K):
    """The wave-split kernel's fp16 / fp32 scale-zero words (one or two dwords per line-step) and
    the +64-byte de-alias row view."""
    c = dict(C.int4_random_case(16400, K, 128, seed=9 + K))
    c["s"] = oq.round_to(c["s"], sdt)
    c["dt"] = sdt
    for M in (6, 16):
        _linear_check(dev, c, M, seed=M, view_pad=64)


def test_linear_w4_wsplit_repeat_bit_identical_and_matches_skinny(dev):
    """Repeated wave-split calls are bit-identical; against the skinny kernel (a call the fast
    decode kernels decline: odd scale row view) they agree within fp32 accumulation order."""
    import torch
    from infinitemodel_amd import ops
    N, K, M = 16400, 4096, 16
    c = C.int4_random_case(N, K, 128, seed=21)
    q, s, z = C.u8(c["q"], dev), C.to_torch(c["s"], "bf16", dev), C.to_torch(c["z"], "bf16", dev)
    x = C.to_torch(C.bf16_normal(C.rng(22), (M, K)), "bf16", dev)
    y1 = ops.linear_w4(x, q, 128, (s, z))
    for _ in range(3):
        assert torch.equal(ops.linear_w4(x, q, 128, (s, z)), y1)
    # scale / zero as views of rows with an odd stride: the decode kernels need 4-byte aligned
    # rows, so the call falls to the skinny GEMV
    ng = K // 128
    sb = torch.zeros((N, ng + 1), dtype=torch.bfloat16, device=dev)
    zb = torch.zeros((N, ng + 1), dtype=torch.bfloat16, device=dev)
    sb[:, :ng].copy_(s)
    zb[:, :ng].copy_(z)
    y2 = ops.linear_w4(x, q, 128, (sb[:, :ng], zb[:, :ng]))
    torch.cuda.synchronize()
    d = (y1.float() - y2.float()).abs().max().item()
    assert d <= 2 ** -7 * y1.float().abs().max().item()


@pytest.mark.parametrize("N,K,M", [(16400, 4096, 16), (16400, 2048, 7), (4100, 4096, 12)])
def test_linear_w4_decode_strided_rows_bit_identical(dev, N, K, M):
    """Activation rows with a stride past K_pad and output rows with a stride past N (views of
    wider buffers) give bit-identical y to the contiguous call: the wave-split kernel (N 16400)
    and the K-split kernel (N 4100)."""
    import torch
    from infinitemodel_amd import ops
    c = C.int4_random_case(N, K, 128, seed=31 + N + M)
    q, s, z = C.u8(c["q"], dev), C.to_torch(c["s"], "bf16", dev), C.to_torch(c["z"], "bf16", dev)
    x = C.to_torch(C.bf16_normal(C.rng(32), (M, K)), "bf16", dev)
    y0 = ops.linear_w4(x, q, 128, (s, z))
    xb = torch.zeros((M, K + 64), dtype=torch.bfloat16, device=dev)
    xb[:, :K].copy_(x)
    yb = torch.full((M, N + 32), float("nan"), dtype=torch.bfloat16, device=dev)
    y1 = ops.linear_w4(xb[:, :K], q, 128, (s, z), out=yb[:, :N])
    torch.cuda.synchronize()
    assert xb[:, :K].stride(0) == K + 64 and y1.stride(0) == N + 32
    assert torch.equal(y1, y0)
    assert torch.isnan(yb[:, N:].float()).all()          # nothing written past the row's N columns


@pytest.mark.parametrize("sdt", ["fp16", "fp32"])
def test_linear_w4_ksplit_scale_dtypes_dealias(dev, sdt):
    """The K-split kernel's fp16 / fp32 scale-zero words and the +64-byte de-alias row view."""
    c = dict(C.int4_case(96, 1280, 128, seed=6))
    c["s"] = oq.round_to(c["s"], sdt)
    c["z"] = oq.round_to(c["z"], sdt)
    c["dt"] = sdt
    c["Wd"] = oq.dequant_int4(c["q"], c["s"], c["z"], c["in_f"], 128, "bf16")
    for M in (6, 16):
        _linear_check(dev, c, M, seed=M, view_pad=64)


def test_linear_w4_ksplit_without_workspace_matches(dev):
    """Without a workspace the C ABI takes the skinny kernel for 4 < M <= 16; both paths agree
    within fp32 accumulation order, and repeated K-split calls are bit-identical."""
    import torch
    from infinitemodel_amd import _lib, ops
    N, K, M = 512, 2048, 12
    c = C.int4_case(N, K, 128, seed=3)
    q, s, z = C.u8(c["q"], dev), C.to_torch(c["s"], "bf16", dev), C.to_torch(c["z"], "bf16", dev)
    x = C.to_torch(C.bf16_normal(C.rng(4), (M, K)), "bf16", dev)
    y1 = ops.linear_w4(x, q, 128, (s, z))
    y2 = torch.empty_like(y1)
    st = torch.cuda.current_stream(dev).cuda_stream
    rc = _lib.lib().imq_linear_w4(x.data_ptr(), K, M, K, q.data_ptr(), q.stride(0), s.data_ptr(), s.stride(0), 1,
                                  0, z.data_ptr(), z.stride(0), 1, 0, N, 128, y2.data_ptr(), N, None, 0, st)
    assert rc == 0
    torch.cuda.synchronize()
    d = (y1.float() - y2.float()).abs().max().item()
    assert d <= 2 ** -7 * y1.float().abs().max().item()
    for _ in range(3):
        assert torch.equal(ops.linear_w4(x, q, 128, (s, z)), y1)


def test_linear_w4_in_features_not_multiple_of_group(dev):
    c = C.int4_case(80, 300, 128, seed=11)     # K_pad = 384, x zero-padded past 300
    for M in (1, 3, 16):
        _linear_check(dev, c, M, seed=M)


def test_linear_w4_dealias_view(dev):
    """The reference's #dram-dealias padded row view (worker_quant.py:685-690) must read the same."""
    c = C.int4_case(512, 1024, 128, seed=21)
    for M in (1, 4, 16):
        _linear_check(dev, c, M, seed=M, view_pad=64)


@pytest.mark.parametrize("G", [64, 256])
def test_linear_w4_other_groups(dev, G):
    c = C.int4_case(96, 1024, G, seed=G)
    for M in (1, 5):
        _linear_check(dev, c, M, seed=M)


@pytest.mark.parametrize("M", [17, 33, 64])
def test_linear_w4_midrange_rows(dev, M):
    c = C.int4_case(256, 512, 128, seed=31)
    _linear_check(dev, c, M, seed=M)


def test_linear_w4_repeat_calls_identical(dev):
    """Repeated M=1 calls are bit-identical (no stale accumulator, deterministic reduction)."""
    import torch
    from infinitemodel_amd import ops
    c = C.int4_case(2048, 2048, 128, seed=9)
    q = C.u8(c["q"], dev)
    s = C.to_torch(c["s"], "bf16", dev)
    z = C.to_torch(c["z"], "bf16", dev)
    x = C.to_torch(C.bf16_normal(C.rng(1), (1, 2048)), "bf16", dev)
    ys = [ops.linear_w4(x, q, 128, (s, z)) for _ in range(4)]
    for y in ys[1:]:
        assert torch.equal(y, ys[0])


def test_linear_w4_one_hot_column_extraction(dev):
    """x = e_k picks column k of the dequantized weight (pins the K index mapping end to end)."""
    import torch
    from infinitemodel_amd import ops
    c = C.int4_case(64, 512, 128, seed=4)
    q = C.u8(c["q"], dev)
    s = C.to_torch(c["s"], "bf16", dev)
    z = C.to_torch(c["z"], "bf16", dev)
    ks = [0, 1, 7, 8, 31, 32, 127, 128, 300, 511]
    x = np.zeros((len(ks), 512), np.float32)
    for i, k in enumerate(ks):
        x[i, k] = 1.0
    y = C.t2np(ops.linear_w4(C.to_torch(x, "bf16", dev), q, 128, (s, z)))
    for i, k in enumerate(ks):
        col = c["Wd"][:, k]
        assert np.all(np.abs(y[i] - col) <= 1e-6 + 8e-3 * np.abs(col)), k


@pytest.mark.parametrize("sdt", ["fp16", "fp32"])
def test_linear_w4_scale_dtypes(dev, sdt):
    """fp16 / fp32 scale-zero storage (GPTQ-style caches keep fp32 s/z)."""
    c = C.int4_case(128, 512, 128, seed=12, dt="bf16")
    c = dict(c)
    c["s"] = oq.round_to(c["s"], sdt)
    c["z"] = oq.round_to(c["z"], sdt)
    c["dt"] = sdt
    c["Wd"] = oq.dequant_int4(c["q"], c["s"], c["z"], c["in_f"], 128, "bf16")
    for M in (1, 16):
        _linear_check(dev, c, M, seed=M)


# ---- int2 (BASELINE C3 style: fp16 s/z, non-integer zeros) and int8 per-row ------------------
@pytest.mark.parametrize("N,K", [(512, 1024), (96, 448), (28672 // 16, 8192 // 4)])
@pytest.mark.parametrize("M", [1, 8, 16, 40])
def test_linear_w2_random_codes(dev, N, K, M):
    c = dict(C.int2_random_case(N, K, 64, seed=2000 + N, dt="fp16"))
    _linear_check(dev, c, M, seed=M, bits=2)


@pytest.mark.parametrize("M", [1, 8, 16])
def test_linear_w2_large_k_chunked(dev, M):
    """C3's 28672 -> 8192 K at M = 8 / 16 does not fit LDS whole: x is staged in K chunks."""
    c = dict(C.int2_random_case(272, 28672, 64, seed=2003, dt="fp16"))
    _linear_check(dev, c, M, seed=M, bits=2)


@pytest.mark.parametrize("N,K", [(36, 512), (100, 1536), (512, 8192), (272, 28672), (1792, 2048)])
@pytest.mark.parametrize("M", [1, 2])
def test_linear_w2_line_kernel_shapes(dev, N, K, M):
    """Decode shapes of the int2 line kernel (M <= 2, G 64, K_pad % 512 == 0): a ragged last tile,
    waves with unused line-steps (K 1536 = 3 line-steps), C3's K 8192 and 28672 (the largest K
    at M = 1 uses 14 waves; at M = 2 it exceeds the kernel's K range and takes the skinny kernel)."""
    c = dict(C.int2_random_case(N, K, 64, seed=2100 + N + M, dt="fp16"))
    _linear_check(dev, c, M, seed=M, bits=2)


@pytest.mark.parametrize("sdt", ["bf16", "fp32"])
def test_linear_w2_line_kernel_scale_dtypes_dealias(dev, sdt):
    """The int2 line kernel's bf16 / fp32 scale-zero words and the +64-byte de-alias row view."""
    c = dict(C.int2_random_case(80, 2048, 64, seed=2200, dt=sdt))
    for M in (1, 2):
        _linear_check(dev, c, M, seed=M, bits=2, view_pad=64)


@pytest.mark.parametrize("N,K", [(36, 512), (100, 1536), (20, 1024), (272, 28672), (1792, 2048), (512, 8192)])
@pytest.mark.parametrize("M", [5, 8, 16])
def test_linear_w2_ksplit_shapes(dev, N, K, M):
    """Decode rows 4 < M <= 16 of int2 take the K-split kernel (workspace from ops): a partial last
    row block, a split with an unused line-step (K 512, 1536), C3's K 8192 and 28672 (28 splits),
    both activation-row instantiations (M <= 8, <= 16)."""
    c = dict(C.int2_random_case(N, K, 64, seed=2300 + N + M, dt="fp16"))
    _linear_check(dev, c, M, seed=M, bits=2)


@pytest.mark.parametrize("sdt", ["bf16", "fp32"])
def test_linear_w2_ksplit_scale_dtypes_dealias(dev, sdt):
    """The int2 K-split kernel's bf16 / fp32 scale-zero words and the +64-byte de-alias row view."""
    c = dict(C.int2_random_case(96, 2560, 64, seed=2400, dt=sdt))
    for M in (6, 16):
        _linear_check(dev, c, M, seed=M, bits=2, view_pad=64)


def test_linear_w2_ksplit_without_workspace_matches(dev):
    """Without a workspace the C ABI takes the skinny int2 kernel for 4 < M <= 16; both paths agree
    within fp32 accumulation order, and repeated K-split calls are bit-identical."""
    import torch
    from infinitemodel_amd import _lib, ops
    N, K, M = 512, 4096, 12
    c = C.int2_random_case(N, K, 64, seed=5, dt="fp16")
    q, s, z = C.u8(c["q"], dev), C.to_torch(c["s"], "fp16", dev), C.to_torch(c["z"], "fp16", dev)
    x = C.to_torch(C.bf16_normal(C.rng(4), (M, K)), "bf16", dev)
    y1 = ops.linear_w2(x, q, 64, (s, z))
    y2 = torch.empty_like(y1)
    st = torch.cuda.current_stream(dev).cuda_stream
    rc = _lib.lib().imq_linear_w2(x.data_ptr(), K, M, K, q.data_ptr(), q.stride(0), s.data_ptr(), s.stride(0), 1,
                                  1, z.data_ptr(), z.stride(0), 1, 1, N, 64, y2.data_ptr(), N, None, 0, st)
    assert rc == 0
    torch.cuda.synchronize()
    d = (y1.float() - y2.float()).abs().max().item()
    assert d <= 2 ** -7 * y1.float().abs().max().item()
    for _ in range(3):
        assert torch.equal(ops.linear_w2(x, q, 64, (s, z)), y1)


@pytest.mark.parametrize("N,K", [(4096, 4096), (4120, 8192), (28672, 8192)])
@pytest.mark.parametrize("M", [5, 8])
@pytest.mark.parametrize("sdt", ["fp16", "bf16"])
def test_linear_w2_ksplit_wide_shapes(dev, N, K, M, sdt):
    """int2 rows 4 < M <= 8 on grids of at least one 16-row tile per CU (the K-split kernel's
    4-tile workgroups, three resident per CU): K_pad 4096 / 8192, a ragged last row block (4120
    rows), C3's 8192 -> 28672, fp16 and bf16 scale / zero words."""
    c = dict(C.int2_random_case(N, K, 64, seed=2500 + N + M, dt=sdt))
    _linear_check(dev, c, M, seed=M, bits=2)


@pytest.mark.parametrize("K", [4096, 8192])
def test_linear_w2_ksplit_wide_fp32_scales_and_dealias(dev, K):
    """fp32 scale / zero words and the +64-byte de-alias row view on those grids; repeated calls
    are bit-identical."""
    import torch
    from infinitemodel_amd import ops
    c = dict(C.int2_random_case(4096, K, 64, seed=2600 + K, dt="fp32"))
    for M in (6, 8):
        _linear_check(dev, c, M, seed=M, bits=2, view_pad=64)
    c16 = C.int2_random_case(4096, K, 64, seed=2601, dt="fp16")
    q, s, z = C.u8(c16["q"], dev), C.to_torch(c16["s"], "fp16", dev), C.to_torch(c16["z"], "fp16", dev)
    x = C.to_torch(C.bf16_normal(C.rng(7), (7, K)), "bf16", dev)
    y = ops.linear_w2(x, q, 64, (s, z))
    for _ in range(3):
        assert torch.equal(ops.linear_w2(x, q, 64, (s, z)), y)


def test_linear_w2_fp32_scales(dev):
    c = dict(C.int2_random_case(160, 4096, 64, seed=2004, dt="fp32"))
    for M in (1, 3):
        _linear_check(dev, c, M, seed=M, bits=2)


def test_linear_w2_rtn_and_dealias(dev):
    c = C.int2_case(256, 1024, 64, seed=8)
    for M in (1, 5):
        _linear_check(dev, c, M, seed=M, bits=2, view_pad=64)


def _int8_check(dev, N, K, M, sdt, seed):
    import torch
    from infinitemodel_amd import ops
    c = C.int8_case(N, K, seed=seed, dt=sdt)
    x = C.bf16_normal(C.rng(seed + 1), (M, K))
    y = ops.linear_w8(C.to_torch(x, "bf16", dev), C.u8(c["q"], dev), C.to_torch(c["s"], sdt, dev))
    assert y.dtype == torch.bfloat16
    yn = C.t2np(y)
    exact = oq.int8_gemm_ref(x, c["q"], c["s"])
    # the naive path's weight bf16(q * s) (bf16 scale) or fp32 (fp16 scale): within 2^-8 of exact
    assert oq.max_rel(yn, exact) <= MAX_REL and oq.mean_rel(yn, exact) <= MEAN_REL
    tol = 2.0 ** -8 * np.abs(exact) + 1e-5 * np.abs(exact).max()
    assert not (np.abs(yn - exact) > tol).any()


@pytest.mark.parametrize("M", [1, 4, 16, 48])
@pytest.mark.parametrize("sdt", ["bf16", "fp16"])
def test_linear_w8(dev, M, sdt):
    _int8_check(dev, 384, 1000, M, sdt, seed=M)


@pytest.mark.parametrize("N,K,M,sdt", [(320, 14336, 1, "fp16"), (320, 14336, 5, "bf16"), (320, 14336, 16, "fp16"),
                                       (1000, 4096, 3, "bf16"), (96, 256, 16, "fp32")])
def test_linear_w8_decode_kernel(dev, N, K, M, sdt):
    """K a multiple of 64: the int8 MFMA decode kernel (x staged in chunks at K = 14336, M = 16)."""
    _int8_check(dev, N, K, M, sdt, seed=N + M)


@pytest.mark.parametrize("N,K", [(37, 128), (100, 384), (512, 3584), (272, 14336), (152064 // 64, 3584)])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_linear_w8_line_kernel(dev, N, K, M):
    """Decode rows M <= 4 with K % 128 == 0 take the int8 line kernel: a ragged last tile, one
    line-step (K 128), waves with unused line-steps (K 384 = 3 of S2 = 4), the Qwen2.5-7B head's
    K 3584 (7 waves) and K 14336 (8 line-steps per wave, 14 waves)."""
    _int8_check(dev, N, K, M, "bf16", seed=3 * N + M)


@pytest.mark.parametrize("sdt", ["fp16", "fp32"])
def test_linear_w8_line_kernel_scale_dtypes(dev, sdt):
    for M in (1, 4):
        _int8_check(dev, 200, 1024, M, sdt, seed=M + 90)


def test_linear_w8_c4_shape_rows(dev):
    _int8_check(dev, 14336 // 8, 4096, 16, "fp16", seed=77)


# ---- fused MoE rows (the reference _w4a16_moe_op contract) ------------------------------------
def test_moe_rows_w4(dev):
    """Each row b against expert eid[b], incl. repeated experts and in_features < K_pad."""
    import torch
    from infinitemodel_amd import ops
    E, N, K, G = 6, 96, 300, 128
    r = C.rng(40)
    W3 = C.bf16_normal(r, (E, N, K), 0.02)
    q, s, z, in_f, _ = oq.pack_linear_int4_3d(W3, G, "bf16")
    B = 13
    eid = r.integers(0, E, size=B).astype(np.int32)
    x = C.bf16_normal(r, (B, K))
    y = ops.moe_rows_w4(C.to_torch(x, "bf16", dev), torch.from_numpy(eid).to(dev), C.u8(q, dev),
                        C.to_torch(s, "bf16", dev), C.to_torch(z, "bf16", dev), G, in_f)
    yn = C.t2np(y)
    for b in range(B):
        e = int(eid[b])
        exact = oq.linear_ref(x[b:b + 1], oq.dequant_exact(oq.unpack_int4(q[e]), s[e], z[e], G, in_f))
        tol = 2.0 ** -8 * np.abs(exact) + 1e-5 * np.abs(exact).max()
        assert not (np.abs(yn[b:b + 1] - exact) > tol).any(), b


# ---- prefill GEMM (M > 16): tiled LDS-dequant MFMA kernel --------------------------------------
@pytest.mark.parametrize("M,N,K,G", [(17, 256, 512, 128), (128, 128, 1024, 128), (129, 200, 1024, 64),
                                     (300, 1000, 4096, 128), (512, 1792, 4096, 128)])
def test_gemm_w4(dev, M, N, K, G):
    c = C.int4_case(N, K, G, seed=M + N)
    _linear_check(dev, c, M, seed=M)


@pytest.mark.parametrize("bits", [4, 2])
def test_gemm_big_tiles_ragged(dev, bits):
    """Enough 256 x 128 tiles to take the 8-wave configuration, ragged in M and N."""
    if bits == 4:
        c = C.int4_case(4000, 256, 128, seed=77)
    else:
        c = dict(C.int2_random_case(4000, 256, 64, seed=78, dt="fp16"))
    _linear_check(dev, c, 2100, seed=9, bits=bits)


def test_gemm_w4_dealias_and_fp16_scales(dev):
    c = dict(C.int4_case(256, 2048, 128, seed=3))
    c["s"] = oq.round_to(c["s"], "fp16")
    c["z"] = oq.round_to(c["z"], "fp16")
    c["dt"] = "fp16"
    c["Wd"] = oq.dequant_int4(c["q"], c["s"], c["z"], c["in_f"], 128, "bf16")
    _linear_check(dev, c, 200, seed=5, view_pad=64)


@pytest.mark.parametrize("M", [33, 256])
def test_gemm_w2(dev, M):
    c = dict(C.int2_random_case(384, 2048, 64, seed=2002, dt="fp16"))
    _linear_check(dev, c, M, seed=M, bits=2)


@pytest.mark.parametrize("M,sdt", [(64, "fp16"), (300, "bf16")])
def test_gemm_w8(dev, M, sdt):
    _int8_check(dev, 640, 2048, M, sdt, seed=M)


# ---- split-K prefill GEMM (tiles fewer than the CUs): last-arriving split reduces ------------
@pytest.mark.parametrize("M,N,K", [(40, 256, 2048), (300, 512, 4096), (512, 4096, 14336), (150, 1000, 8192)])
def test_gemm_w4_split_k(dev, M, N, K):
    """Shapes whose tiles do not fill the CUs split K (2, 4 or 8 ways); repeated calls reuse the
    workspace and give bit-identical results (fixed-order reduction)."""
    import torch
    from infinitemodel_amd import _lib, ops
    assert _lib.lib().imq_linear_workspace_bytes(M, N, K) > 0
    c = C.int4_case(N, K, 128, seed=M + N + K)
    y = _linear_check(dev, c, M, seed=M)
    x = torch.zeros((M, K), dtype=torch.bfloat16, device=dev)
    x[:, : c["in_f"]] = C.to_torch(C.bf16_normal(C.rng(M), (M, c["in_f"])), "bf16", dev)
    q, s, z = C.u8(c["q"], dev), C.to_torch(c["s"], "bf16", dev), C.to_torch(c["z"], "bf16", dev)
    for _ in range(3):
        assert torch.equal(ops.linear_w4(x, q, 128, (s, z)), y)


def test_gemm_w8_split_k(dev):
    """int8 per-row prefill at the C4 14336 -> 4096 shape, M = 512 (8 x 32 tiles -> split 4)."""
    _int8_check(dev, 4096, 14336, 512, "fp16", seed=4)
