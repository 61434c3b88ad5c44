"""GPU: the line-tiled layout of packed int4 / int2 / int8 weights.

* imq_line_tile / imq_line_untile against the layout's definition (tests/_cases.line_tile_np);
* imq_linear_w4_tiled bit-identical to imq_linear_w4 on the row layout, for every kernel that
  reads the tiled layout: the decode line kernel (M 1-4, 2 and 4 line-steps per wave), the
  wave-split and K-split kernels (4 < M <= 16), the LDS-dequant GEMM (16 < M <= 512) and the
  register-B GEMM (M > 512, with and without K splits, ragged N). The kernels read the same bytes
  into the same lanes in both layouts, so equality is exact, not within a tolerance; the row-layout
  results themselves are pinned against the oracle by the other parity tests;
* imq_linear_w2_tiled likewise for the int2 line kernel (M 1-2), K-split kernel (4 < M <= 16) and
  LDS-dequant GEMM (M > 16); where the int2 line kernel declines below 5 rows (M 3-4, or K beyond
  its 16 waves) the tiled call runs the K-split kernel and the row layout the skinny kernel, so
  those calls are checked against the oracle instead;
* imq_linear_w8_tiled bit-identical to imq_linear_w8 for the int8 line kernel (M 1-4), the skinny
  kernel (4 < M <= 16) and both prefill GEMMs.
"""
import numpy as np
import pytest

from tests import _cases as C

pytestmark = pytest.mark.gpu


def _weights(dev, N, K, dt="bf16", seed=0):
    c = C.int4_random_case(N, K, 128, seed=seed, dt=dt)
    return c, C.u8(c["q"], dev), C.to_torch(c["s"], dt, dev), C.to_torch(c["z"], dt, dev)


@pytest.mark.parametrize("N,K", [(16, 256), (48, 768), (4096, 4096)])
def test_tile_and_untile_match_the_definition(dev, N, K):
    import torch
    from infinitemodel_amd import ops
    c, q, _, _ = _weights(dev, N, K, seed=N)
    t = ops.line_tile(q)
    torch.cuda.synchronize()
    assert np.array_equal(t.cpu().numpy(), C.line_tile_np(c["q"]))
    assert torch.equal(ops.line_untile(t), q)


def test_tile_reads_strided_rows_and_untile_writes_them(dev):
    import torch
    from infinitemodel_amd import ops
    c, q, _, _ = _weights(dev, 32, 512, seed=7)
    wide = torch.zeros((32, 256 + 48), dtype=torch.uint8, device=dev)
    wide[:, :256] = q
    t = ops.line_tile(wide[:, :256])
    assert np.array_equal(t.cpu().numpy(), C.line_tile_np(c["q"]))
    back = torch.full((32, 256 + 32), 7, dtype=torch.uint8, device=dev)
    ops.line_untile(t, out=back[:, :256])
    assert torch.equal(back[:, :256], q) and bool((back[:, 256:] == 7).all())


# (N, K, M, scale dtype): the kernel each row lands on is named in the id
CASES = [
    pytest.param(4096, 4096, 1, "bf16", id="line-M1"),
    pytest.param(4096, 4096, 2, "bf16", id="line-M2"),
    pytest.param(6144, 4096, 3, "fp16", id="line-M3-fp16"),
    pytest.param(4096, 4096, 4, "fp32", id="line-M4-fp32"),
    pytest.param(4096, 14336, 1, "bf16", id="line-M1-4steps"),
    pytest.param(1008, 2048, 2, "bf16", id="line-M2-ragged-tiles"),
    pytest.param(28672, 4096, 5, "bf16", id="wsplit-M5"),
    pytest.param(28672, 4096, 16, "fp16", id="wsplit-M16-fp16"),
    pytest.param(4096, 14336, 8, "bf16", id="ksplit-M8"),
    pytest.param(4096, 14336, 16, "bf16", id="ksplit-M16"),
    pytest.param(1024, 4096, 12, "fp32", id="ksplit-M12-fp32"),
    pytest.param(4096, 4096, 17, "bf16", id="gemm-M17"),
    pytest.param(1008, 2048, 100, "fp16", id="gemm-M100-fp16"),
    pytest.param(4096, 14336, 512, "bf16", id="gemm-M512"),
    pytest.param(4096, 4096, 600, "bf16", id="rb-M600"),
    pytest.param(14336, 4096, 1024, "fp16", id="rb-M1024-fp16"),
    pytest.param(1008, 14336, 600, "bf16", id="rb-M600-ragged-N-split"),
]


@pytest.mark.parametrize("N,K,M,dt", CASES)
def test_tiled_linear_is_bit_identical_to_the_row_layout(dev, N, K, M, dt):
    import torch
    from infinitemodel_amd import ops
    _, q, s, z = _weights(dev, N, K, dt=dt, seed=N + K)
    x = torch.randn(M, K, generator=torch.Generator(device=dev).manual_seed(M + N), device=dev).to(torch.bfloat16)
    t = ops.line_tile(q)
    y_row = ops.linear_w4(x, q, 128, (s, z))
    y_t = ops.linear_w4_tiled(x, t, 128, (s, z))
    torch.cuda.synchronize()
    assert torch.equal(y_t, y_row)
    assert bool(torch.isfinite(y_t.float()).all())


@pytest.mark.parametrize("M", [1, 4])
def test_tiled_rows_beyond_the_line_kernel_match_the_oracle(dev, M):
    """K beyond the line kernel's 16 waves (K_pad 16640): the K-split kernel on tiled weights,
    the skinny kernel on the row layout -- both against the oracle."""
    import torch
    from oracle import quant as oq
    from infinitemodel_amd import ops
    K = 16640
    c = C.int4_random_case(256, K, 128, seed=21)
    q, s, z = C.u8(c["q"], dev), C.to_torch(c["s"], "bf16", dev), C.to_torch(c["z"], "bf16", dev)
    x = C.bf16_normal(C.rng(M), (M, K))
    t = ops.line_tile(q)
    y = ops.linear_w4_tiled(C.to_torch(x, "bf16", dev), t, 128, (s, z))
    y_row = ops.linear_w4(C.to_torch(x, "bf16", dev), q, 128, (s, z))
    torch.cuda.synchronize()
    ref = oq.linear_ref(x, oq.dequant_int4(c["q"], c["s"], c["z"], K, 128, "bf16"))
    assert oq.max_rel(C.t2np(y), ref) <= 1e-2
    assert oq.max_rel(C.t2np(y), C.t2np(y_row)) <= 1e-2


def test_tiled_linear_repeats_bit_identically(dev):
    """Two calls in a row (split-K partials and the persistent kernels' LDS reused) agree."""
    import torch
    from infinitemodel_amd import ops
    _, q, s, z = _weights(dev, 4096, 14336, seed=3)
    t = ops.line_tile(q)
    for M in (16, 1, 700):
        x = torch.randn(M, 14336, device=dev).to(torch.bfloat16)
        a = ops.linear_w4_tiled(x, t, 128, (s, z))
        b = ops.linear_w4_tiled(x, t, 128, (s, z))
        torch.cuda.synchronize()
        assert torch.equal(a, b)


def test_tiled_shapes_outside_the_layout_are_rejected(dev):
    import torch
    from infinitemodel_amd import ops
    from infinitemodel_amd._lib import ImqError
    with pytest.raises(ValueError):
        ops.line_tile(torch.zeros((40, 128), dtype=torch.uint8, device=dev))    # N % 16
    with pytest.raises(ValueError):
        ops.line_tile(torch.zeros((32, 192), dtype=torch.uint8, device=dev))    # K_pad % 256
    _, q, s, z = _weights(dev, 64, 512, seed=1)
    t = ops.line_tile(q)
    x = torch.zeros((1, 512), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        ops.linear_w4_tiled(x, t, 64, (s, z))                                        # groups of 128 only
    with pytest.raises(ImqError):
        # direct call with a row stride other than K_pad / 2: IMQ_ERR_INVALID
        from infinitemodel_amd._lib import call, IMQ_DT_BF16
        y = torch.empty((1, 64), dtype=torch.bfloat16, device=dev)
        call("imq_linear_w4_tiled", x.data_ptr(), 512, 1, 512, t.data_ptr(), 512, s.data_ptr(), s.stride(0), 1,
             IMQ_DT_BF16, z.data_ptr(), z.stride(0), 1, IMQ_DT_BF16, 64, 128, y.data_ptr(), 64, None, 0,
             torch.cuda.current_stream(dev).cuda_stream)


def _w2(dev, N, K, seed):
    c = C.int2_random_case(N, K, 64, seed=seed, dt="fp16")
    return c, C.u8(c["q"], dev), C.to_torch(c["s"], "fp16", dev), C.to_torch(c["z"], "fp16", dev)


W2_CASES = [
    pytest.param(4096, 8192, 1, id="w2-line-M1"),
    pytest.param(1008, 4096, 2, id="w2-line-M2-ragged-tiles"),
    pytest.param(4096, 8192, 5, id="w2-ksplit-M5"),
    pytest.param(8192, 4096, 8, id="w2-ksplit-M8"),
    pytest.param(1008, 8192, 16, id="w2-ksplit-M16"),
    pytest.param(4096, 4096, 17, id="w2-gemm-M17"),
    pytest.param(1008, 8192, 300, id="w2-gemm-M300"),
    pytest.param(4096, 4096, 700, id="w2-gemm-M700"),
]


@pytest.mark.parametrize("N,K,M", W2_CASES)
def test_tiled_int2_linear_is_bit_identical_to_the_row_layout(dev, N, K, M):
    import torch
    from infinitemodel_amd import ops
    _, q, s, z = _w2(dev, N, K, seed=N + K)
    x = torch.randn(M, K, generator=torch.Generator(device=dev).manual_seed(M), device=dev).to(torch.bfloat16)
    t = ops.line_tile(q)
    y_row = ops.linear_w2(x, q, 64, (s, z))
    y_t = ops.linear_w2_tiled(x, t, 64, (s, z))
    torch.cuda.synchronize()
    assert torch.equal(y_t, y_row)


@pytest.mark.parametrize("M,K", [(3, 4096), (4, 4096), (2, 28672), (1, 33792)])
def test_tiled_int2_rows_without_a_line_kernel_match_the_oracle(dev, M, K):
    """M 3..4, and M 1..2 with K beyond the line kernel's 16 waves: the K-split kernel."""
    import torch
    from oracle import quant as oq
    from infinitemodel_amd import ops
    c, q, s, z = _w2(dev, 1024, K, seed=77)
    x = C.bf16_normal(C.rng(M), (M, K))
    t = ops.line_tile(q)
    y = ops.linear_w2_tiled(C.to_torch(x, "bf16", dev), t, 64, (s, z))
    y_row = ops.linear_w2(C.to_torch(x, "bf16", dev), q, 64, (s, z))
    torch.cuda.synchronize()
    ref = oq.linear_ref(x, c["Wd"])
    assert oq.max_rel(C.t2np(y), ref) <= 1e-2
    assert oq.max_rel(C.t2np(y), C.t2np(y_row)) <= 1e-2


W8_CASES = [
    pytest.param(4096, 3584, 1, "bf16", id="w8-line-M1"),
    pytest.param(1008, 4096, 2, "fp16", id="w8-line-M2"),
    pytest.param(4096, 3584, 4, "bf16", id="w8-line-M4"),
    pytest.param(4096, 4096, 5, "bf16", id="w8-skinny-M5"),
    pytest.param(1008, 3584, 16, "fp16", id="w8-skinny-M16"),
    pytest.param(4096, 4096, 17, "bf16", id="w8-gemm-M17"),
    pytest.param(1008, 4096, 100, "fp16", id="w8-gemm-M100-small-tiles"),
    pytest.param(4096, 14336, 512, "bf16", id="w8-gemm-M512"),
    pytest.param(14336, 4096, 1024, "fp16", id="w8-rb-M1024"),
    pytest.param(1008, 14336, 600, "bf16", id="w8-rb-M600-ragged-N-split"),
]


@pytest.mark.parametrize("N,K,M,dt", W8_CASES)
def test_tiled_int8_linear_is_bit_identical_to_the_row_layout(dev, N, K, M, dt):
    import torch
    from infinitemodel_amd import ops
    c = C.int8_case(N, K, seed=N + K, dt=dt)
    q = torch.from_numpy(c["q"].astype(np.int8)).to(dev)
    s = C.to_torch(c["s"], dt, dev)
    x = torch.randn(M, K, generator=torch.Generator(device=dev).manual_seed(M), device=dev).to(torch.bfloat16)
    t = ops.line_tile(q)
    assert t.dtype == torch.int8 and torch.equal(ops.line_untile(t), q)
    y_row = ops.linear_w8(x, q, s)
    y_t = ops.linear_w8_tiled(x, t, s)
    torch.cuda.synchronize()
    assert torch.equal(y_t, y_row)
