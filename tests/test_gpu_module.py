"""The reference module API on the GPU: prepare_fused binds the HIP ops (never a torch
substitute), forward matches the oracle, the naive path uses the HIP dequant, and the fused MoE
forward installs on a transformers OlmoeExperts module and matches the oracle."""
import numpy as np
import pytest

from oracle import moe as om
from oracle import quant as oq
from tests import _cases as C

pytestmark = pytest.mark.gpu

MAX_REL = 1e-2


@pytest.fixture(autouse=True)
def _small_prefill_bench(monkeypatch):
    monkeypatch.setenv("INFINITEMODEL_PREFILL_CHUNK", "256")


def _q4(dev, N, K, seed, bias):
    import torch
    from infinitemodel_amd import worker_quant as wq
    c = C.int4_case(N, K, 128, seed)
    b = torch.nn.Parameter((torch.randn(N) * 0.1).to(torch.bfloat16).to(dev)) if bias else None
    m = wq._quant4_linear_cls()(C.u8(c["q"], dev), C.to_torch(c["s"], "bf16", dev),
                                C.to_torch(c["z"], "bf16", dev), b, K, 128)
    return m, c


def test_quantlinear4_binds_hip_op_and_matches(dev):
    import torch
    from infinitemodel_amd import ops
    m, c = _q4(dev, 512, 1000, 3, bias=True)
    m.prepare_fused()
    assert m._fused is not None and m._fused[2] is ops.linear_w4_tiled and m._fused[3] == 1024
    assert m._line_tiled and m.qweight.is_contiguous() and m._fused[0] is m.qweight
    assert np.array_equal(m.qweight.cpu().numpy(), C.line_tile_np(c["q"]))
    bias = C.t2np(m.bias)
    for shape in [(1, 1000), (2, 3, 1000), (16, 1000), (40, 1000)]:
        x = C.bf16_normal(C.rng(len(shape)), shape)
        y = m(C.to_torch(x, "bf16", dev))
        assert y.dtype == torch.bfloat16 and y.shape[:-1] == shape[:-1]
        ref = oq.linear_ref(x.reshape(-1, 1000), c["Wd"]) + bias
        assert oq.max_rel(C.t2np(y).reshape(-1, 512), ref) <= MAX_REL


def test_quantlinear4_row_layout_when_tiling_is_off_or_does_not_fit(dev, monkeypatch):
    """Row layout with de-aliased rows: the switch off, or rows not a multiple of 16."""
    from infinitemodel_amd import ops
    from infinitemodel_amd import worker_quant as wq
    monkeypatch.setattr(wq, "_LINE_TILED", False)
    m, c = _q4(dev, 512, 1000, 3, bias=False)
    m.prepare_fused()
    assert m._fused[2] is ops.linear_w4 and not m._line_tiled
    assert m.qweight.stride(0) == 512 + 64          # de-aliased rows (512-byte rows -> 576)
    monkeypatch.setattr(wq, "_LINE_TILED", True)
    m2, c2 = _q4(dev, 40, 512, 4, bias=False)
    m2.prepare_fused()
    assert m2._fused[2] is ops.linear_w4 and not m2._line_tiled
    x = C.bf16_normal(C.rng(9), (3, 512))
    assert oq.max_rel(C.t2np(m2(C.to_torch(x, "bf16", dev))), oq.linear_ref(x, c2["Wd"])) <= MAX_REL


def test_quantlinear4_line_tiled_state_dict_round_trip(dev):
    """A line-tiled module saves qweight in the row layout, dequantizes bit-exactly, and a
    row-layout state dict loaded after binding serves the new weights."""
    import torch
    m, c = _q4(dev, 256, 512, 11, bias=False)
    m.prepare_fused()
    assert m._line_tiled
    sd = m.state_dict()
    assert np.array_equal(sd["qweight"].cpu().numpy(), c["q"])
    assert np.array_equal(C.t2np(m._dequant(torch.bfloat16)), c["Wd"])
    c2 = C.int4_case(256, 512, 128, 12)
    m.load_state_dict({"qweight": C.u8(c2["q"], "cpu"), "scale": C.to_torch(c2["s"], "bf16", "cpu"),
                       "zero": C.to_torch(c2["z"], "bf16", "cpu")}, strict=False)
    assert np.array_equal(m.state_dict()["qweight"].cpu().numpy(), c2["q"])
    x = C.bf16_normal(C.rng(13), (5, 512))
    y = m(C.to_torch(x, "bf16", dev))
    assert oq.max_rel(C.t2np(y), oq.linear_ref(x, c2["Wd"])) <= MAX_REL


def test_quantlinear4_fp16_activations(dev):
    import torch
    m, c = _q4(dev, 256, 512, 4, bias=False)
    m.prepare_fused()
    x = C.bf16_normal(C.rng(1), (4, 512))
    y = m(C.to_torch(x, "fp16", dev))
    assert y.dtype == torch.float16
    assert oq.max_rel(C.t2np(y), oq.linear_ref(x, c["Wd"])) <= MAX_REL


def test_quantlinear4_dequant_on_gpu_is_bitexact(dev):
    import torch
    m, c = _q4(dev, 128, 300, 5, bias=False)
    w = m._dequant(torch.bfloat16)
    assert np.array_equal(C.t2np(w), c["Wd"])


def test_quantlinear4_naive_path_when_disabled(dev, monkeypatch):
    """With the fused op off the forward is F.linear over the HIP dequant (no torch dequant)."""
    import torch
    import torch.nn.functional as F
    from infinitemodel_amd import worker_quant as wq
    monkeypatch.setattr(wq, "_FUSED_INT4", False)
    m, c = _q4(dev, 128, 256, 6, bias=False)
    m.prepare_fused()
    assert getattr(m, "_fused", None) is None
    x = C.to_torch(C.bf16_normal(C.rng(2), (3, 256)), "bf16", dev)
    assert torch.equal(m(x), F.linear(x, m._dequant(torch.bfloat16)))


def test_quantlinear4_prefill_threshold_falls_through(dev):
    """A bound module whose measured threshold is the 64-row bucket (worker_quant.py:817-853):
    calls whose row bucket reaches 64 (33..64 rows and above) run the naive F.linear over the HIP
    dequant, bit for bit; 32 rows and fewer keep the fused op, bit for bit its output."""
    import torch
    import torch.nn.functional as F
    from infinitemodel_amd import ops
    m, c = _q4(dev, 512, 1000, 7, bias=True)
    m.prepare_fused()
    assert m._fused is not None
    m._naive_m_min = 64
    w = m._dequant(torch.bfloat16)
    qw, pair, op, in_pad = m._fused
    assert op is ops.linear_w4_tiled and qw is m.qweight      # line-tiled binding
    for rows in (1, 16, 32, 33, 64, 100):
        x = C.to_torch(C.bf16_normal(C.rng(rows), (rows, 1000)), "bf16", dev)
        y = m(x)
        if rows <= 32:
            xp = torch.nn.functional.pad(x, (0, in_pad - 1000))
            ref = op(xp, qw, 128, pair) + m.bias
        else:
            ref = F.linear(x, w, m.bias)
        assert torch.equal(y, ref), rows
    # leading dims are rows: 2 x 20 = 40 rows -> bucket 64 -> naive
    x = C.to_torch(C.bf16_normal(C.rng(9), (2, 20, 1000)), "bf16", dev)
    assert torch.equal(m(x), F.linear(x, w, m.bias))
    # and the fused rows still match the oracle
    x = C.bf16_normal(C.rng(10), (32, 1000))
    ref = oq.linear_ref(x, c["Wd"]) + C.t2np(m.bias)
    assert oq.max_rel(C.t2np(m(C.to_torch(x, "bf16", dev))), ref) <= MAX_REL


def test_quantlinear2_module(dev):
    import torch
    from infinitemodel_amd import ops
    from infinitemodel_amd import worker_quant as wq
    c = C.int2_random_case(256, 512, 64, seed=2001, dt="fp16")
    m = wq._quant2_linear_cls()(C.u8(c["q"], dev), C.to_torch(c["s"], "fp16", dev),
                                C.to_torch(c["z"], "fp16", dev), None, 512, 64)
    m.prepare_fused()
    assert m._fused is not None and m._fused[2] is ops.linear_w2_tiled and m._line_tiled   # line-tiled
    assert np.array_equal(m.state_dict()["qweight"].cpu().numpy(), c["q"])
    for M in (1, 3, 8, 32):
        x = C.bf16_normal(C.rng(M), (M, 512))
        y = m(C.to_torch(x, "bf16", dev))
        assert oq.max_rel(C.t2np(y), oq.linear_ref(x, c["Wd"])) <= MAX_REL


def test_quantlinear_int8_module(dev):
    import torch
    from infinitemodel_amd import ops
    from infinitemodel_amd import worker_quant as wq
    c = C.int8_case(512, 1024, seed=7, dt="bf16")
    m = wq._quant_linear_cls()(C.u8(c["q"], dev), C.to_torch(c["s"], "bf16", dev), None)
    m.prepare_fused()
    assert m._fused_tried
    if getattr(m, "_w8", None) is not None:
        # the op serves every M -> line-tiled weights; decode only -> the row layout
        assert (m._w8 is ops.linear_w8_tiled) == (m._w8_m_max == 0 and m._line_tiled)
        assert np.array_equal(m.state_dict()["qweight"].cpu().numpy().astype(np.int8), c["q"].astype(np.int8))
    for M in (1, 4, 64):
        x = C.bf16_normal(C.rng(M), (M, 1024))
        y = m(C.to_torch(x, "bf16", dev))
        assert oq.max_rel(C.t2np(y), oq.int8_gemm_ref(x, c["q"], c["s"])) <= MAX_REL


def test_packed4_expert_weight_subclass(dev):
    import torch
    import torch.nn.functional as F
    from infinitemodel_amd import worker_quant as wq
    r = C.rng(12)
    W3 = C.bf16_normal(r, (4, 128, 256), 0.02)
    p = wq._pack4_3d(C.to_torch(W3, "bf16", dev))
    w1 = p[1]
    assert p._expert_kernel is True and type(w1).__name__ == "_W4A16Weight"
    x = C.bf16_normal(r, (3, 256))
    y = F.linear(C.to_torch(x, "bf16", dev), w1)
    ref = oq.linear_ref(x, oq.dequant_int4_3d(C.t2np(p.qweight).astype(np.uint8), C.t2np(p.scale),
                                               C.t2np(p.zero), 1, 256))
    assert oq.max_rel(C.t2np(y), ref) <= MAX_REL
    assert torch.equal(w1 + 0, w1._materialize())         # any other op materializes the bf16 dequant


def test_fused_moe_forward_on_olmoe_experts(dev):
    import torch
    from transformers.models.olmoe.configuration_olmoe import OlmoeConfig
    from transformers.models.olmoe.modeling_olmoe import OlmoeExperts
    from infinitemodel_amd import worker_quant as wq
    E, H, I, k = 8, 256, 128, 2
    cfg = OlmoeConfig(hidden_size=H, intermediate_size=I, num_experts=E, num_experts_per_tok=k)
    torch.manual_seed(0)
    ex = OlmoeExperts(cfg)
    with torch.no_grad():
        ex.gate_up_proj.normal_(0, 0.02)
        ex.down_proj.normal_(0, 0.02)
    ex = ex.to(torch.bfloat16)
    holder = torch.nn.Module()
    holder.experts = ex
    wq._quantize_experts4_(holder)
    holder.to(dev)
    for sub in holder.modules():
        if hasattr(sub, "prepare_fused"):
            sub.prepare_fused()
    gu, dn = ex.gate_up_proj, ex.down_proj
    Dgu = np.stack([oq.dequant_int4_3d(C.t2np(gu.qweight).astype(np.uint8), C.t2np(gu.scale),
                                       C.t2np(gu.zero), e, H) for e in range(E)])
    Ddn = np.stack([oq.dequant_int4_3d(C.t2np(dn.qweight).astype(np.uint8), C.t2np(dn.scale),
                                       C.t2np(dn.zero), e, I) for e in range(E)])
    r = C.rng(4)
    for T in (1, 5):
        idx, w = om.route_topk(r.standard_normal((T, E)).astype(np.float32), k)
        x = C.bf16_normal(r, (T, H))
        y = ex(C.to_torch(x, "bf16", dev), torch.from_numpy(idx).to(dev), C.to_torch(w, "bf16", dev))
        assert ex._fused_moe_ok is True
        exact = om.moe_exact(x, idx, w, Dgu, Ddn)
        assert oq.max_rel(C.t2np(y), exact) <= MAX_REL, T
    # the installed forward never waits on the device (no id check read back per layer), also at
    # the grouped-GEMM token counts
    for T in (1, 16, 300):
        idx, w = om.route_topk(r.standard_normal((T, E)).astype(np.float32), k)
        xt = C.to_torch(C.bf16_normal(r, (T, H)), "bf16", dev)
        it, wt = torch.from_numpy(idx).to(dev), C.to_torch(w, "bf16", dev)
        torch.cuda.synchronize()
        torch.cuda.set_sync_debug_mode("error")
        try:
            y = ex(xt, it, wt)
        finally:
            torch.cuda.set_sync_debug_mode("default")
        exact = om.moe_exact(C.t2np(xt), idx, w, Dgu, Ddn)
        assert oq.max_rel(C.t2np(y), exact) <= MAX_REL, T
