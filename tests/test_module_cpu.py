"""The reference module API on a CPU device (no GPU): construction, state_dict keys, the
reference dequant, the forward dispatch rules (bf16 below 16 rows, fp32 GEMM at >= 16 rows, bias
after the op), prepare_fused binding torch's CPU int4 GEMM (and nothing for int2 / int8), and the
router-excluding walkers."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from infinitemodel_amd import worker_quant as wq
from oracle import quant as oq
from tests import _cases as C


def _mod4(N=48, K=300, G=128, seed=1, bias=False):
    c = C.int4_case(N, K, G, seed)
    b = torch.nn.Parameter(torch.randn(N, dtype=torch.bfloat16) * 0.1) if bias else None
    m = wq._quant4_linear_cls()(C.u8(c["q"], "cpu"), C.to_torch(c["s"], "bf16", "cpu"),
                                C.to_torch(c["z"], "bf16", "cpu"), b, K, G)
    return m, c


def test_class_factories_are_cached_and_named():
    assert wq._quant4_linear_cls() is wq._quant4_linear_cls()
    assert wq._quant4_linear_cls().__name__ == "QuantLinear4"
    assert wq._quant2_linear_cls().__name__ == "QuantLinear2"
    assert wq._quant_linear_cls().__name__ == "QuantLinear"
    assert wq._packed4_3d_cls().__name__ == "Packed4Tensor3D"


def test_state_dict_keys_match_reference():
    m, _ = _mod4(bias=True)
    assert set(m.state_dict()) == {"qweight", "scale", "zero", "bias"}
    assert (m.in_features, m.group_size) == (300, 128)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16, torch.float32])
def test_dequant_is_the_reference_dequant(dt):
    m, c = _mod4()
    name = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[dt]
    ref = oq.dequant_int4(c["q"], c["s"], c["z"], c["in_f"], c["G"], name)
    got = m._dequant(dt)
    assert got.dtype == dt and tuple(got.shape) == (48, 300)
    assert np.array_equal(got.float().numpy(), ref)


def test_int2_dequant_is_the_reference_dequant():
    c = C.int2_random_case(40, 256, 64, 2000, "fp16")
    m = wq._quant2_linear_cls()(C.u8(c["q"], "cpu"), C.to_torch(c["s"], "fp16", "cpu"),
                                C.to_torch(c["z"], "fp16", "cpu"), None, 256, 64)
    assert np.array_equal(m._dequant(torch.bfloat16).float().numpy(), c["Wd"])


def test_forward_small_rows_is_bf16_linear():
    m, c = _mod4(bias=True)
    x = torch.randn(2, 3, 300).to(torch.bfloat16)
    y = m(x)
    ref = F.linear(x, m._dequant(torch.bfloat16), m.bias)
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (2, 3, 48)
    assert torch.equal(y, ref)


def test_forward_large_rows_takes_fp32_gemm():
    m, c = _mod4(bias=True)
    x = torch.randn(20, 300).to(torch.bfloat16)
    y = m(x)
    ref = F.linear(x.float(), m._dequant(torch.float32), m.bias.float()).to(torch.bfloat16)
    assert torch.equal(y, ref)


@pytest.mark.parametrize("rows", [1, 4, 20])
def test_prepare_fused_on_cpu_binds_the_cpu_int4_gemm(rows):
    """worker_quant.py:725-815: on a CPU device the int4 module binds torch's CPU int4 GEMM over
    the same codes (no re-quantization), releases qweight / scale / zero, and serves every row
    count from it; its results stay within the binding's self-check bar of the exact product."""
    m, c = _mod4(bias=True)
    m.prepare_fused()
    m.prepare_fused()                                    # idempotent
    assert m._fused_tried and m._fused is not None
    assert m._fused[2] is torch.ops.aten._weight_int4pack_mm_for_cpu and m._fused[3] == 384
    assert m.qweight is None and m.scale is None and m.zero is None
    x = torch.randn(rows, 300).to(torch.bfloat16)
    y = m(x)
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (rows, 48)
    exact = oq.linear_ref(x.float().numpy(), c["Wd"]) + m.bias.detach().float().numpy()
    yn = y.detach().float().numpy()
    assert oq.mean_rel(yn, exact) < 0.05 and oq.max_rel(yn, exact) < 2e-2


def test_prepare_fused_on_cpu_int2_stays_naive():
    c = C.int2_random_case(40, 256, 64, 2000, "fp16")
    m = wq._quant2_linear_cls()(C.u8(c["q"], "cpu"), C.to_torch(c["s"], "fp16", "cpu"),
                                C.to_torch(c["z"], "fp16", "cpu"), None, 256, 64)
    m.prepare_fused()
    assert getattr(m, "_fused", None) is None and m._fused_tried and m.qweight is not None


def test_int8_module_cpu():
    c = C.int8_case(32, 256)
    m = wq._quant_linear_cls()(C.u8(c["q"], "cpu"), C.to_torch(c["s"], "bf16", "cpu"), None)
    x = torch.randn(4, 256).to(torch.bfloat16)
    assert torch.equal(m(x), F.linear(x, m.qweight.to(torch.bfloat16) * m.scale))
    m.prepare_fused()
    assert getattr(m, "_w8", None) is None


def test_packed4_3d_getitem_cpu():
    r = np.random.default_rng(9)
    W3 = oq.round_to((r.standard_normal((3, 32, 256)) * 0.02).astype(np.float32), "bf16")
    p = wq._pack4_3d(torch.from_numpy(W3).to(torch.bfloat16))
    for e in range(3):
        ref = oq.dequant_int4_3d(p.qweight.numpy(), p.scale.float().numpy(), p.zero.float().numpy(), e, 256)
        assert np.array_equal(p[e].float().numpy(), ref)


def test_m_bucket_and_rows():
    assert [wq._m_bucket(m) for m in (0, 1, 2, 3, 5, 16, 17, 2048)] == [0, 1, 2, 4, 8, 16, 32, 2048]
    assert wq._rows(torch.empty(2, 3, 7)) == 6


def test_walker_skips_routers():
    class OlmoeTopKRouter(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.proj = torch.nn.Linear(128, 8)

    class Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.q_proj = torch.nn.Linear(128, 128)
            self.gate = torch.nn.Linear(128, 8)          # bare router leaf
            self.router = OlmoeTopKRouter()             # router subtree
            self.mlp = torch.nn.Sequential(torch.nn.Linear(128, 256), torch.nn.Linear(256, 128))

    b = Block().to(torch.bfloat16)
    wq._quantize_int4_(b)
    QL4 = wq._quant4_linear_cls()
    assert isinstance(b.q_proj, QL4) and isinstance(b.mlp[0], QL4) and isinstance(b.mlp[1], QL4)
    assert type(b.gate) is torch.nn.Linear and type(b.router.proj) is torch.nn.Linear
    b2 = Block().to(torch.bfloat16)
    wq._quantize_int8_linears_(b2)
    assert isinstance(b2.q_proj, wq._quant_linear_cls()) and type(b2.gate) is torch.nn.Linear


def test_experts_walker_packs_3d_params():
    from transformers.models.olmoe.configuration_olmoe import OlmoeConfig
    from transformers.models.olmoe.modeling_olmoe import OlmoeExperts
    cfg = OlmoeConfig(hidden_size=128, intermediate_size=64, num_experts=4, num_experts_per_tok=2)
    ex = OlmoeExperts(cfg).to(torch.bfloat16)
    with torch.no_grad():
        ex.gate_up_proj.normal_(0, 0.02)
        ex.down_proj.normal_(0, 0.02)
    holder = torch.nn.Module()
    holder.experts = ex
    wq._quantize_experts4_(holder)
    PT = wq._packed4_3d_cls()
    assert isinstance(ex.gate_up_proj, PT) and isinstance(ex.down_proj, PT)
    assert tuple(ex.gate_up_proj.qweight.shape) == (4, 128, 64)
    assert tuple(ex.down_proj.qweight.shape) == (4, 128, 64)   # K=64 pads to one 128 group
    assert ex.down_proj.in_features == 64
    # on CPU the eager forward runs over the dequantized experts
    x = torch.randn(3, 128).to(torch.bfloat16)
    idx = torch.tensor([[0, 1], [2, 3], [1, 2]])
    w = torch.rand(3, 2).to(torch.bfloat16)
    y = ex(x, idx, w)
    assert tuple(y.shape) == (3, 128) and torch.isfinite(y.float()).all()


def test_expert_ids_outside_range_are_refused():
    """The MoE ops refuse routing ids outside [0, E) as the reference's eager loop does
    (one_hot(num_classes=E) raises) instead of routing them to some expert."""
    import torch
    from infinitemodel_amd import ops
    ops._check_expert_ids(torch.tensor([[0, 63], [5, 7]], dtype=torch.int32), 64)
    ops._check_expert_ids(torch.zeros((0, 8), dtype=torch.int32), 64)
    for bad in ([[0, 64]], [[-1, 3]]):
        with pytest.raises(ValueError, match=r"\[0, 64\)"):
            ops._check_expert_ids(torch.tensor(bad, dtype=torch.int32), 64)
