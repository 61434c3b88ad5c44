"""The module boundary the reference's main caller binds (client.py:539-549), on the CPU: every
name it imports from worker_quant exists here, and the load-time helpers behind those names
behave as the caller relies on -- streamed expert builds equal the in-memory quantizers, the MoE
layer predicates, the CPU device bridge, meta materialization and the CPU thread / fp32 helpers."""
import numpy as np
import pytest
import torch
from torch import nn
import torch.nn.functional as F

from infinitemodel_amd import worker_quant as wq

# client.py:539-549, the caller's import list, kept as data.
CLIENT_IMPORTS = (
    "_quantize_int4_", "_quantize_int8_", "_quantize_experts4_", "_quantize_linear", "_quantize_linear4",
    "_assign_meta_from_sd", "_accelerate_cpu_linears", "tune_cpu_threads", "_find_moe_block", "_moe_bridge_cls",
    "_model_has_fused_experts", "_model_has_nonfused_experts", "_layer_has_meta_experts",
    "_layer_has_meta_experts_nonfused", "_quantize_experts4_streamed", "_quantize_experts4_streamed_nonfused",
    "_quant4_linear_cls", "_packed4_3d_cls", "_INT4_GROUP", "_install_fused_moe_forward", "_w4a16_triton_op",
    "_w4a16_moe_op", "_pack4_expert", "_pack4_3d", "_quantize_int2_", "_quantize_linear2", "_quant2_linear_cls",
    "_INT2_GROUP",
)


def test_every_name_the_client_imports_is_exported():
    assert len(CLIENT_IMPORTS) == 28
    missing = [n for n in CLIENT_IMPORTS if not hasattr(wq, n)]
    assert not missing, missing


# ---- MoE fixtures: a fused-3D experts block and a per-expert ModuleList block ------------------
class _FusedExperts(nn.Module):
    def __init__(self, E, H, I, meta=False):
        super().__init__()
        dev = "meta" if meta else "cpu"
        g = torch.Generator().manual_seed(5)
        gu = torch.randn(E, 2 * I, H, generator=g) * 0.02
        dn = torch.randn(E, H, I, generator=g) * 0.02
        self.gate_up_proj = nn.Parameter(gu.to(torch.bfloat16).to(dev), requires_grad=False)
        self.down_proj = nn.Parameter(dn.to(torch.bfloat16).to(dev), requires_grad=False)
        self.act_fn = nn.SiLU()


class _Expert(nn.Module):
    def __init__(self, H, I):
        super().__init__()
        self.w1 = nn.Linear(H, I, bias=False)
        self.w3 = nn.Linear(H, I, bias=False)
        self.w2 = nn.Linear(I, H, bias=False)


class _Layer(nn.Module):
    def __init__(self, block):
        super().__init__()
        self.self_attn = nn.Linear(8, 8)
        self.mlp = block


def _fused_weights(E=4, H=256, I=128):
    ref = _FusedExperts(E, H, I)
    return ref.gate_up_proj.data.clone(), ref.down_proj.data.clone()


@pytest.mark.parametrize("layout", ["fused", "per_expert"])
def test_streamed_fused_build_equals_in_memory_quantizer(layout, monkeypatch):
    """_quantize_experts4_streamed over a META layer (chunked fetches, both server layouts) gives
    holders bit-identical to _quantize_experts4_ over the materialized experts."""
    monkeypatch.setattr(wq, "_STREAM_CHUNK_BYTES", 3 * 2 * 128 * 256 * 2)     # 3 experts per fetch
    E, H, I = 7, 256, 128
    gu, dn = _fused_weights(E, H, I)
    full = _Layer(_FusedExperts(E, H, I))
    full.mlp.gate_up_proj = nn.Parameter(gu.clone(), requires_grad=False)
    full.mlp.down_proj = nn.Parameter(dn.clone(), requires_grad=False)
    wq._quantize_experts4_(full)
    streamed = _Layer(_FusedExperts(E, H, I, meta=True))
    assert wq._layer_has_meta_experts(streamed) and not wq._layer_has_meta_experts(full)
    calls = []

    def fetch(layer_idx, e0, k):
        calls.append((layer_idx, e0, k))
        if layout == "fused":
            return {"gate_up_proj": gu[e0:e0 + k], "down_proj": dn[e0:e0 + k]}
        blob = {}
        for j in range(k):
            blob[f"{j}.w1"], blob[f"{j}.w3"] = gu[e0 + j, :I], gu[e0 + j, I:]
            blob[f"{j}.w2"] = dn[e0 + j].t().contiguous()          # transposed: orientation detected
        return blob

    wq._quantize_experts4_streamed(streamed, 3, fetch, torch.bfloat16)
    assert calls == [(3, 0, 3), (3, 3, 3), (3, 6, 1)]
    PT = wq._packed4_3d_cls()
    for attr in ("gate_up_proj", "down_proj"):
        a, b = getattr(full.mlp, attr), getattr(streamed.mlp, attr)
        assert isinstance(b, PT) and b.in_features == a.in_features
        for t in ("qweight", "scale", "zero"):
            assert torch.equal(getattr(a, t), getattr(b, t)), (attr, t)
    assert streamed.mlp._fused_moe_installed is full.mlp._fused_moe_installed


def test_streamed_build_rejects_a_foreign_blob():
    E, H, I = 2, 256, 128
    layer = _Layer(_FusedExperts(E, H, I, meta=True))
    with pytest.raises(RuntimeError, match="expert blob key"):
        wq._quantize_experts4_streamed(layer, 0, lambda l, e0, k: {"gate_up_proj": torch.zeros(1)}, torch.bfloat16)
    with pytest.raises(RuntimeError, match="no gate / up"):
        wq._quantize_experts4_streamed(layer, 0, lambda l, e0, k: {"0.w2": torch.zeros(H, I)}, torch.bfloat16)


def test_streamed_nonfused_build_equals_in_memory_quantizer(monkeypatch):
    monkeypatch.setattr(wq, "_STREAM_CHUNK_BYTES", 2 * 3 * 128 * 256 * 2)   # 2 experts per fetch
    E, H, I = 5, 256, 128
    torch.manual_seed(3)
    src = [_Expert(H, I).to(torch.bfloat16) for _ in range(E)]
    full = _Layer(nn.Module())
    full.mlp.experts = nn.ModuleList([_Expert(H, I).to(torch.bfloat16) for _ in range(E)])
    full.mlp.experts.load_state_dict(nn.ModuleList(src).state_dict())
    with torch.device("meta"):
        meta_experts = nn.ModuleList([_Expert(H, I).to(torch.bfloat16) for _ in range(E)])
    streamed = _Layer(nn.Module())
    streamed.mlp.experts = meta_experts
    assert wq._model_has_nonfused_experts(streamed) and not wq._model_has_fused_experts(streamed)
    assert wq._layer_has_meta_experts_nonfused(streamed) and not wq._layer_has_meta_experts_nonfused(full)

    def fetch(layer_idx, e0, k):
        return {f"{j}.{p}": getattr(src[e0 + j], p).weight.data for j in range(k) for p in ("w1", "w3", "w2")}

    wq._quantize_experts4_streamed_nonfused(streamed, 1, fetch, torch.bfloat16)
    wq._quantize_int4_(full)
    QL = wq._quant4_linear_cls()
    for e in range(E):
        for p in ("w1", "w3", "w2"):
            a, b = getattr(full.mlp.experts[e], p), getattr(streamed.mlp.experts[e], p)
            assert isinstance(b, QL)
            for t in ("qweight", "scale", "zero"):
                assert torch.equal(getattr(a, t), getattr(b, t)), (e, p, t)


def test_find_moe_block_and_model_predicates():
    dense = _Layer(nn.Sequential(nn.Linear(8, 8)))
    assert wq._find_moe_block(dense) == (None, None)
    assert not wq._model_has_fused_experts(dense) and not wq._model_has_nonfused_experts(dense)
    fused = _Layer(_FusedExperts(2, 128, 64))
    assert wq._find_moe_block(fused) == ("mlp", fused.mlp)
    assert wq._model_has_fused_experts(fused)
    wq._quantize_experts4_(fused)                        # packed holders are still found
    assert wq._find_moe_block(fused) == ("mlp", fused.mlp)
    sparse = _Layer(nn.Module())
    sparse.mlp.experts = nn.ModuleList([_Expert(16, 8)])
    assert wq._find_moe_block(sparse) == ("mlp", sparse.mlp)


def test_moe_bridge_runs_the_block_on_its_device_and_returns_to_the_caller():
    seen = {}

    class Block(nn.Module):
        def forward(self, h, scale, *, shift):
            seen["dev"] = (h.device, scale.device, shift.device)
            return h * scale + shift, (h.sum(), 3)

    Bridge = wq._moe_bridge_cls()
    assert Bridge is wq._moe_bridge_cls()
    br = Bridge(Block(), torch.device("cpu"))
    h = torch.randn(2, 4)
    out, (s, three) = br(h, torch.tensor(2.0), shift=torch.tensor(1.0))
    assert seen["dev"] == (torch.device("cpu"),) * 3
    assert torch.equal(out, h * 2 + 1) and three == 3 and s.device == h.device


def test_assign_meta_from_sd_materializes_skipped_tensors():
    class Router(nn.Module):
        def __init__(self):
            super().__init__()
            self.weight = nn.Parameter(torch.empty(4, 8, device="meta"))
            self.register_buffer("e_score_correction_bias", torch.empty(4, device="meta"), persistent=False)

    class Mlp(nn.Module):
        def __init__(self):
            super().__init__()
            self.gate = Router()
            self.experts = nn.Module()

    model = nn.Module()
    model.mlp = Mlp()
    sd = {"mlp.gate.weight": torch.ones(4, 8), "mlp.experts.e_score_correction_bias": torch.arange(4.0),
          "mlp.nowhere.thing": torch.zeros(3)}
    assert wq._assign_meta_from_sd(model, sd) == 2
    assert isinstance(model.mlp.gate.weight, nn.Parameter) and not model.mlp.gate.weight.requires_grad
    assert torch.equal(model.mlp.gate.weight, torch.ones(4, 8))
    # the bias lives on the router (sibling of 'experts'), as transformers builds it
    assert torch.equal(model.mlp.gate.e_score_correction_bias, torch.arange(4.0))
    assert "e_score_correction_bias" not in model.mlp.gate.state_dict()
    assert wq._assign_meta_from_sd(model, sd) == 0      # nothing meta is left


def test_tune_cpu_threads_honours_the_environment(monkeypatch):
    before = torch.get_num_threads()
    try:
        monkeypatch.setenv("OMP_NUM_THREADS", "3")
        assert wq.tune_cpu_threads() is None
        assert torch.get_num_threads() == 3
        monkeypatch.setenv("OMP_NUM_THREADS", "999")
        wq.tune_cpu_threads()
        assert torch.get_num_threads() == 128
    finally:
        torch.set_num_threads(before)


def test_accelerate_cpu_linears_takes_fp32_from_16_rows():
    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(64, 32).to(torch.bfloat16), nn.ReLU())
    q = wq._quantize_linear4(nn.Linear(256, 16).to(torch.bfloat16))
    model.add_module("q", q)
    lin = model[0]
    wq._accelerate_cpu_linears(model)
    wq._accelerate_cpu_linears(model)                   # idempotent
    assert lin._im_fp32_wrapped and not getattr(q, "_im_fp32_wrapped", False)
    for rows, fp32 in ((4, False), (16, True)):
        x = torch.randn(rows, 64).to(torch.bfloat16)
        with torch.no_grad():
            y = lin(x)
            want = (F.linear(x.float(), lin.weight.float(), lin.bias.float()).to(torch.bfloat16) if fp32
                    else F.linear(x, lin.weight, lin.bias))
        assert y.dtype == torch.bfloat16 and torch.equal(y, want), rows
    assert np.isfinite(y.float().numpy()).all()
