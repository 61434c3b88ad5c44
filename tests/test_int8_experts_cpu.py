"""int8 fused 3D experts and the int8 lm_head option without a GPU: Packed8Tensor3D packing
(twin identity with the 2D int8 packer and the oracle), its eager-loop dequant, the int8 layer
walker (routers kept, experts packed, eager implementation forced), its refusals (gpt-oss, meta
experts) and the head_quant decisions that keep a head bf16."""
import numpy as np
import pytest
import torch

from oracle import quant as oq
from infinitemodel_amd import shard_compile as sc
from infinitemodel_amd import worker_quant as wq
from tests import _cases as C


def _olmoe_experts(E=4, H=128, I=64, seed=3):
    from transformers.models.olmoe.configuration_olmoe import OlmoeConfig
    from transformers.models.olmoe.modeling_olmoe import OlmoeExperts
    cfg = OlmoeConfig(hidden_size=H, intermediate_size=I, num_experts=E, num_experts_per_tok=2)
    cfg._experts_implementation = "grouped_mm"
    ex = OlmoeExperts(cfg).to(torch.bfloat16)
    r = C.rng(seed)
    with torch.no_grad():
        ex.gate_up_proj.copy_(torch.from_numpy(C.bf16_normal(r, tuple(ex.gate_up_proj.shape), 0.05)))
        ex.down_proj.copy_(torch.from_numpy(C.bf16_normal(r, tuple(ex.down_proj.shape), 0.05)))
    return ex


def test_pack8_3d_is_the_2d_packer_per_expert():
    W3 = torch.from_numpy(C.bf16_normal(C.rng(1), (3, 40, 72), 0.1)).to(torch.bfloat16)
    W3[1, 5] = 0                                            # an all-zero row: the 1e-8 scale floor
    h = wq._pack8_3d(W3)
    assert isinstance(h, wq._packed8_3d_cls()) and h.in_features == 72
    assert h.qweight.dtype == torch.int8 and tuple(h.scale.shape) == (3, 40, 1) and h.scale.dtype == W3.dtype
    for e in range(3):
        q, s = sc.pack_linear_int8(W3[e])
        assert torch.equal(h.qweight[e], q) and torch.equal(h.scale[e], s)
        oq_q, oq_s = oq.pack_linear_int8(W3[e].float().numpy(), "bf16")
        assert np.array_equal(h.qweight[e].numpy(), oq_q)
        assert np.array_equal(h.scale[e].float().numpy(), oq_s)
    assert torch.equal(h[1], (h.qweight[1].to(torch.bfloat16) * h.scale[1]))


def test_quantize_int8_packs_linears_and_experts_keeps_router():
    class Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.q_proj = torch.nn.Linear(128, 128, bias=False)
            self.gate = torch.nn.Linear(128, 4, bias=False)     # router leaf
            self.experts = _olmoe_experts()

    b = Block().to(torch.bfloat16)
    gu = b.experts.gate_up_proj.detach().clone()
    wq._quantize_int8_(b)
    PT8 = wq._packed8_3d_cls()
    assert isinstance(b.q_proj, wq._quant_linear_cls()) and type(b.gate) is torch.nn.Linear
    assert isinstance(b.experts.gate_up_proj, PT8) and isinstance(b.experts.down_proj, PT8)
    assert b.experts.config._experts_implementation == "eager"
    assert torch.equal(b.experts.gate_up_proj.qweight, torch.stack([sc.pack_linear_int8(gu[e])[0] for e in range(4)]))
    # the eager loop over the holders is the eager loop over the dequantized experts
    ex = b.experts
    ref = _olmoe_experts()
    ref.config._experts_implementation = "eager"
    with torch.no_grad():
        ref.gate_up_proj.copy_(torch.stack([ex.gate_up_proj[e] for e in range(4)]))
        ref.down_proj.copy_(torch.stack([ex.down_proj[e] for e in range(4)]))
    x = torch.from_numpy(C.bf16_normal(C.rng(4), (5, 128))).to(torch.bfloat16)
    idx = torch.tensor([[0, 1], [2, 3], [1, 2], [3, 0], [2, 1]])
    w = torch.rand(5, 2, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    assert torch.equal(ex(x, idx, w), ref(x, idx, w))


def test_quantize_experts8_refuses_gptoss_and_meta():
    from transformers import GptOssConfig
    from transformers.models.gpt_oss.modeling_gpt_oss import GptOssExperts
    cfg = GptOssConfig(hidden_size=64, intermediate_size=32, num_local_experts=2, num_experts_per_tok=1,
                       num_hidden_layers=1, num_attention_heads=4, num_key_value_heads=4, head_dim=16)
    with pytest.raises(RuntimeError, match="gpt-oss"):
        wq._quantize_experts8_(GptOssExperts(cfg))
    from transformers.models.olmoe.configuration_olmoe import OlmoeConfig
    from transformers.models.olmoe.modeling_olmoe import OlmoeExperts
    with torch.device("meta"):
        meta = OlmoeExperts(OlmoeConfig(hidden_size=64, intermediate_size=32, num_experts=2,
                                        num_experts_per_tok=1))
    with pytest.raises(RuntimeError, match="META"):
        wq._quantize_experts8_(meta)
    wq._quantize_experts8_(torch.nn.Linear(4, 4))            # no fused experts: a no-op


def test_head_quant_keeps_bf16_where_the_reference_does():
    class M(torch.nn.Module):
        def __init__(self, tied):
            super().__init__()
            self.config = type("Cfg", (), {"tie_word_embeddings": tied})()
            self.lm_head = torch.nn.Linear(64, 100, bias=False)

    m = M(False)
    assert wq.apply_head_quant(m, m.lm_head, "int8") is m.lm_head          # CPU head: stays bf16
    # a pack that cannot reach its device (no GPU here) keeps the head as built
    assert wq.apply_head_quant(m, m.lm_head, "int8", "cuda:0") is m.lm_head
    mt = M(True)
    assert wq.apply_head_quant(mt, mt.lm_head, "int8", torch.device("cuda", 0)) is mt.lm_head   # tied
    assert wq.apply_head_quant(m, m.lm_head, "int4", torch.device("cuda", 0)) is m.lm_head      # refused
    assert wq.apply_head_quant(m, m.lm_head, "bf16") is m.lm_head
    assert wq.apply_head_quant(m, m.lm_head, "") is m.lm_head
    q = wq._quantize_linear(torch.nn.Linear(64, 100, bias=False))
    assert wq.apply_head_quant(m, q, "int8", torch.device("cuda", 0)) is q                     # already packed
