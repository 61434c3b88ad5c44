"""GPU parity of the int8 fused 3D experts (Packed8Tensor3D + the w8a16 expert subclass in the
eager experts loop) and of the int8 lm_head option, against the oracle's int8 pack and the exact
float64 products over the dequantized weights.

Tolerance: normwise max relative error <= 1e-2, mean relative error <= 5e-3."""
import numpy as np
import pytest

from oracle import moe as om
from oracle import quant as oq
from tests import _cases as C

pytestmark = pytest.mark.gpu

MAX_REL = 1e-2
MEAN_REL = 5e-3


def _olmoe(E, H, I, k, seed):
    import torch
    from transformers.models.olmoe.configuration_olmoe import OlmoeConfig
    from transformers.models.olmoe.modeling_olmoe import OlmoeExperts
    cfg = OlmoeConfig(hidden_size=H, intermediate_size=I, num_experts=E, num_experts_per_tok=k)
    ex = OlmoeExperts(cfg).to(torch.bfloat16)
    r = C.rng(seed)
    with torch.no_grad():
        ex.gate_up_proj.copy_(torch.from_numpy(C.bf16_normal(r, tuple(ex.gate_up_proj.shape), 0.02)))
        ex.down_proj.copy_(torch.from_numpy(C.bf16_normal(r, tuple(ex.down_proj.shape), 0.02)))
    return ex


@pytest.mark.parametrize("T", [1, 6])
def test_int8_experts_eager_loop(dev, T):
    """int8 experts through transformers' eager loop: each routed expert's F.linear runs the HIP
    w8a16 op on the int8 bytes (the subclass path is taken), the layer matches the exact MoE
    over the int8-dequantized experts."""
    import torch
    from infinitemodel_amd import worker_quant as wq
    E, H, I, k = 8, 512, 256, 2
    ex = _olmoe(E, H, I, k, seed=11)
    Wg = ex.gate_up_proj.detach().float().numpy()
    Wd = ex.down_proj.detach().float().numpy()
    wq._quantize_experts8_(ex)
    Dg = np.stack([oq.dequant_int8(*oq.pack_linear_int8(Wg[e], "bf16"), "bf16")[0] for e in range(E)])
    Dd = np.stack([oq.dequant_int8(*oq.pack_linear_int8(Wd[e], "bf16"), "bf16")[0] for e in range(E)])
    ex.to(dev)
    w0 = ex.gate_up_proj[0]
    assert type(w0).__name__ == "_W8A16Weight" and ex.gate_up_proj._expert_kernel
    r = C.rng(12 + T)
    idx, w = om.route_topk(r.standard_normal((T, E)).astype(np.float32), k)
    x = C.bf16_normal(r, (T, H))
    with torch.no_grad():
        y = C.t2np(ex(C.to_torch(x, "bf16", dev), torch.from_numpy(idx).to(dev), C.to_torch(w, "bf16", dev)))
    exact = om.moe_exact(x, idx, w, Dg, Dd)
    eager = om.moe_eager_bf16(x, idx, w, Dg, Dd)
    assert oq.max_rel(y, exact) <= 2e-2 and oq.mean_rel(y, eager) < 1e-2, (oq.max_rel(y, exact), oq.mean_rel(y, eager))


def test_int8_expert_subclass_linear(dev):
    """F.linear on one expert's subclass == the kernel-form int8 product (scale * x @ q^T)."""
    import torch
    import torch.nn.functional as F
    from infinitemodel_amd import worker_quant as wq
    W3 = torch.from_numpy(C.bf16_normal(C.rng(21), (3, 384, 640), 0.05)).to(torch.bfloat16)
    h = wq._pack8_3d(W3).to(dev)
    x = C.bf16_normal(C.rng(22), (5, 640))
    for e in range(3):
        w = h[e]
        assert type(w).__name__ == "_W8A16Weight"
        y = C.t2np(F.linear(C.to_torch(x, "bf16", dev), w))
        ref = oq.int8_gemm_ref(x, h.qweight[e].cpu().numpy(), h.scale[e].float().cpu().numpy())
        assert oq.max_rel(y, ref) <= MAX_REL and oq.mean_rel(y, ref) <= MEAN_REL
        # any other op materializes the dequantized weight
        assert torch.equal((w * 1).cpu(), (h.qweight[e].to(torch.bfloat16) * h.scale[e]).cpu())


def test_int8_head_quant_on_gpu(dev):
    """head_quant=int8 replaces a GPU nn.Linear head with an int8 QuantLinear whose decode rows
    match the kernel-form product over its own packed weight."""
    import torch
    from infinitemodel_amd import worker_quant as wq

    class M(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.config = type("Cfg", (), {"tie_word_embeddings": False})()
            self.lm_head = torch.nn.Linear(1024, 32000, bias=False)

    m = M().to(torch.bfloat16)
    with torch.no_grad():
        m.lm_head.weight.copy_(torch.from_numpy(C.bf16_normal(C.rng(31), (32000, 1024), 0.02)))
    m.lm_head.to(dev)
    head = wq.apply_head_quant(m, m.lm_head, "int8")
    assert isinstance(head, wq._quant_linear_cls()) and m.lm_head is head
    assert head.qweight.device == dev
    wq.finalize_placement(m)
    x = C.bf16_normal(C.rng(32), (2, 1024))
    with torch.no_grad():
        y = C.t2np(head(C.to_torch(x, "bf16", dev)))
    # the packed weight in the reference's row layout (the bound module may hold it line-tiled)
    ref = oq.int8_gemm_ref(x, head.state_dict()["qweight"].cpu().numpy(), head.scale.float().cpu().numpy())
    assert oq.max_rel(y, ref) <= MAX_REL and oq.mean_rel(y, ref) <= MEAN_REL
