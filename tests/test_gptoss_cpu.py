"""gpt-oss experts host logic without a GPU: block detection, the transpose-pack of the in-major
experts (bit-identical to the cache packer's in_major recipe), the dedicated forward install and
its refusal without the fused kernel, the cache compiler's refusal of in-major experts, and the
kernel layout's K padding of a Packed4Tensor3D."""
import numpy as np
import pytest

from oracle import quant as oq
from tests import _cases as C


def _gptoss(E=4, H=320, I=160, k=2, seed=1):
    import torch
    from transformers import GptOssConfig
    from transformers.models.gpt_oss.modeling_gpt_oss import GptOssExperts
    cfg = GptOssConfig(hidden_size=H, intermediate_size=I, num_local_experts=E, num_experts_per_tok=k,
                       num_hidden_layers=1, num_attention_heads=4, num_key_value_heads=4, head_dim=16)
    mod = GptOssExperts(cfg).to(torch.bfloat16)
    r = C.rng(seed)
    with torch.no_grad():
        for p in mod.parameters():
            p.copy_(torch.from_numpy(C.bf16_normal(r, tuple(p.shape), 0.05)))
    return mod


def test_is_gptoss_experts():
    from transformers import OlmoeConfig
    from transformers.models.olmoe.modeling_olmoe import OlmoeExperts
    from infinitemodel_amd import worker_quant as wq
    assert wq._is_gptoss_experts(_gptoss())
    cfg = OlmoeConfig(hidden_size=64, intermediate_size=32, num_experts=4, num_experts_per_tok=2,
                      num_hidden_layers=1, num_attention_heads=4, num_key_value_heads=4)
    assert not wq._is_gptoss_experts(OlmoeExperts(cfg))


def test_quantize_experts4_transpose_packs_gptoss():
    """gate_up [E, H, 2I] / down [E, I, H] are packed as their [E, out, in] transposes, byte for
    byte the cache packer's in_major=True result and the oracle's; the experts keep their own
    implementation (no eager switch) and get the dedicated forward."""
    import torch
    from infinitemodel_amd import shard_compile as sc
    from infinitemodel_amd import worker_quant as wq
    mod = _gptoss()
    gu_in = mod.gate_up_proj.detach().clone()
    dn_in = mod.down_proj.detach().clone()
    wq._quantize_experts4_(mod)
    assert getattr(mod, "_gptoss_fused_installed", False)
    assert getattr(mod.config, "_experts_implementation", None) != "eager"
    for holder, W in ((mod.gate_up_proj, gu_in), (mod.down_proj, dn_in)):
        q, s, z, in_f, _ng = sc.pack_linear_int4_3d(W, 128, in_major=True)
        assert torch.equal(holder.qweight, q) and torch.equal(holder.scale, s) and torch.equal(holder.zero, z)
        assert holder.in_features == W.shape[1] == in_f
        oq_q, oq_s, oq_z, _, _ = oq.pack_linear_int4_3d(W.float().numpy(), 128, "bf16", in_major=True)
        assert np.array_equal(holder.qweight.numpy(), oq_q)
        assert np.array_equal(holder.scale.float().numpy(), oq_s)
    # negative control: the square-free shapes make a missed transpose visible as a shape error,
    # the values make it visible on a square expert too
    W = torch.from_numpy(C.bf16_normal(C.rng(3), (2, 256, 256), 0.05)).to(torch.bfloat16)
    a = sc.pack_linear_int4_3d(W, 128, in_major=True)[0]
    b = sc.pack_linear_int4_3d(W, 128)[0]
    assert not torch.equal(a, b)


def test_quantize_experts4_gptoss_refuses_without_fused_kernel(monkeypatch):
    from infinitemodel_amd import worker_quant as wq
    monkeypatch.setenv("INFINITEMODEL_NO_FUSED_MOE", "1")
    mod = _gptoss()
    with pytest.raises(RuntimeError, match="gpt-oss int4 requires the fused"):
        wq._quantize_experts4_(mod)
    assert mod.gate_up_proj.dim() == 3 and mod.gate_up_proj.dtype.is_floating_point   # untouched


def test_cache_compile_refuses_in_major_experts():
    import torch
    from infinitemodel_amd import shard_compile as sc
    W = torch.zeros((2, 128, 256), dtype=torch.bfloat16)
    raw = {"model.layers.0.mlp.experts.gate_up_proj": W,
           "model.layers.0.mlp.experts.gate_up_proj_bias": torch.zeros((2, 256), dtype=torch.bfloat16)}
    with pytest.raises(ValueError, match="in-major"):
        sc.pack_unit_tensors(raw, None, "int4")
    out, _ = sc.pack_unit_tensors({"model.layers.0.mlp.experts.gate_up_proj": W}, None, "int4")
    assert "model.layers.0.mlp.experts.gate_up_proj.qweight" in out


def test_kernel_tensors_pad_k_to_256():
    """A holder of K_pad 2944 (23 groups) gets a 3072-wide kernel layout; its own buffers become
    views of it with unchanged shapes and values, the pad is zero, and the call is idempotent."""
    import torch
    from infinitemodel_amd import worker_quant as wq
    PT = wq._packed4_3d_cls()
    E, N, in_f = 2, 64, 2880
    r = C.rng(5)
    q = torch.from_numpy(r.integers(0, 256, (E, N, 1472), dtype=np.uint8))
    s = torch.from_numpy(C.bf16_normal(r, (E, N, 23), 0.01)).to(torch.bfloat16)
    z = torch.from_numpy(r.integers(0, 16, (E, N, 23)).astype(np.float32)).to(torch.bfloat16)
    h = PT(q.clone(), s.clone(), z.clone(), in_f, 128)
    kq, ks, kz = h._kernel_tensors()
    assert kq.shape == (E, N, 1536) and ks.shape == (E, N, 24) and kz.shape == (E, N, 24)
    assert h.qweight.shape == q.shape and torch.equal(h.qweight, q)
    assert torch.equal(h.scale, s) and torch.equal(h.zero, z)
    assert h.qweight.data_ptr() == kq.data_ptr()
    assert not kq[:, :, 1472:].any() and not ks[:, :, 23:].float().any() and not kz[:, :, 23:].float().any()
    assert h._kernel_tensors()[0] is kq
    sd = h.state_dict()
    assert torch.equal(sd["qweight"], q)
    # already aligned: the buffers themselves
    h2 = PT(q[:, :, :1024].clone(), s[:, :, :16].clone(), z[:, :, :16].clone(), 2048, 128)
    assert h2._kernel_tensors()[0] is h2.qweight
