"""Serve-from-cache: a `_shards/<quant>/` cache written from a model and installed into a fresh
model equals a cold load (the reference's twin identity, scratch_moe_int8_pack_test.py:129-142 and
scratch_gptoss_pack_layout_test.py:64-106), the verifier catches corrupt / missing / foreign
units (shard_compile.py:701-736), and the installer refuses the packs the reference refuses
(shard_build.py:934-1030). CPU only: the modules run the reference's CPU semantics."""
import copy
import os

import pytest

torch = pytest.importorskip("torch")
transformers = pytest.importorskip("transformers")

from infinitemodel_amd import shard_compile as sc          # noqa: E402
from infinitemodel_amd import shard_install as si          # noqa: E402
from infinitemodel_amd import worker_quant as wq           # noqa: E402


def _llama(seed, layers=2):
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(seed)
    cfg = LlamaConfig(vocab_size=320, hidden_size=256, intermediate_size=384, num_hidden_layers=layers,
                      num_attention_heads=4, num_key_value_heads=2, tie_word_embeddings=False,
                      bos_token_id=0, eos_token_id=1, pad_token_id=2)
    return LlamaForCausalLM(cfg).to(torch.bfloat16).eval()


def _olmoe(seed):
    from transformers import OlmoeConfig, OlmoeForCausalLM
    torch.manual_seed(seed)
    cfg = OlmoeConfig(vocab_size=320, hidden_size=256, intermediate_size=128, num_hidden_layers=1,
                      num_attention_heads=4, num_key_value_heads=4, num_experts=8, num_experts_per_tok=2,
                      bos_token_id=0, eos_token_id=1, pad_token_id=2)
    return OlmoeForCausalLM(cfg).to(torch.bfloat16).eval()


def _units(model):
    """{unit file: {name: tensor}}: embed, one file per decoder layer, head (norm + lm_head)."""
    sd = {k: v.detach().clone() for k, v in model.state_dict().items()}
    n = model.config.num_hidden_layers
    units = {"embed.safetensors": {"model.embed_tokens.weight": sd.pop("model.embed_tokens.weight")},
             "head.safetensors": {"model.norm.weight": sd.pop("model.norm.weight"),
                                  "lm_head.weight": sd.pop("lm_head.weight")}}
    for i in range(n):
        pre = f"model.layers.{i}."
        units[f"L{i:04d}.safetensors"] = {k: sd.pop(k) for k in list(sd) if k.startswith(pre)}
    assert not [k for k in sd if not k.endswith("inv_freq")], sorted(sd)
    return units


def _cold(model, quant):
    """Load-time quantization, per decoder layer as the reference's _quant_after does."""
    m = copy.deepcopy(model)
    for lyr in m.model.layers:
        if quant == "int4":
            wq._quantize_int4_(lyr)
            wq._quantize_experts4_(lyr)
        elif quant == "int2":
            wq._quantize_int2_(lyr)
        else:
            wq._quantize_int8_linears_(lyr)
    if quant == "int8":
        m.lm_head = wq._quantize_linear(m.lm_head)
    return m


def _from_cache(tmp_path, quant, fresh):
    d = os.path.join(str(tmp_path), "_shards", quant)
    head = fresh.lm_head
    for f in sorted(os.listdir(d)):
        if not f.endswith(".safetensors"):
            continue
        from safetensors.torch import load_file
        r = si.install_cached(fresh, load_file(os.path.join(d, f)), quant, torch.bfloat16, head=head)
        head = r["head"]
    si.install_fused_moe_sweep(fresh)
    return fresh


def _assert_same_state(a, b):
    sa, sb = a.state_dict(), b.state_dict()
    assert sorted(sa) == sorted(sb)
    for k in sa:
        assert sa[k].dtype == sb[k].dtype, k
        assert torch.equal(sa[k], sb[k]), k


@pytest.mark.parametrize("quant", ["int4", "int2", "int8"])
def test_cache_install_equals_cold_load_dense(tmp_path, quant):
    src = _llama(0)
    lin2d, exp3d = sc.quant_scope(src)
    assert len(lin2d) == 2 * 7 and not exp3d
    man = sc.write_cache(str(tmp_path), _units(src), quant, 128, num_layers=2, lin2d=lin2d)
    assert man["quant"] == quant and man["num_layers"] == 2 and len(man["files"]) == 4
    ok, problems = sc.verify_shard_cache(str(tmp_path), quant)
    assert ok, problems
    cold = _cold(src, quant)
    warm = _from_cache(tmp_path, quant, _llama(1))
    _assert_same_state(cold, warm)
    kinds = {type(m).__name__ for m in warm.modules()}
    assert {"int4": "QuantLinear4", "int2": "QuantLinear2", "int8": "QuantLinear"}[quant] in kinds
    assert (type(warm.lm_head).__name__ == "QuantLinear") == (quant == "int8")
    ids = torch.tensor([[3, 17, 255, 40, 9, 100, 7]])
    with torch.no_grad():
        assert torch.equal(cold(ids).logits, warm(ids).logits)


def test_cache_install_equals_cold_load_moe_experts(tmp_path):
    src = _olmoe(0)
    lin2d, exp3d = sc.quant_scope(src)
    assert "model.layers.0.mlp.gate.weight" not in lin2d          # the router stays bf16
    assert exp3d == {"model.layers.0.mlp.experts.gate_up_proj", "model.layers.0.mlp.experts.down_proj"}
    man = sc.write_cache(str(tmp_path), _units(src), "int4", 128, num_layers=1, lin2d=lin2d)
    assert man["expert_layout"] == "fused3d"
    assert sc.verify_shard_cache(str(tmp_path), "int4")[0]
    cold = _cold(src, "int4")
    warm = _from_cache(tmp_path, "int4", _olmoe(1))
    _assert_same_state(cold, warm)
    ex = warm.model.layers[0].mlp.experts
    assert type(ex.gate_up_proj).__name__ == "Packed4Tensor3D" and ex.gate_up_proj.in_features == 256
    assert type(warm.model.layers[0].mlp.gate).__name__ != "QuantLinear4"
    assert warm.config._experts_implementation == "eager"
    ids = torch.tensor([[3, 17, 255, 40, 9]])
    with torch.no_grad():
        assert torch.equal(cold(ids).logits, warm(ids).logits)


def test_verify_catches_corrupt_missing_and_foreign_units(tmp_path):
    src = _llama(0, layers=1)
    sc.write_cache(str(tmp_path), _units(src), "int4", 128, num_layers=1, lin2d=sc.quant_scope(src)[0])
    d = os.path.join(str(tmp_path), "_shards", "int4")
    assert sc.verify_shard_cache(str(tmp_path), "int4") == (True, [])
    p = os.path.join(d, "L0000.safetensors")
    data = bytearray(open(p, "rb").read())
    data[-5] ^= 0xFF                                         # same size, different bytes
    open(p, "wb").write(bytes(data))
    ok, probs = sc.verify_shard_cache(str(tmp_path), "int4")
    assert not ok and any(s.startswith("L0000.safetensors: sha256 differs") for s in probs)
    open(p, "wb").write(bytes(data[:-1]))                    # truncated
    assert any(s.startswith("L0000.safetensors: ") and "bytes on disk" in s
               for s in sc.verify_shard_cache(str(tmp_path), "int4")[1])
    os.remove(os.path.join(d, "head.safetensors"))
    assert any(s.startswith("head.safetensors: ") and "absent" in s
               for s in sc.verify_shard_cache(str(tmp_path), "int4")[1])
    import json
    mf = os.path.join(d, "manifest.json")
    man = json.load(open(mf))
    man["packer_hash"] = "rtn-int4-g64-v0"
    man["files"].pop("head.safetensors")
    json.dump(man, open(mf, "w"))
    probs = sc.verify_shard_cache(str(tmp_path), "int4")[1]
    assert any("packer tag" in s for s in probs) and any("incomplete" in s for s in probs)
    os.remove(mf)
    assert sc.verify_shard_cache(str(tmp_path), "int4") == (False, ["no manifest.json"])


def test_install_refusals():
    m = _llama(0, layers=1)
    q = torch.zeros(384, 128, dtype=torch.uint8)
    s = torch.ones(384, 2, dtype=torch.bfloat16)
    base = "model.layers.0.mlp.gate_proj.weight"
    # int4 / int2 need the zero point
    with pytest.raises(si.CacheInstallError, match="incomplete"):
        si.install_cached(m, {base + ".qweight": q, base + ".scale": s}, "int4")
    # int8 packs are symmetric: a zero point means a foreign pack
    with pytest.raises(si.CacheInstallError, match="zero point"):
        si.install_cached(m, {base + ".qweight": q.to(torch.int8), base + ".scale": s[:, :1],
                              base + ".zero": s}, "int8")
    # 3D expert tensors exist only at int4
    with pytest.raises(si.CacheInstallError, match="only int4"):
        e = "model.layers.0.mlp.experts.gate_up_proj"
        si.install_cached(m, {e + ".qweight": q[None], e + ".scale": s[None], e + ".zero": s[None]}, "int2")
    # a packed 2D weight must map to a Linear
    with pytest.raises(si.CacheInstallError, match="not a Linear"):
        n = "model.layers.0.input_layernorm.weight"
        si.install_cached(m, {n + ".qweight": q, n + ".scale": s, n + ".zero": s}, "int4")
    # a 3D tensor needs a 3D parameter to replace, at a path the model has
    with pytest.raises(si.CacheInstallError, match="no 3D parameter"):
        e = "model.layers.0.mlp.gate_proj.weight"
        si.install_cached(m, {e + ".qweight": q[None], e + ".scale": s[None], e + ".zero": s[None]}, "int4")
    with pytest.raises(si.CacheInstallError, match="has no module"):
        e = "model.layers.0.mlp.experts.gate_up_proj"
        si.install_cached(m, {e + ".qweight": q[None], e + ".scale": s[None], e + ".zero": s[None]}, "int4")
    with pytest.raises(ValueError):
        si.install_cached(m, {}, "int3")
