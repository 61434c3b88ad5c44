"""Serve-from-cache install of one pre-packed ``_shards/<quant>/`` unit into a model.

Restates the reference's ``_install_cached`` (shard_build.py:934-1030) and its fused-MoE sweep
(shard_build.py:1256-1265): a unit's safetensors dict, already packed at ``quant`` by the cache
compiler (``shard_compile.pack_unit_tensors``, bit-identical to the load-time packers), becomes
the resident quantized holders directly, with no bf16 detour and no re-quantization:

* ``<lin>.weight.{qweight,scale[,zero]}`` (2D) -> QuantLinear4 / QuantLinear2 / QuantLinear (int8)
  in place of the model's Linear at ``<lin>``, keeping its ``in_features`` (the cache stores
  padded widths only) and its bias from the unit's ``<lin>.bias``;
* ``<experts>.{gate_up,down}_proj.{qweight,scale,zero}`` (3D, int4 only) -> Packed4Tensor3D in
  place of the 3D Parameter, with the eager experts implementation forced on its config;
* every other tensor is passed through (cast to ``dtype``) with ``load_state_dict(assign=True)``.

Refusals are the reference's, because each guards against a load that would succeed and serve
wrong weights: an incomplete packed triple, a zero point in an int8 cache (the int8 pack is
symmetric and never writes one), a 3D expert tensor in an int2/int8 cache, a packed 2D weight
whose module is not a Linear, a 3D tensor without a matching 3D parameter.
"""
from __future__ import annotations

from . import worker_quant as wq


class CacheInstallError(RuntimeError):
    """A cached unit does not match the model or the quant tier it is installed at."""


def _nav(model, path: str):
    parent = model
    if not path:
        return parent
    try:
        for p in path.split("."):
            parent = parent[int(p)] if p.isdigit() else getattr(parent, p)
    except (AttributeError, IndexError, TypeError) as exc:
        raise CacheInstallError(f"cache: the model has no module {path!r} ({exc})") from exc
    return parent


def install_cached(model, sd: dict, quant: str, dtype=None, head=None) -> dict:
    """Install one cached unit ``sd`` ({name: tensor}) into ``model`` at ``quant`` (int4 | int2 |
    int8), as shard_build.py:934-1030 does. ``dtype`` is the passthrough dtype (default bf16);
    ``head`` is the model's current lm_head module, returned replaced when an int8 cache packs it.
    Returns ``{"loaded_params": n, "head": head, "quantized": [module paths]}``."""
    import torch

    if quant not in ("int4", "int2", "int8"):
        raise ValueError(f"cache install supports quant int4|int2|int8 (got {quant!r})")
    dt = dtype if dtype is not None else torch.bfloat16
    QL = (wq._quant_linear_cls() if quant == "int8" else
          wq._quant2_linear_cls() if quant == "int2" else wq._quant4_linear_cls())
    PT = wq._packed4_3d_cls()
    G = wq._INT2_GROUP if quant == "int2" else wq._INT4_GROUP
    need_zero = quant != "int8"

    packed: dict = {}
    plain: dict = {}
    for k, v in sd.items():
        if k.endswith(".qweight"):
            packed.setdefault(k[:-8], {})["q"] = v
        elif k.endswith(".scale"):
            packed.setdefault(k[:-6], {})["s"] = v
        elif k.endswith(".zero"):
            packed.setdefault(k[:-5], {})["z"] = v
        else:
            plain[k] = v if v.dtype == dt else v.to(dt)

    loaded = 0
    done = []
    eager_cfgs: set = set()
    for base, tr in packed.items():
        qw, sc, ze = tr.get("q"), tr.get("s"), tr.get("z")
        if qw is None or sc is None or (need_zero and ze is None):
            raise CacheInstallError(f"cache: incomplete packed tensor {base!r} (have {sorted(tr)})")
        if not need_zero and ze is not None:
            raise CacheInstallError(f"cache: packed tensor {base!r} carries a zero point in an int8 "
                                    "cache; the int8 pack is symmetric (w = q*scale) and never "
                                    "writes one, so this unit was packed by something else")
        if qw.dim() == 3:
            if quant != "int4":
                raise CacheInstallError(f"cache: 3D expert tensor {base!r} in a {quant} cache; only "
                                        "int4 has a 3D-expert format")
            ppath, _, attr = base.rpartition(".")
            parent = _nav(model, ppath)
            metap = parent._parameters.get(attr)
            if metap is None or metap.dim() != 3:
                raise CacheInstallError(f"cache: no 3D parameter for expert tensor {base!r}")
            in_f = int(metap.shape[2])
            delattr(parent, attr)
            setattr(parent, attr, PT(qw, sc, ze, in_f, G))
            loaded += int(qw.shape[0]) * int(qw.shape[1]) * in_f
            cfg = getattr(parent, "config", None)
            if cfg is not None and hasattr(cfg, "_experts_implementation") and id(cfg) not in eager_cfgs:
                cfg._experts_implementation = "eager"
                eager_cfgs.add(id(cfg))
            done.append(base)
        else:
            mod_path = base[:-7] if base.endswith(".weight") else base
            ppath, _, attr = mod_path.rpartition(".")
            parent = _nav(model, ppath)
            lin = getattr(parent, attr)
            if not hasattr(lin, "in_features"):
                raise CacheInstallError(f"cache: {mod_path!r} is {type(lin).__name__}, not a Linear; "
                                        "cache / model layout mismatch")
            in_f = int(lin.in_features)
            bp = plain.pop(mod_path + ".bias", None)
            bias = torch.nn.Parameter(bp, requires_grad=False) if bp is not None else None
            if quant == "int8":
                mod = QL(qw, sc, bias)                   # unpadded [out, in], per-row scale, no zero
            else:
                mod = QL(qw, sc, ze, bias, in_f, G)
            setattr(parent, attr, mod)
            if head is not None and lin is head:
                head = mod                               # int8 packs lm_head and replaces the module
            loaded += int(qw.shape[0]) * in_f
            done.append(mod_path)
    if plain:
        model.load_state_dict(plain, strict=False, assign=True)
        loaded += sum(int(t.numel()) for t in plain.values())
    return {"loaded_params": loaded, "head": head, "quantized": done}


def install_fused_moe_sweep(model) -> int:
    """Patch the fused experts forward onto every fused-3D int4 experts module, however it was
    built (shard_build.py:1256-1265); idempotent. Returns the number of experts modules patched."""
    n = 0
    for m in model.modules():
        before = getattr(m, "_fused_moe_installed", False)
        wq._install_fused_moe_forward(m)
        n += int(getattr(m, "_fused_moe_installed", False) and not before)
    return n
