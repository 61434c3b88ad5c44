"""Serve-from-cache install of one pre-packed ``_shards/<quant>/`` unit into a model.

The cache compiler (``shard_compile.pack_unit_tensors``) writes every quantized weight already
packed, bit-identical to the load-time packers, so serving from the cache needs no bf16 detour and
no re-quantization (the reference's ``_install_cached``, shard_build.py:934-1030, and its fused-MoE
sweep, 1256-1265). A unit's tensors fall into three kinds:

* a packed Linear ``<lin>.weight.{qweight, scale[, zero]}`` (2D) -> QuantLinear4 / QuantLinear2 /
  QuantLinear (int8) in place of the model's Linear, keeping its ``in_features`` (the cache stores
  padded widths only) and taking its bias from the unit's ``<lin>.bias``;
* packed fused experts ``<block>.{gate_up,down}_proj.{qweight, scale, zero}`` (3D, int4 only) ->
  Packed4Tensor3D in place of the 3D Parameter, with the eager experts implementation forced on
  the block's config;
* anything else -> passed through (cast to ``dtype``) by ``load_state_dict(assign=True)``.

Each refusal guards a load that would otherwise succeed and serve wrong weights: an incomplete
packed set, a zero point in an int8 cache (the int8 pack is symmetric and never writes one), a 3D
expert tensor in an int2 / int8 cache, a packed 2D weight whose module is not a Linear, a 3D tensor
without a matching 3D parameter.
"""
from __future__ import annotations

from dataclasses import dataclass, field

from . import worker_quant as wq

_PART_OF = {"qweight": "q", "scale": "s", "zero": "z"}


class CacheInstallError(RuntimeError):
    """A cached unit does not match the model or the quant tier it is installed at."""


@dataclass
class _Packed:
    """The packed parts of one weight (``q``, ``s`` and, except int8, ``z``) under ``base``."""
    base: str
    parts: dict = field(default_factory=dict)

    def tensors(self):
        return self.parts.get("q"), self.parts.get("s"), self.parts.get("z")


def _split_unit(sd: dict, dt):
    """({base: _Packed}, {name: passthrough tensor cast to dt}) of a unit's state dict."""
    packed: dict = {}
    plain: dict = {}
    for name, t in sd.items():
        base, _, leaf = name.rpartition(".")
        role = _PART_OF.get(leaf)
        if role is not None and base:
            packed.setdefault(base, _Packed(base)).parts[role] = t
        else:
            plain[name] = t if t.dtype == dt else t.to(dt)
    return packed, plain


def _check_parts(p: _Packed, quant: str) -> None:
    q, s, z = p.tensors()
    symmetric = quant == "int8"
    if q is None or s is None or (z is None and not symmetric):
        raise CacheInstallError(f"cache: packed weight {p.base!r} is incomplete (found {sorted(p.parts)})")
    if symmetric and z is not None:
        raise CacheInstallError(f"cache: packed weight {p.base!r} has a zero point, but an int8 cache is "
                                "symmetric (w = q * scale) -- the unit was not written by this packer")
    if q.dim() == 3 and quant != "int4":
        raise CacheInstallError(f"cache: fused 3D experts {p.base!r} in a {quant} cache; only int4 packs "
                                "3D experts")


def _module_at(model, path: str):
    node = model
    for part in filter(None, path.split(".")):
        try:
            node = node[int(part)] if part.isdigit() else getattr(node, part)
        except (AttributeError, IndexError, TypeError) as exc:
            raise CacheInstallError(f"cache: the model has no module {path!r} ({exc})") from exc
    return node


class _Installer:
    def __init__(self, model, quant: str, plain: dict, head):
        import torch
        self.torch = torch
        self.model, self.quant, self.plain, self.head = model, quant, plain, head
        self.group = wq._INT2_GROUP if quant == "int2" else wq._INT4_GROUP
        self.linear_cls = {"int4": wq._quant4_linear_cls, "int2": wq._quant2_linear_cls,
                           "int8": wq._quant_linear_cls}[quant]()
        self.loaded = 0
        self.paths: list = []
        self._eager_configs: set = set()

    def experts(self, p: _Packed) -> None:
        q, s, z = p.tensors()
        parent_path, _, attr = p.base.rpartition(".")
        block = _module_at(self.model, parent_path)
        slot = block._parameters.get(attr)
        if slot is None or slot.dim() != 3:
            raise CacheInstallError(f"cache: {p.base!r} is packed 3D experts but the model has no 3D "
                                    "parameter there")
        in_features = int(slot.shape[2])
        delattr(block, attr)
        setattr(block, attr, wq._packed4_3d_cls()(q, s, z, in_features, self.group))
        cfg = getattr(block, "config", None)
        if cfg is not None and hasattr(cfg, "_experts_implementation") and id(cfg) not in self._eager_configs:
            cfg._experts_implementation = "eager"
            self._eager_configs.add(id(cfg))
        self.loaded += int(q.shape[0]) * int(q.shape[1]) * in_features
        self.paths.append(p.base)

    def linear(self, p: _Packed) -> None:
        q, s, z = p.tensors()
        path = p.base[:-len(".weight")] if p.base.endswith(".weight") else p.base
        parent_path, _, attr = path.rpartition(".")
        parent = _module_at(self.model, parent_path)
        old = getattr(parent, attr)
        if not hasattr(old, "in_features"):
            raise CacheInstallError(f"cache: {path!r} holds a packed 2D weight but the model has a "
                                    f"{type(old).__name__} there, not a Linear")
        in_features = int(old.in_features)
        bias_t = self.plain.pop(path + ".bias", None)
        bias = None if bias_t is None else self.torch.nn.Parameter(bias_t, requires_grad=False)
        if self.quant == "int8":
            new = self.linear_cls(q, s, bias)            # [out, in] int8, per-row scale
        else:
            new = self.linear_cls(q, s, z, bias, in_features, self.group)
        setattr(parent, attr, new)
        if self.head is not None and old is self.head:
            self.head = new                              # an int8 cache packs the lm_head too
        self.loaded += int(q.shape[0]) * in_features
        self.paths.append(path)


def install_cached(model, sd: dict, quant: str, dtype=None, head=None) -> dict:
    """Install one cached unit ``sd`` ({name: tensor}) into ``model`` at ``quant`` (int4 | int2 |
    int8), as shard_build.py:934-1030 does. ``dtype`` is the passthrough dtype (default bf16);
    ``head`` is the model's current lm_head module, returned replaced when an int8 cache packs it.
    Returns ``{"loaded_params": n, "head": head, "quantized": [module paths]}``."""
    import torch
    if quant not in ("int4", "int2", "int8"):
        raise ValueError(f"cache install supports quant int4|int2|int8 (got {quant!r})")
    packed, plain = _split_unit(sd, dtype if dtype is not None else torch.bfloat16)
    for p in packed.values():
        _check_parts(p, quant)
    inst = _Installer(model, quant, plain, head)
    for p in packed.values():
        (inst.experts if p.tensors()[0].dim() == 3 else inst.linear)(p)
    if inst.plain:
        model.load_state_dict(inst.plain, strict=False, assign=True)
        inst.loaded += sum(int(t.numel()) for t in inst.plain.values())
    return {"loaded_params": inst.loaded, "head": inst.head, "quantized": inst.paths}


def install_fused_moe_sweep(model) -> int:
    """Put the fused experts forward on every fused-3D int4 experts module, however it was built
    (shard_build.py:1256-1265); idempotent. Returns the number of modules newly patched."""
    patched = 0
    for m in model.modules():
        had = bool(getattr(m, "_fused_moe_installed", False))
        wq._install_fused_moe_forward(m)
        patched += int(not had and bool(getattr(m, "_fused_moe_installed", False)))
    return patched
