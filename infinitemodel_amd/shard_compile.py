"""The ``_shards/<quant>/`` format: packers, packer tags, manifest verification, unit paths.

Keeps the reference's on-disk format and function names (shard_compile.py) so an existing cache
loads unchanged and a cache written here loads in the reference:

* int4: ``qweight u8 [out, in_pad/2]`` (low nibble = even column), ``scale``/``zero`` ``[out, ng]``
  in W's dtype, group 128 (shard_compile.py:74-94).
* int2: ``qweight u8 [out, in_pad/4]`` (crumb i = column 4j+i), group 64 (shard_compile.py:50-71).
* int8: ``qweight int8 [out, in]``, ``scale [out, 1]`` in W's dtype (shard_compile.py:170-178).
* 3D experts: per-expert stacks ``[E, out, ...]`` (shard_compile.py:97-140).

The packers are torch code mirroring the reference arithmetic op for op (same ops, same order,
same dtypes), so they are bit-identical to it on the same device; they run on whatever device W
lives on. The CPU oracle (oracle/quant.py) pins them in tests/test_packers.py.
"""
from __future__ import annotations

import hashlib
import json
import os
from typing import Optional

INT4_GROUP = 128
INT2_GROUP = 64
PACKER_VERSION = 1
INT2_PACKER_VERSION = 2


def _packer_tag(quant: str, group_size: int) -> str:
    """Manifest packer identity (shard_compile.py:36-39)."""
    if quant == "int2":
        return f"v{INT2_PACKER_VERSION}-g{group_size}-int2-gptq"
    return f"v{PACKER_VERSION}-g{group_size}-{quant}"


def _default_group(quant: str, group_size: int) -> int:
    """int2 packs at INT2_GROUP when handed the int4 default (shard_compile.py:42-47)."""
    if quant == "int2" and group_size == INT4_GROUP:
        return INT2_GROUP
    return group_size


def _rtn(W, G: int, qmax: int):
    import torch
    import torch.nn.functional as F
    out, in_f = W.shape
    ng = (in_f + G - 1) // G
    in_pad = ng * G
    Wp = F.pad(W, (0, in_pad - in_f)) if in_pad != in_f else W
    Wg = Wp.reshape(out, ng, G).float()
    wmin = Wg.amin(dim=2)
    wmax = Wg.amax(dim=2)
    scale = ((wmax - wmin) / float(qmax)).clamp(min=1e-8)
    zero = torch.round(-wmin / scale).clamp(0, qmax)
    q = torch.round(Wg / scale.unsqueeze(2) + zero.unsqueeze(2)).clamp(0, qmax).to(torch.uint8)
    return q.reshape(out, in_pad), scale, zero, in_f


def _device_packer(W, group_size: int):
    """libimq's device packer for a weight on a ROCm device (bit-identical to the host packers
    below; the torch expression stays the definition on other devices and group sizes)."""
    if getattr(W, "is_cuda", False) and W.dim() == 2 and group_size in (64, 128, 256):
        import torch
        if getattr(torch.version, "hip", None) and W.dtype in (torch.bfloat16, torch.float16, torch.float32):
            from . import ops
            return ops
    return None


def pack_linear_int4(W, group_size: int = INT4_GROUP):
    """Returns (qweight u8 [out, in_pad/2], scale, zero, in_features) (shard_compile.py:74-94)."""
    dev_ops = _device_packer(W, group_size)
    if dev_ops is not None:
        return dev_ops.pack_w4(W, group_size)
    q, scale, zero, in_f = _rtn(W, group_size, 15)
    qpacked = (q[:, 0::2] | (q[:, 1::2] << 4)).contiguous()
    return qpacked, scale.to(W.dtype), zero.to(W.dtype), in_f


def pack_linear_int2(W, group_size: int = INT2_GROUP):
    """Returns (qweight u8 [out, in_pad/4], scale, zero, in_features) (shard_compile.py:50-71)."""
    dev_ops = _device_packer(W, group_size)
    if dev_ops is not None:
        return dev_ops.pack_w2(W, group_size)
    q, scale, zero, in_f = _rtn(W, group_size, 3)
    qpacked = (q[:, 0::4] | (q[:, 1::4] << 2) | (q[:, 2::4] << 4) | (q[:, 3::4] << 6)).contiguous()
    return qpacked, scale.to(W.dtype), zero.to(W.dtype), in_f


def pack_linear_int4_3d(W3, group_size: int = INT4_GROUP, in_major: bool = False):
    """Per-expert int4 stack (shard_compile.py:97-140): each expert ``[out, in]`` (the transpose of
    ``W3[e]`` when ``in_major``) through pack_linear_int4 -- group quantization never crosses an
    expert -- stacked on a leading expert axis. Returns
    (qweight [E, out, in_pad/2], scale [E, out, ng], zero [E, out, ng], in_features, ng)."""
    import torch
    packs = [pack_linear_int4(W3[e].t().contiguous() if in_major else W3[e], group_size)
             for e in range(int(W3.shape[0]))]
    q, scale, zero = (torch.stack([p[i] for p in packs]) for i in range(3))
    return q, scale, zero, packs[0][3], int(scale.shape[2])


def pack_linear_int8(W):
    """Per-row symmetric int8 in W's own dtype (shard_compile.py:170-178): returns
    (qweight int8 [out, in], scale [out, 1])."""
    import torch
    dev_ops = _device_packer(W, 128)
    if dev_ops is not None:
        return dev_ops.pack_w8(W)
    scale = (W.abs().amax(dim=1, keepdim=True) / 127.0).clamp(min=1e-8)
    qW = (W / scale).round().clamp(-127, 127).to(torch.int8).contiguous()
    return qW, scale.to(W.dtype)


# ---------------------------------------------------------------------------------------------
# cache layout helpers (shard_compile.py:262-355 manifest fragments, 701-787 verify / unit path)
# ---------------------------------------------------------------------------------------------
def _shard_cache_root(model_dir: str) -> str:
    return os.path.join(model_dir, "_shards")


def _sha256_file(path: str) -> str:
    """Hex sha256 of a file, read through one reused 4 MiB buffer."""
    h = hashlib.sha256()
    buf = bytearray(4 << 20)
    view = memoryview(buf)
    with open(path, "rb", buffering=0) as f:
        while True:
            n = f.readinto(buf)
            if not n:
                break
            h.update(view[:n])
    return h.hexdigest()


_ROUTER_LEAF = frozenset({"gate", "router", "wg"})   # == worker_quant._ROUTER_LEAF_NAMES


def quant_scope(model) -> tuple:
    """(linear2d_names, expert3d_names): the exact weights a cold load quantizes, from the model
    skeleton (shard_compile.py:367-419 without the config loading): every nn.Linear ``.weight``
    inside a decoder layer except routers (a *Router / *Gate ancestor, or a leaf named gate /
    router / wg), and every fused 3D ``.experts.*.gate_up_proj`` / ``down_proj``. Names are the
    model's own parameter names."""
    from torch import nn
    by_name = dict(model.named_modules())

    def under_router(nm: str) -> bool:
        parts = nm.split(".")
        for i in range(1, len(parts)):
            anc = by_name.get(".".join(parts[:i]))
            if anc is not None and type(anc).__name__.endswith(("Router", "Gate")):
                return True
        return False

    lin2d, exp3d = set(), set()
    for name, mod in model.named_modules():
        if (isinstance(mod, nn.Linear) and ".layers." in name and not under_router(name)
                and name.rsplit(".", 1)[-1] not in _ROUTER_LEAF):
            lin2d.add(name + ".weight")
    for name, p in model.named_parameters():
        if p.dim() == 3 and ".experts." in name and (name.endswith(".gate_up_proj") or name.endswith(".down_proj")):
            exp3d.add(name)
    return lin2d, exp3d


def _in_major_expert_names(raw: dict) -> set:
    """Fused 3D expert tensors whose layout is in-major [E, in, out] (shard_compile.py:143-167):
    the ones with a per-expert ``<name>_bias`` beside them, the gpt-oss signature that survives
    checkpoint normalization. Packing such a tensor as [E, out, in] would write a cache that loads
    and verifies but serves the wrong axis."""
    return {n for n, W in raw.items() if W.dim() == 3 and (n + "_bias") in raw}


def _unit_tensor_kind(name: str, W, quant: str, lin2d, in_major: set) -> str:
    """How the cache stores one tensor of a unit: "experts" (fused 3D experts, int4 per-expert
    packs), "linear" (a packed 2D Linear weight: a decoder-layer Linear, or the lm_head at int8)
    or "plain" (written as is). Refuses what the serve side could not install correctly."""
    fused_expert = (W.dim() == 3 and ".experts." in name
                    and (name.endswith(".gate_up_proj") or name.endswith(".down_proj")))
    if fused_expert:
        if quant != "int4":
            raise ValueError(f"{name}: fused 3D MoE experts are only cacheable at int4 (got {quant})")
        if name in in_major:
            # the serve side cannot install transpose-packed gpt-oss experts from a cache, so
            # the compiler refuses instead of writing one (shard_compile.py:315-330)
            raise ValueError(f"{name}: in-major fused MoE experts (gpt-oss, [E, in, out]) are not "
                             "shard-cacheable; load gpt-oss at int4 without a shard cache, or at quant=none")
        return "experts"
    if W.dim() == 3 and ".experts." in name and quant != "int4":
        raise ValueError(f"{name}: fused 3D MoE experts cannot be packed at {quant}")
    if W.dim() == 2:
        in_layer = name in lin2d if lin2d is not None else (name.endswith(".weight") and ".layers." in name)
        if in_layer or (quant == "int8" and name == "lm_head.weight"):
            return "linear"
    return "plain"


def pack_unit_tensors(raw: dict, lin2d: Optional[set] = None, quant: str = "int4",
                      group_size: int = INT4_GROUP):
    """Pack one unit's tensors (logical 'model.*' names) into the cache dict + per-tensor manifest
    entries (shard_compile.py:262-355, for dense units and already-fused 3D experts). Decoder-layer
    Linears (those in ``lin2d``, or when None every 2D '.weight' under '.layers.') are packed at
    ``quant``, fused 3D experts per expert at int4, the lm_head at int8; the rest passes through."""
    if quant not in ("int4", "int8", "int2"):
        raise ValueError(f"shard pack supports quant int4|int8|int2 (got {quant!r})")
    group_size = _default_group(quant, group_size)
    in_major = _in_major_expert_names(raw) if quant == "int4" else set()
    packers = {"int4": pack_linear_int4, "int2": pack_linear_int2}
    out_sd: dict = {}
    meta: dict = {}
    for name, W in raw.items():
        kind = _unit_tensor_kind(name, W, quant, lin2d, in_major)
        shape = [int(d) for d in W.shape]
        if kind == "experts":
            q, s, z, in_f, ng = pack_linear_int4_3d(W, group_size)
            parts = {"qweight": q, "scale": s, "zero": z}
            info = {"q": True, "is_3d": True, "num_experts": shape[0], "out": shape[1], "in_features": in_f,
                    "ng": ng, "group_size": group_size}
        elif kind == "linear" and quant == "int8":
            q, s = pack_linear_int8(W)
            parts = {"qweight": q, "scale": s}
            info = {"q": True}
        elif kind == "linear":
            q, s, z, in_f = packers[quant](W, group_size)
            parts = {"qweight": q, "scale": s, "zero": z}
            info = {"q": True, "in_features": in_f}
        else:
            out_sd[name] = W.contiguous()
            meta[name] = {"q": False, "shape": shape}
            continue
        for leaf, t in parts.items():
            out_sd[f"{name}.{leaf}"] = t
        meta[name] = {**info, "shape": shape}
    return out_sd, meta


def write_cache(model_dir: str, units: dict, quant: str, group_size: int, num_layers: int,
                tied: bool = False, lin2d: Optional[set] = None) -> dict:
    """Write ``_shards/<quant>/`` from in-memory units {filename: {name: tensor}} (embed / L%04d /
    head) with the reference manifest schema (shard_compile.py:593-598, 664-674, 696-697)."""
    from safetensors.torch import save_file
    group_size = _default_group(quant, group_size)
    out_dir = os.path.join(_shard_cache_root(model_dir), quant)
    os.makedirs(out_dir, exist_ok=True)
    manifest = {"format": 1, "quant": quant, "group_size": group_size, "num_layers": num_layers,
                "tied": tied, "files": {}, "tensors": {}, "packer_hash": _packer_tag(quant, group_size),
                "expert_layout": None}
    for unit, raw in units.items():
        sd, mt = pack_unit_tensors(raw, lin2d, quant, group_size)
        for name, meta in mt.items():
            manifest["tensors"][name] = {"file": unit, **meta}
            if meta.get("is_3d"):
                manifest["expert_layout"] = "fused3d"
        path = os.path.join(out_dir, unit)
        save_file({k: v.detach().cpu().contiguous() for k, v in sd.items()}, path)
        manifest["files"][unit] = {"sha256": _sha256_file(path), "bytes": os.path.getsize(path)}
    with open(os.path.join(out_dir, "manifest.json"), "w", encoding="utf-8") as f:
        json.dump(manifest, f)
    return manifest


def _read_manifest(d: str):
    """(manifest dict, None) or (None, problem) for the cache directory ``d``."""
    path = os.path.join(d, "manifest.json")
    if not os.path.isfile(path):
        return None, "no manifest.json"
    try:
        with open(path, encoding="utf-8") as f:
            return json.load(f), None
    except Exception as exc:
        return None, f"manifest.json cannot be read ({exc})"


def _unit_file_problem(d: str, fname: str, entry: dict):
    """The first way cached unit ``fname`` disagrees with its manifest entry, or None."""
    path = os.path.join(d, fname)
    if not os.path.isfile(path):
        return f"{fname}: listed in the manifest but absent"
    size = os.path.getsize(path)
    if size != entry.get("bytes"):
        return f"{fname}: {size} bytes on disk, {entry.get('bytes')} in the manifest"
    if _sha256_file(path) != entry.get("sha256"):
        return f"{fname}: sha256 differs from the manifest (corrupt unit)"
    return None


def verify_shard_cache(model_dir: str, quant: str) -> tuple:
    """(ok, problems) of ``_shards/<quant>/`` (shard_compile.py:701-736): a readable manifest, each
    listed unit present with the manifest's size and sha256, one unit per layer plus embed and
    head, and -- when the manifest records one (older caches do not) -- this packer's tag."""
    d = os.path.join(_shard_cache_root(model_dir), quant)
    man, err = _read_manifest(d)
    if err is not None:
        return False, [err]
    units = man.get("files", {})
    problems = [p for p in (_unit_file_problem(d, f, e) for f, e in units.items()) if p is not None]
    layers = int(man.get("num_layers", 0))
    if len(units) != layers + 2:
        problems.append(f"manifest lists {len(units)} units; {layers} layers need {layers + 2} "
                        "(embed, layers, head) -- incomplete cache")
    tag = man.get("packer_hash")
    if tag is not None:
        want = _packer_tag(man.get("quant", quant), int(man.get("group_size", INT4_GROUP)))
        if tag != want:
            problems.append(f"packer tag {tag!r} is not this packer's {want!r}: recompile the cache")
    return not problems, problems


def _unit_file_name(start: int, end: int, embed: bool, head: bool):
    """File name of a cached unit: the embedding, the head, or one decoder layer L%04d; None for
    a span of several layers (the cache stores layers one per file)."""
    if embed:
        return "embed.safetensors"
    if head:
        return "head.safetensors"
    return f"L{start:04d}.safetensors" if end == start + 1 else None


def cache_unit_path(model_dir: str, quant: str, start: int, end: int, embed: bool, head: bool):
    """Path of one cached unit when it exists, else None (shard_compile.py:768-787)."""
    name = _unit_file_name(start, end, embed, head)
    if name is None:
        return None
    path = os.path.join(_shard_cache_root(model_dir), quant, name)
    return path if os.path.isfile(path) else None
