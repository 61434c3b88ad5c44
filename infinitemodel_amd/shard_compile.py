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
    """Per-expert int4 stack (shard_compile.py:97-140): returns
    (qweight [E, out, in_pad/2], scale [E, out, ng], zero [E, out, ng], in_features, ng)."""
    import torch

    def _expert(i):
        return W3[i].t().contiguous() if in_major else W3[i]

    E = int(W3.shape[0])
    q0, s0, z0, in_f = pack_linear_int4(_expert(0), group_size)
    qpacked = torch.empty((E,) + tuple(q0.shape), dtype=q0.dtype, device=q0.device)
    scale = torch.empty((E,) + tuple(s0.shape), dtype=s0.dtype, device=s0.device)
    zero = torch.empty((E,) + tuple(z0.shape), dtype=z0.dtype, device=z0.device)
    qpacked[0], scale[0], zero[0] = q0, s0, z0
    for e in range(1, E):
        qe, se, ze, _ = pack_linear_int4(_expert(e), group_size)
        qpacked[e], scale[e], zero[e] = qe, se, ze
    return qpacked, scale, zero, in_f, int(scale.shape[2])


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
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
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


def pack_unit_tensors(raw: dict, lin2d: Optional[set] = None, quant: str = "int4",
                      group_size: int = INT4_GROUP):
    """Pack one unit's tensors (logical 'model.*' names) into the cache dict + manifest fragments,
    for dense units and already-fused 3D experts (shard_compile.py:262-355, without the meta-
    skeleton MoE fuse). 2D layer Linears in ``lin2d`` (or, when None, every 2D '.weight' under
    '.layers.') are packed; 3D '.experts.*.gate_up_proj/down_proj' are int4-packed per expert;
    int8 also packs 'lm_head.weight'; everything else passes through."""
    if quant not in ("int4", "int8", "int2"):
        raise ValueError(f"shard pack supports quant int4|int8|int2 (got {quant!r})")
    group_size = _default_group(quant, group_size)
    in_major = _in_major_expert_names(raw) if quant == "int4" else set()
    out_sd: dict = {}
    mt: dict = {}
    for name, W in raw.items():
        is_expert3d = (quant == "int4" and W.dim() == 3 and ".experts." in name
                       and (name.endswith(".gate_up_proj") or name.endswith(".down_proj")))
        if is_expert3d and name in in_major:
            # shard_compile.py:315-330: the serve side cannot install transpose-packed gpt-oss
            # experts from a cache, so the compile refuses rather than writing one
            raise ValueError(f"{name}: in-major fused MoE experts (gpt-oss, [E, in, out]) are not "
                             "shard-cacheable; load gpt-oss at int4 without a shard cache, or at "
                             "quant=none")
        if lin2d is not None:
            is_lin = W.dim() == 2 and name in lin2d
        else:
            is_lin = W.dim() == 2 and name.endswith(".weight") and ".layers." in name
        is_int8_head = quant == "int8" and name == "lm_head.weight" and W.dim() == 2
        if W.dim() == 3 and quant != "int4" and ".experts." in name:
            raise ValueError(f"fused 3D MoE experts cannot be packed at {quant}")
        if is_expert3d:
            qw, sc, ze, in_f, ng = pack_linear_int4_3d(W, group_size)
            out_sd[name + ".qweight"], out_sd[name + ".scale"], out_sd[name + ".zero"] = qw, sc, ze
            mt[name] = {"q": True, "is_3d": True, "num_experts": int(W.shape[0]), "out": int(W.shape[1]),
                        "in_features": in_f, "ng": ng, "group_size": group_size,
                        "shape": [int(x) for x in W.shape]}
        elif is_lin or is_int8_head:
            if quant in ("int4", "int2"):
                pk = pack_linear_int4 if quant == "int4" else pack_linear_int2
                qw, sc, ze, in_f = pk(W, group_size)
                out_sd[name + ".qweight"], out_sd[name + ".scale"], out_sd[name + ".zero"] = qw, sc, ze
                mt[name] = {"q": True, "in_features": in_f, "shape": [int(x) for x in W.shape]}
            else:
                qw, sc = pack_linear_int8(W)
                out_sd[name + ".qweight"], out_sd[name + ".scale"] = qw, sc
                mt[name] = {"q": True, "shape": [int(x) for x in W.shape]}
        else:
            out_sd[name] = W.contiguous()
            mt[name] = {"q": False, "shape": [int(x) for x in W.shape]}
    return out_sd, mt


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


def verify_shard_cache(model_dir: str, quant: str) -> tuple:
    """(ok, problems) -- manifest present, every file's size and sha256, file count, packer_hash
    (shard_compile.py:701-736; a missing packer_hash is accepted as legacy)."""
    d = os.path.join(_shard_cache_root(model_dir), quant)
    mf = os.path.join(d, "manifest.json")
    if not os.path.isfile(mf):
        return False, ["manifest.json missing"]
    try:
        with open(mf, encoding="utf-8") as fh:
            man = json.load(fh)
    except Exception as exc:
        return False, [f"manifest.json unreadable: {exc}"]
    problems = []
    files = man.get("files", {})
    for fname, meta in files.items():
        p = os.path.join(d, fname)
        if not os.path.isfile(p):
            problems.append(f"missing file {fname}")
            continue
        if os.path.getsize(p) != meta.get("bytes"):
            problems.append(f"size mismatch {fname}")
            continue
        if _sha256_file(p) != meta.get("sha256"):
            problems.append(f"sha256 mismatch {fname} (corrupt)")
    exp = int(man.get("num_layers", 0)) + 2
    if len(files) != exp:
        problems.append(f"incomplete: {len(files)} files, expected {exp}")
    ph = man.get("packer_hash")
    if ph is not None:
        want = _packer_tag(man.get("quant", quant), int(man.get("group_size", INT4_GROUP)))
        if ph != want:
            problems.append(f"packer_hash mismatch ({ph} != {want}) — recompile")
    return (len(problems) == 0), problems


def cache_unit_path(model_dir: str, quant: str, start: int, end: int, embed: bool, head: bool):
    """Path of one cached unit or None (shard_compile.py:768-787)."""
    d = os.path.join(_shard_cache_root(model_dir), quant)
    if embed:
        name = "embed.safetensors"
    elif head:
        name = "head.safetensors"
    elif end - start == 1:
        name = f"L{start:04d}.safetensors"
    else:
        return None
    p = os.path.join(d, name)
    return p if os.path.isfile(p) else None
