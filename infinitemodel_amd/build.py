"""Build libimq.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

Usage: ``python -m infinitemodel_amd.build`` (or ``__graft_entry__.build()``). Each ``csrc/*.hip``
is compiled to an object in parallel, then linked into ``infinitemodel_amd/_lib/libimq.so``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_lib")
OBJ_DIR = os.path.join(HERE, "_lib", "obj")
LIB = os.path.join(OUT_DIR, "libimq.so")
ARCH = os.environ.get("IMQ_OFFLOAD_ARCH", "gfx950")

# Packed-fp32 VALU ops are disabled for all device code (hipcc flag; the host pass ignores it).
COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libimq.so)")


# Per-source extra flags. moe_rb.hip: MFMA results in VGPRs (LLVM's VGPR form of the MFMA
# instructions), so the folded MoE kernels' per-group fold reads them without AGPR copies and two
# waves fit per SIMD; the option is scoped to that file's kernels.
EXTRA = {"moe_rb.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src).replace(".hip", ".o"))
    cmd = [hipcc(), *COMMON, *EXTRA.get(os.path.basename(src), []), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), *COMMON, "-shared", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"[imq] built {LIB} ({len(srcs)} sources, {ARCH})", flush=True)
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
