"""The C ABI without a GPU: libimq.so loads, exports exactly what include/imq.h declares with the
ctypes signatures the Python layer binds, and rejects invalid arguments before touching a device."""
import ctypes
import os
import re

import pytest

from infinitemodel_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "imq.h")


def _declared():
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    txt = re.sub(r"//[^\n]*", "", txt)
    return sorted(set(re.findall(r"\b(imq_[a-z0-9_]+)\s*\(", txt)))


@pytest.fixture(scope="module")
def L():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} is not built (python -m infinitemodel_amd.build)")
    return _lib.lib()


def test_header_and_bindings_agree():
    assert _declared() == sorted(_lib.SIGNATURES)


def _prototypes():
    """name -> (return type, [parameter types]) of every declaration in the header."""
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    txt = re.sub(r"//[^\n]*", "", txt)
    out = {}
    for m in re.finditer(r"([A-Za-z_][A-Za-z0-9_ \*]*?)\b(imq_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", txt):
        ret, name, params = m.group(1).strip(), m.group(2), m.group(3).strip()
        types = []
        if params and params != "void":
            for p in params.split(","):
                p = " ".join(p.split())
                types.append(re.sub(r"\s*\b[a-zA-Z_][a-zA-Z0-9_]*$", "", p) if not p.endswith("*") else p)
        out[name] = (ret, types)
    return out


def _ctype(c: str):
    c = c.replace("const ", "").strip()
    if c.endswith("*"):
        return ctypes.c_char_p if c == "char*" or c == "char *" else ctypes.c_void_p
    return {"int64_t": ctypes.c_int64, "int": ctypes.c_int, "float": ctypes.c_float, "double": ctypes.c_double,
            "void": None}[c]


def test_bindings_match_header_prototypes():
    """Every SIGNATURES entry has the header's return type and parameter types, in order."""
    protos = _prototypes()
    assert sorted(protos) == sorted(_lib.SIGNATURES)
    for name, (ret, params) in protos.items():
        rt, at = _lib.SIGNATURES[name]
        assert _ctype(ret) == rt, (name, ret)
        assert [_ctype(p) for p in params] == list(at), name


def test_library_exports_every_declared_symbol(L):
    missing = [n for n in _declared() if not hasattr(L, n)]
    assert not missing, missing


def test_exports_are_c_linkage():
    """Every declared name is an unmangled dynamic symbol (nm -D), so any FFI can bind it."""
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    syms = {line.split()[-1] for line in out.splitlines() if line.strip()}
    for n in _declared():
        assert n in syms, n


def test_abi_version_and_strerror(L):
    assert L.imq_abi_version() == 8
    assert L.imq_strerror(0) == b"ok"
    for rc in (_lib.IMQ_ERR_INVALID, _lib.IMQ_ERR_UNSUPPORTED, _lib.IMQ_ERR_ALIGN, _lib.IMQ_ERR_SCRATCH):
        assert len(L.imq_strerror(rc)) > 5


def test_moe_workspace_bytes(L):
    # gu fp32 [B, 2I] + h bf16 [B, I_pad] + z fp32 [B, H], each 256-aligned
    T, k, E, H, I, G = 3, 8, 64, 2048, 1024, 128
    B = T * k
    al = lambda v: -(-v // 256) * 256  # noqa: E731
    assert L.imq_moe_workspace_bytes(T, k, E, H, I, G) >= al(B * 2 * I * 4) + al(B * I * 2) + al(B * H * 4)
    assert L.imq_moe_workspace_bytes(-1, k, E, H, I, G) < 0


def test_linear_workspace_bytes_host_rules(L):
    """Decode rows M <= 2 split K only where the int2 line kernel declines a line-tiled weight (K
    beyond its 16 waves), M 3..4 only on line-tiled int2 weights (1024-code chunks); 4 < M <= 16 split K into 1024-code chunks (512-code chunks for grids
    of at most two 4-tile workgroups per CU, at the host's default 256 CUs) with fp32 partials
    [splits][M][N]; negative sizes are rejected."""
    assert L.imq_linear_workspace_bytes(1, 4096, 4096) == 0
    assert L.imq_linear_workspace_bytes(2, 4096, 14336) == 0
    assert L.imq_linear_workspace_bytes(4, 4096, 14336) == 14 * 4 * 4096 * 4
    assert L.imq_linear_workspace_bytes(3, 4096, 14592) == 0      # K_pad % 512: no int2 K-split
    assert L.imq_linear_workspace_bytes(2, 8192, 28672) == 28 * 2 * 8192 * 4   # int2 line kernel declines
    assert L.imq_linear_workspace_bytes(1, 256, 16640) > 0        # int4 line kernel declines (65 line-steps)
    assert L.imq_linear_workspace_bytes(16, 4096, 14336) == 14 * 16 * 4096 * 4
    assert L.imq_linear_workspace_bytes(5, 6144, 4096) == 8 * 5 * 6144 * 4    # short grid: 512-code splits
    assert L.imq_linear_workspace_bytes(8, 96, 384) == 0          # K_pad % 256: skinny kernel
    assert L.imq_linear_workspace_bytes(-1, 4096, 4096) < 0


def _w4_need(L, M, K, N, G=128, sdt=0):
    return L.imq_linear_w4_workspace_bytes(M, K, N, G, K // 2, K, K // G, 1, sdt, K // G, 1, sdt)


def test_linear_w4_workspace_bytes_host_rules(L):
    """The per-call query follows the dispatcher's plans: decode rows M <= 4 take the line kernel
    (no partials); 4 < M <= 16 at K_pad 14336 take the K-split kernel ([splits][M][N] fp32,
    1024-code splits); a skinny-only shape and invalid sizes. (Which K_pad 2048 / 4096 shapes the
    wave-split kernel takes depends on the device's LDS, so the GPU tests cover them.)"""
    assert _w4_need(L, 1, 4096, 4096) == 0
    assert _w4_need(L, 4, 14336, 4096) == 0
    assert _w4_need(L, 16, 14336, 4096) == 14 * 16 * 4096 * 4
    assert _w4_need(L, 8, 14336, 4096) == 14 * 8 * 4096 * 4
    assert _w4_need(L, 8, 384, 96) == 0          # K_pad % 256: skinny kernel
    assert _w4_need(L, 0, 4096, 4096) == 0
    assert _w4_need(L, -1, 4096, 4096) < 0
    assert L.imq_linear_w4_workspace_bytes(1, 4000, 4096, 128, 2000, 4000, 32, 1, 0, 32, 1, 0) < 0
    # never above the shape-only bound
    for M, K, N in ((16, 14336, 4096), (5, 4096, 6144), (16, 4096, 28672), (512, 14336, 4096)):
        assert 0 <= _w4_need(L, M, K, N) <= L.imq_linear_workspace_bytes(M, N, K)


def test_invalid_arguments_are_rejected_on_the_host(L):
    """Null pointers and inconsistent shapes return IMQ_ERR_INVALID without a device call."""
    nul = None
    rc = L.imq_linear_w4(nul, 4096, 1, 4096, nul, 2048, nul, 32, 1, 0, nul, 32, 1, 0, 4096, 128, nul, 4096, nul, 0,
                         nul)
    assert rc == _lib.IMQ_ERR_INVALID
    one = ctypes.c_void_p(16)   # never dereferenced: validation fails first
    # K_pad not a multiple of the group
    rc = L.imq_linear_w4(one, 4096, 1, 4000, one, 2048, one, 32, 1, 0, one, 32, 1, 0, 4096, 128, one, 4096, nul, 0,
                         nul)
    assert rc == _lib.IMQ_ERR_INVALID
    # packed row stride shorter than the packed row
    rc = L.imq_linear_w2(one, 4096, 1, 4096, one, 512, one, 64, 1, 0, one, 64, 1, 0, 4096, 64, one, 4096, nul, 0, nul)
    assert rc == _lib.IMQ_ERR_INVALID
    # bad dtype code
    rc = L.imq_linear_w8(one, 4096, 1, 4096, one, 4096, one, 1, 7, 4096, one, 4096, nul, 0, nul)
    assert rc == _lib.IMQ_ERR_INVALID
    rc = L.imq_dequant_w4(one, 2048, one, 32, 1, 0, one, 32, 1, 0, 4096, 4096, 100, one, 4096, 0, nul)
    assert rc == _lib.IMQ_ERR_INVALID


def test_noalloc_rejects_on_the_host(L):
    """imq_linear_w4_noalloc validates like imq_linear_w4 and refuses, before any device call,
    calls whose own workspace need exceeds its static scratch (IMQ_ERR_SCRATCH)."""
    nul = None
    rc = L.imq_linear_w4_noalloc(nul, 4096, 1, 4096, nul, 2048, nul, 32, 1, 0, nul, 32, 1, 0, 4096, 128, nul,
                                 4096, nul)
    assert rc == _lib.IMQ_ERR_INVALID
    one = ctypes.c_void_p(16)   # never dereferenced: the size check fails first
    M, N, K = 16, 1 << 20, 14336     # K-split: 14 splits x 16 x 2^20 x 4 B of partials
    need = _w4_need(L, M, K, N)
    assert need == 14 * 16 * N * 4 > _lib.IMQ_NOALLOC_SCRATCH_BYTES
    rc = L.imq_linear_w4_noalloc(one, K, M, K, one, K // 2, one, K // 128, 1, 0, one, K // 128, 1, 0, N, 128, one,
                                 N, nul)
    assert rc == _lib.IMQ_ERR_SCRATCH
    assert b"scratch" in L.imq_strerror(rc)
