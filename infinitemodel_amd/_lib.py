"""ctypes binding of libimq.so (the gfx950 kernels' C ABI, declared in include/imq.h).

torch is imported before the library is loaded so that libimq's ``libamdhip64.so.7``
dependency resolves to the HIP runtime torch already loaded (same SONAME): device pointers and
``hipStream_t`` handles from torch are then valid in every libimq call.

There is no fallback here: if the library is missing or fails to load, ``lib()`` raises
``ImqUnavailable``. The reference-compatible modules above this layer turn that into their
documented "naive path" behaviour (worker_quant.py prepare_fused never raises); the ops in
``infinitemodel_amd.ops`` raise.
"""
from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("IMQ_LIB_PATH") or os.path.join(HERE, "_lib", "libimq.so")

IMQ_DT_BF16, IMQ_DT_FP16, IMQ_DT_FP32, IMQ_DT_I32, IMQ_DT_I64 = 0, 1, 2, 3, 4
IMQ_OK, IMQ_ERR_INVALID, IMQ_ERR_UNSUPPORTED, IMQ_ERR_ALIGN, IMQ_ERR_SCRATCH = 0, -1, -2, -3, -4
IMQ_NOALLOC_SCRATCH_BYTES = 64 << 20

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_vp = ctypes.c_void_p
_c_float = ctypes.c_float

# name -> (restype, argtypes); must match include/imq.h exactly.
SIGNATURES = {
    "imq_abi_version": (_c_int, []),
    "imq_strerror": (ctypes.c_char_p, [_c_int]),
    "imq_dequant_w4": (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_i64, _c_int, _c_vp, _c_i64, _c_i64, _c_int,
                                _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_int, _c_vp]),
    "imq_dequant_w2": (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_i64, _c_int, _c_vp, _c_i64, _c_i64, _c_int,
                                _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_int, _c_vp]),
    "imq_dequant_w8": (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_int, _c_i64, _c_i64, _c_vp, _c_i64, _c_int,
                                _c_vp]),
    "imq_pack_w4": (_c_int, [_c_vp, _c_i64, _c_int, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp,
                             _c_i64, _c_vp]),
    "imq_pack_w2": (_c_int, [_c_vp, _c_i64, _c_int, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp,
                             _c_i64, _c_vp]),
    "imq_pack_w8": (_c_int, [_c_vp, _c_i64, _c_int, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp]),
    "imq_linear_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "imq_linear_w4_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                               _c_int, _c_i64, _c_i64, _c_int]),
    "imq_linear_w4": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_i64, _c_int,
                               _c_vp, _c_i64, _c_i64, _c_int, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64,
                               _c_vp]),
    "imq_line_tile": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp]),
    "imq_line_untile": (_c_int, [_c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp]),
    "imq_linear_w4_tiled": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_i64, _c_int,
                                     _c_vp, _c_i64, _c_i64, _c_int, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64,
                                     _c_vp]),
    "imq_linear_w8_tiled": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_int, _c_i64,
                                     _c_vp, _c_i64, _c_vp, _c_i64, _c_vp]),
    "imq_linear_w2_tiled": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_i64, _c_int,
                                     _c_vp, _c_i64, _c_i64, _c_int, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64,
                                     _c_vp]),
    "imq_linear_w4_noalloc": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_i64,
                                       _c_int, _c_vp, _c_i64, _c_i64, _c_int, _c_i64, _c_i64, _c_vp, _c_i64,
                                       _c_vp]),
    "imq_linear_w2": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_i64, _c_int,
                               _c_vp, _c_i64, _c_i64, _c_int, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64,
                               _c_vp]),
    "imq_linear_w8": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_int, _c_i64,
                               _c_vp, _c_i64, _c_vp, _c_i64, _c_vp]),
    "imq_moe_rows_w4": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_i64, _c_vp,
                                 _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_i64, _c_i64, _c_int, _c_i64, _c_i64,
                                 _c_vp, _c_i64, _c_vp]),
    "imq_moe_workspace_bytes": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "imq_moe_experts_w4": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64,
                                    _c_vp, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,
                                    _c_vp, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_i64,
                                    _c_int, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp]),
    "imq_moe_experts_w4_ex": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_int, _c_vp, _c_i64,
                                       _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,
                                       _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_i64,
                                       _c_int, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_int, _c_int,
                                       _c_float, _c_float, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp]),
    "imq_probe_sink_bytes": (_c_i64, []),
    "imq_probe_stream": (_c_int, [_c_vp, _c_vp, _c_int, _c_i64, _c_int, _c_int, _c_int, _c_vp, _c_i64, _c_vp]),
    "imq_probe_copy": (_c_int, [_c_vp, _c_vp, _c_i64, _c_int, _c_int, _c_vp]),
    "imq_probe_empty": (_c_int, [_c_int, _c_vp]),
    "imq_probe_mfma": (_c_int, [_c_int, _c_i64, _c_int, _c_vp, _c_i64, _c_vp]),
    "imq_gptq_int2_workspace_bytes": (_c_i64, [_c_i64, _c_i64]),
    "imq_gptq_int2_params": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_int, ctypes.c_double, _c_vp, _c_vp, _c_vp]),
    "imq_gptq_int2_solve": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_i64, _c_int, ctypes.c_double,
                                     _c_i64, _c_vp, _c_i64, _c_vp, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64,
                                     _c_vp]),
    "imq_launch_plan": (_c_int, [_c_int, _c_vp, _c_vp]),
}

IMQ_PLAN_W4_LINE, IMQ_PLAN_W4_KSPLIT, IMQ_PLAN_W4_WSPLIT, IMQ_PLAN_W4_SKINNY = 1, 2, 3, 4
IMQ_PLAN_W2_LINE, IMQ_PLAN_W2_KSPLIT, IMQ_PLAN_W8_LINE, IMQ_PLAN_GEMM, IMQ_PLAN_GEMM_RB = 5, 6, 7, 8, 9


class ImqUnavailable(RuntimeError):
    """libimq.so is not built or cannot be loaded."""


class ImqError(RuntimeError):
    """A libimq call returned a non-zero status."""

    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(f"{fn} failed with status {status}: {msg}")
        self.status = status


_LIB = None
_LOCK = threading.Lock()


def lib():
    """The loaded library (thread-safe lazy load). Raises ImqUnavailable."""
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        import torch  # noqa: F401  -- bind libimq to torch's HIP runtime (see module docstring)
        if not os.path.exists(LIB_PATH):
            raise ImqUnavailable(f"{LIB_PATH} not built (run `python -m infinitemodel_amd.build`)")
        try:
            L = ctypes.CDLL(LIB_PATH)
        except OSError as exc:
            raise ImqUnavailable(f"cannot load {LIB_PATH}: {exc}") from exc
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _LIB = L
        return _LIB


def call(name: str, *args) -> None:
    """Call a status-returning entry point; raise ImqError on a non-zero status."""
    L = lib()
    rc = getattr(L, name)(*args)
    if rc != IMQ_OK:
        raise ImqError(name, rc, L.imq_strerror(rc).decode())


def dtype_code(dt) -> int:
    import torch
    if dt == torch.bfloat16:
        return IMQ_DT_BF16
    if dt == torch.float16:
        return IMQ_DT_FP16
    if dt == torch.float32:
        return IMQ_DT_FP32
    raise TypeError(f"unsupported dtype {dt} (bf16/fp16/fp32 only)")


def launch_plan(kind: int, M: int, K: int, G: int, N: int, sqn: int = 0, sxm: int = 0, ssn: int = 0,
                sdt: int = IMQ_DT_BF16, max_lds: int = 160 * 1024, cus: int = 256):
    """The dispatcher's launch plan for a shape (imq_launch_plan; host code only, no device):
    None when that kernel does not take the call, else (p1, p2, p3, lds_bytes)."""
    inp = (ctypes.c_int64 * 10)(M, K, G, N, sqn, sxm, ssn, sdt, max_lds, cus)
    out = (ctypes.c_int64 * 5)()
    call("imq_launch_plan", kind, ctypes.cast(inp, ctypes.c_void_p), ctypes.cast(out, ctypes.c_void_p))
    return tuple(out[1:]) if out[0] else None
