"""numpy restatement of the reference's weight-only quantization arithmetic (TEST ORACLE ONLY).

Every function states the reference lines it follows. All float arithmetic is done the way
torch's CPU kernels do it: each elementwise op is evaluated in float32 and rounded once to the
tensor dtype (bf16 / fp16 / fp32); numpy float32 array ops are IEEE single-rounding, and
``np.rint`` is round-half-to-even like ``torch.round``.

Tensors of a reduced dtype are carried as float32 arrays whose values are exactly
representable in that dtype, together with a dtype name ("bf16", "fp16", "fp32").

Pins (independent checks, see tests/test_oracle.py):
  * bf16 RNE emulation      -> hand-computed constants + torch's own bf16 conversion/arithmetic
                               over an exhaustive operand grid.
  * nibble / crumb layout   -> brute force of all 256 byte values and literal packed bytes of a
                               hand-derived ramp.
  * RTN packers             -> hand-derived group KATs (incl. the constant-group quirk), range
                               and round-trip error invariants, padded-tail KAT.
  * int8 packer             -> all-zero row KAT, |q|<=127 and amax-element invariants,
                               bf16-division quirk KAT.
  * dequant-then-matmul     -> torch tinygemm CPU (independent ATen int4 consumer with its own
                               (q-8)*S + (8-z)*S dequant), one-hot column extraction.
  * int8_gemm_ref           -> hand-computed KAT; torch float64 dequantize-then-F.linear (the
                               scale applied per weight row), with a wrong-axis negative control.
  * dequant_exact           -> hand-computed KATs (integer and non-integer zeros); torch float64
                               over torch's own bf16 casts; rounded once to bf16 it equals the
                               reference dequant for integer zeros; within one rounding of it for
                               C3's non-integer zeros.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32
DTYPES = ("bf16", "fp16", "fp32")


# ---------------------------------------------------------------------------------------------
# rounding helpers
# ---------------------------------------------------------------------------------------------
def f32_to_bf16_bits(x) -> np.ndarray:
    """float32 -> bf16 bit pattern, round-to-nearest-even (torch's float->bfloat16 rule)."""
    x = np.ascontiguousarray(x, dtype=F32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r = np.where(nan, np.uint16(0x7FC0), r)
    return r


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(F32)


def round_to(x, dt: str) -> np.ndarray:
    """Round float32 values to dtype ``dt`` (returned as float32 holding representable values)."""
    x = np.asarray(x, dtype=F32)
    if dt == "fp32":
        return x.copy()
    if dt == "bf16":
        return bf16_bits_to_f32(f32_to_bf16_bits(x))
    if dt == "fp16":
        return x.astype(np.float16).astype(F32)
    raise ValueError(dt)


def dt_op(a, b, op, dt: str) -> np.ndarray:
    """One torch elementwise op on dtype-``dt`` tensors: float32 evaluation, one rounding."""
    a = np.asarray(a, F32)
    b = np.asarray(b, F32)
    if op == "+":
        r = a + b
    elif op == "-":
        r = a - b
    elif op == "*":
        r = a * b
    elif op == "/":
        r = a / b
    else:
        raise ValueError(op)
    return round_to(r, dt)


# ---------------------------------------------------------------------------------------------
# packers (shard_compile.py:50-94, 97-140, 170-178; worker_quant.py:1588-1608, 1921-1944,
# 511-529 (int8 _pack8_expert), 2394-2436 (_pack4_expert/_pack4_3d))
# ---------------------------------------------------------------------------------------------
def _rtn_groups(W, G: int, qmax: int):
    """Shared RTN body of pack_linear_int4/int2 (shard_compile.py:81-91 / 58-68): zero-pad K to
    a multiple of G *before* the min/max (the pad participates), fp32 min/max per group,
    scale=clamp((max-min)/qmax, 1e-8), zero=clamp(round(-min/scale),0,qmax),
    q=clamp(round(W/scale + zero),0,qmax) -- the divide and the add are two separate roundings."""
    W = np.asarray(W, F32)
    out, in_f = W.shape
    ng = -(-in_f // G)
    in_pad = ng * G
    Wp = np.zeros((out, in_pad), F32)
    Wp[:, :in_f] = W
    Wg = Wp.reshape(out, ng, G)
    wmin = Wg.min(axis=2)
    wmax = Wg.max(axis=2)
    scale = np.maximum((wmax - wmin) / F32(qmax), F32(1e-8)).astype(F32)
    zero = np.clip(np.rint((-wmin) / scale), 0, qmax).astype(F32)
    t = (Wg / scale[:, :, None]).astype(F32)
    t = (t + zero[:, :, None]).astype(F32)
    q = np.clip(np.rint(t), 0, qmax).astype(np.uint8).reshape(out, in_pad)
    return q, scale, zero, in_f


def pack_linear_int4(W, group_size: int = 128, dt: str = "bf16"):
    """shard_compile.pack_linear_int4 (shard_compile.py:74-94) == worker_quant._quantize_linear4
    (worker_quant.py:1588-1608). ``W`` holds dtype-``dt`` values. Returns
    (qweight u8 [N, K_pad/2], scale [N, ng] (dt values), zero [N, ng] (dt values), in_features).
    Byte j = column 2j (low nibble) | column 2j+1 << 4 (shard_compile.py:93)."""
    q, scale, zero, in_f = _rtn_groups(W, group_size, 15)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    return packed, round_to(scale, dt), round_to(zero, dt), in_f


def pack_linear_int2(W, group_size: int = 64, dt: str = "bf16"):
    """shard_compile.pack_linear_int2 (shard_compile.py:50-71) == worker_quant._quantize_linear2
    (worker_quant.py:1921-1944). Crumb i of byte j = column 4j+i, lowest bits first."""
    q, scale, zero, in_f = _rtn_groups(W, group_size, 3)
    packed = (q[:, 0::4] | (q[:, 1::4] << 2) | (q[:, 2::4] << 4) | (q[:, 3::4] << 6)).astype(np.uint8)
    return packed, round_to(scale, dt), round_to(zero, dt), in_f


def pack_linear_int4_3d(W3, group_size: int = 128, dt: str = "bf16", in_major: bool = False):
    """shard_compile.pack_linear_int4_3d (shard_compile.py:97-140) == worker_quant._pack4_3d
    (2415-2436): pack_linear_int4 per expert; ``in_major`` transposes each expert first.
    Returns (qweight [E,N,K_pad/2], scale [E,N,ng], zero [E,N,ng], in_features, ng)."""
    W3 = np.asarray(W3, F32)
    qs, ss, zs = [], [], []
    in_f = None
    for e in range(W3.shape[0]):
        We = W3[e].T.copy() if in_major else W3[e]
        q, s, z, in_f = pack_linear_int4(We, group_size, dt)
        qs.append(q)
        ss.append(s)
        zs.append(z)
    return np.stack(qs), np.stack(ss), np.stack(zs), in_f, ss[0].shape[1]


def pack_linear_int8(W, dt: str = "bf16"):
    """shard_compile.pack_linear_int8 (shard_compile.py:170-178) == worker_quant._pack8_expert
    (worker_quant.py:511-529). Arithmetic stays in W's own dtype: amax exact, ``/127.0``
    evaluated in float32 then rounded to dt, clamp(min=1e-8) against dt(1e-8),
    ``W / scale`` rounded to dt *before* ``.round()`` (so e.g. 126.6 can round via bf16 126.5 to
    126), clamp to [-127, 127]. Returns (qweight int8 [N,K], scale [N,1] dt values)."""
    W = np.asarray(W, F32)
    amax = np.abs(W).max(axis=1, keepdims=True)
    scale = dt_op(amax, F32(127.0), "/", dt)
    scale = np.maximum(scale, round_to(F32(1e-8), dt))
    # fp16 quirk: fp16(1e-8) is 0, so an all-zero row has scale 0 and codes 0/0 = NaN; the
    # float->int8 cast of NaN then gives 0 on x86 (torch's CPU cast does the same).
    with np.errstate(invalid="ignore", divide="ignore"):
        t = dt_op(W, scale, "/", dt)
        q = np.clip(np.rint(t), -127, 127).astype(np.int8)
    return q, scale


# ---------------------------------------------------------------------------------------------
# unpack + reference dequant (worker_quant.py:638-648, 1652-1664, 439, 2033-2043)
# ---------------------------------------------------------------------------------------------
def unpack_int4(packed) -> np.ndarray:
    """[N, K_pad/2] u8 -> [N, K_pad] codes 0..15; low nibble = even column (worker_quant.py:641-643)."""
    p = np.asarray(packed, np.uint8)
    lo = p & 0x0F
    hi = p >> 4
    return np.stack((lo, hi), axis=-1).reshape(p.shape[:-1] + (p.shape[-1] * 2,))


def unpack_int2(packed) -> np.ndarray:
    """[N, K_pad/4] u8 -> [N, K_pad] codes 0..3; crumb i = column 4j+i (worker_quant.py:1655-1659)."""
    p = np.asarray(packed, np.uint8)
    c = [(p >> (2 * i)) & 0x3 for i in range(4)]
    return np.stack(c, axis=-1).reshape(p.shape[:-1] + (p.shape[-1] * 4,))


def _dequant_groups(q, scale, zero, G: int, in_features: int, dt: str):
    """``(q.to(dt) - zero.to(dt)) * scale.to(dt)`` with each op rounding in dt
    (worker_quant.py:646-647). For integer zeros the subtraction is exact, so the result is one
    exact product rounded once; non-integer zeros (fp16 int2 configs) round twice."""
    N = q.shape[0]
    ng = scale.shape[1]
    qf = q.reshape(N, ng, G).astype(F32)
    z = round_to(zero, dt)[:, :, None]
    s = round_to(scale, dt)[:, :, None]
    d = dt_op(qf, z, "-", dt)
    w = dt_op(d, s, "*", dt)
    return w.reshape(N, ng * G)[:, :in_features].copy()


def dequant_int4(packed, scale, zero, in_features: int, group_size: int = 128, dt: str = "bf16"):
    """QuantLinear4._dequant(dt) (worker_quant.py:638-648)."""
    return _dequant_groups(unpack_int4(packed), scale, zero, group_size, in_features, dt)


def dequant_int2(packed, scale, zero, in_features: int, group_size: int = 64, dt: str = "bf16"):
    """QuantLinear2._dequant(dt) (worker_quant.py:1652-1664)."""
    return _dequant_groups(unpack_int2(packed), scale, zero, group_size, in_features, dt)


def dequant_exact(codes, scale, zero, G: int, in_features: int):
    """float64 ``(q - bf16(z)) * bf16(s)`` with no rounding of the product: the weight the fused
    kernels accumulate with (the reference's split-K GEMV keeps the dequantized weight in fp32
    un-rounded, worker_quant.py:1176-1177; scale/zero are first taken to bf16 as
    _dequant(torch.bfloat16) does, worker_quant.py:646-647). ``codes`` are unpacked [N, K_pad]."""
    N = codes.shape[0]
    ng = scale.shape[1]
    z = round_to(zero, "bf16").astype(np.float64)[:, :, None]
    s = round_to(scale, "bf16").astype(np.float64)[:, :, None]
    w = (codes.reshape(N, ng, G).astype(np.float64) - z) * s
    return w.reshape(N, ng * G)[:, :in_features]


def promote(a: str, b: str) -> str:
    """torch type promotion between two float dtypes of this path."""
    if a == b:
        return a
    return "fp32"


def dequant_int8(q, scale, scale_dt: str, x_dt: str = "bf16"):
    """QuantLinear naive weight ``qweight.to(x.dtype) * scale`` (worker_quant.py:439): the scale is
    NOT cast, so bf16 x with an fp16 scale promotes to fp32. Returns (values, result dtype)."""
    res = promote(x_dt, scale_dt)
    qf = round_to(np.asarray(q, F32), x_dt)
    return dt_op(qf, np.asarray(scale, F32), "*", res), res


def dequant_int4_3d(packed, scale, zero, e: int, in_features: int, group_size: int = 128, dt: str = "bf16"):
    """Packed4Tensor3D.__getitem__(e) naive path (worker_quant.py:2033-2043): expert e dequant in
    the scale dtype."""
    return dequant_int4(packed[e], scale[e], zero[e], in_features, group_size, dt)


# ---------------------------------------------------------------------------------------------
# dequantize-then-matmul references and error metrics
# ---------------------------------------------------------------------------------------------
def linear_ref(x, Wdeq) -> np.ndarray:
    """Exact (float64) ``x @ Wdeq.T`` of the bf16 activations and the bit-exact dequantized
    weight. The reference's naive path F.linear(x, _dequant(bf16)) (worker_quant.py:853) is this
    product rounded to bf16 after an fp32 accumulation."""
    return np.asarray(x, np.float64) @ np.asarray(Wdeq, np.float64).T


def int8_gemm_ref(x, q, scale) -> np.ndarray:
    """Kernel-form int8 reference: ``s * (x @ q.T)`` exact (worker_quant.py:977-980, 1019-1020)."""
    return (np.asarray(x, np.float64) @ np.asarray(q, np.float64).T) * np.asarray(scale, np.float64).reshape(1, -1)


def max_rel(y, ref) -> float:
    """Normwise max relative error max|y-ref| / max|ref| (the north-star 'max rel err')."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.abs(ref).max()
    return float(np.abs(y - ref).max() / (den if den > 0 else 1.0))


def mean_rel(y, ref) -> float:
    """The reference self-check metric mean|y-ref| / (mean|ref| + 1e-6) (worker_quant.py:368)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(y - ref).mean() / (np.abs(ref).mean() + 1e-6))
