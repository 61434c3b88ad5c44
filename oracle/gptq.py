"""CPU restatement of the reference's GPTQ int2 solver (gptq_pack.py:78-189) -- test
infrastructure only (imported by tests/, never by the package).

What it follows:
  * find_params      gptq_pack.py:78-100 (_find_params): asymmetric 0..3 grid, range-shrink
                     candidates p = 1 - k / grid for k < int(maxshrink * grid), scale
                     max((xmax - xmin) * fp32(p / 3), 1e-8), zero clamp(round(-xmin * p / s), 0, 3),
                     the candidate with the smallest sum |dq - w|^2.4 (first one on ties);
  * solve            gptq_pack.py:124-176 (_GPTQ.solve after the Cholesky stage): blocks of
                     `blocksize` columns, group parameters from W's block-start values at each
                     group's first column, q = clamp(round(w / s + z), 0, 3), dq = (q - z) s,
                     err = (w - dq) / Hinv[c, c], in-block propagation W1[:, j] -= err Hinv[c, j],
                     cross-block W[:, i2:] -= Err1 @ Hinv[i1:i2, i2:]; padded tail columns take the
                     last group's rounded zero point (176-178); crumb packing (179-180).

The arithmetic is float32 with every operation rounded on its own (numpy's float32 ufuncs), in
an order fixed here -- sums over columns and over K left to right, each product rounded before
the add -- so that the HIP solver (compiled without FMA contraction) reproduces it bit for bit.
|x|^2.4 is pow24() below, a deterministic range-reduced evaluation shared with the kernel
(torch.pow, the reference's, is not specified to the last bit); against float64 np.power its
relative error is below 2e-6, which the tests pin. The Cholesky stage (dead columns, damping,
cholesky_inverse, the upper factor -- gptq_pack.py:130-139) is an input: both the kernel and
this restatement take the same Hinv.
"""
from __future__ import annotations

import math

import numpy as np

f32 = np.float32
_LN2 = f32(0.6931471805599453)
_INV_LN2 = f32(1.4426950408889634)
_SQRT2 = f32(1.4142135623730951)
_C04 = f32(0.4)
# atanh series 2 t (1 + t^2/3 + t^4/5 + t^6/7 + t^8/9), |t| <= 0.1716
_A = (f32(1.0 / 9.0), f32(1.0 / 7.0), f32(1.0 / 5.0), f32(1.0 / 3.0), f32(1.0))
# 2^f = e^(f ln2), |f| <= 0.5: Taylor through degree 7 (Horner in u = f ln2)
_E = (f32(1.0 / 5040.0), f32(1.0 / 720.0), f32(1.0 / 120.0), f32(1.0 / 24.0), f32(1.0 / 6.0), f32(0.5),
      f32(1.0), f32(1.0))


def pow24(a):
    """|a|^2.4 in float32 (a >= 0 array) as a^2 * a^0.4: a = m 2^e with m in [sqrt(1/2), sqrt(2)),
    log2 a = e + ln(m) / ln 2 by the atanh series, y = 0.4 log2 a split as n + f with n = rint(y),
    2^f by its Taylor polynomial, 2^n placed in the exponent. Inputs below 2^-50 give 0 (the
    result would be below 2^-120)."""
    a = np.asarray(a, dtype=f32)
    out = np.zeros_like(a)
    ok = a >= f32(2.0 ** -50)
    x = a[ok]
    bits = x.view(np.int32)
    e = ((bits >> 23) & 0xFF) - 127
    m = ((bits & 0x7FFFFF) | 0x3F800000).view(f32)
    big = m > _SQRT2
    m = np.where(big, m * f32(0.5), m)
    e = np.where(big, e + 1, e)
    t = (m - f32(1.0)) / (m + f32(1.0))
    t2 = t * t
    p = _A[0]
    for c in _A[1:]:
        p = p * t2 + c
    ln_m = (t + t) * p
    log2a = e.astype(f32) + ln_m * _INV_LN2
    y = _C04 * log2a
    n = np.rint(y)
    u = (y - n) * _LN2
    q = _E[0]
    for c in _E[1:]:
        q = q * u + c
    ni = n.astype(np.int32)                      # within [-20, 52] for these inputs
    scale = ((ni + 127).astype(np.int32) << 23).view(f32)
    with np.errstate(over="ignore"):            # a^2 past the float32 range: inf, as on the GPU
        out[ok] = (x * x) * (q * scale)
    return out


def shrink_factors(grid: int, maxshrink: float):
    """(fp32(p / 3), fp32(p)) for the candidates p = 1 - k / grid, k < int(maxshrink * grid): the
    reference's Python-double p meets the float32 tensors as a float32 scalar."""
    ks = range(int(maxshrink * grid))
    return ([f32((1.0 - k / grid) / 3.0) for k in ks], [f32(1.0 - k / grid) for k in ks])


def find_params(Wg, grid: int = 48, maxshrink: float = 0.75):
    """gptq_pack.py:78-100. Wg [rows, g] float32 -> (scale [rows], zero [rows]) float32."""
    Wg = np.asarray(Wg, dtype=f32)
    xmin = np.minimum(Wg.min(axis=1), f32(0.0))
    xmax = np.maximum(Wg.max(axis=1), f32(0.0))
    best_err = np.full(Wg.shape[0], np.inf, dtype=f32)
    best_s = np.ones(Wg.shape[0], dtype=f32)
    best_z = np.zeros(Wg.shape[0], dtype=f32)
    span = xmax - xmin
    for pf3, pf in zip(*shrink_factors(grid, maxshrink)):
        s1 = np.maximum(span * pf3, f32(1e-8))
        z1 = np.clip(np.rint(((-xmin) * pf) / s1), f32(0.0), f32(3.0))
        err = np.zeros(Wg.shape[0], dtype=f32)
        for c in range(Wg.shape[1]):
            w = Wg[:, c]
            q = np.clip(np.rint(w / s1 + z1), f32(0.0), f32(3.0))
            dq = (q - z1) * s1
            err = err + pow24(np.abs(dq - w))
        better = err < best_err
        best_err = np.where(better, err, best_err)
        best_s = np.where(better, s1, best_s)
        best_z = np.where(better, z1, best_z)
    return best_s, best_z


def solve(W, Hinv, group_size: int = 64, grid: int = 48, maxshrink: float = 0.75, blocksize: int = 128):
    """gptq_pack.py:141-180 on float32 W [out, in_f] (dead columns already zeroed) and the upper
    Cholesky factor Hinv [in_f, in_f] of the damped H^-1. Returns (qpacked uint8 [out, in_pad/4],
    scale fp32 [out, ng], zero fp32 [out, ng], dq fp32 [out, in_f])."""
    W = np.array(W, dtype=f32, copy=True)
    Hinv = np.asarray(Hinv, dtype=f32)
    G = group_size
    out, in_f = W.shape
    if blocksize % G:
        raise ValueError("blocksize must be a multiple of the group size")
    ng = (in_f + G - 1) // G
    in_pad = ng * G
    qall = np.zeros((out, in_pad), dtype=np.uint8)
    scales = np.zeros((out, ng), dtype=f32)
    zeros = np.zeros((out, ng), dtype=f32)
    DQ = np.zeros_like(W)
    for i1 in range(0, in_f, blocksize):
        i2 = min(i1 + blocksize, in_f)
        count = i2 - i1
        W1 = W[:, i1:i2].copy()
        Err1 = np.zeros((out, count), dtype=f32)
        for i in range(count):
            col = i1 + i
            g = col // G
            if col % G == 0:
                sc, zp = find_params(W[:, col:min(col + G, in_f)], grid, maxshrink)
                scales[:, g] = sc
                zeros[:, g] = zp
            w = W1[:, i]
            d = Hinv[col, col]
            s = scales[:, g]
            z = zeros[:, g]
            q = np.clip(np.rint(w / s + z), f32(0.0), f32(3.0))
            dq = (q - z) * s
            qall[:, col] = q.astype(np.uint8)
            DQ[:, col] = dq
            err = (w - dq) / d
            for j in range(i + 1, count):
                W1[:, j] = W1[:, j] - err * Hinv[col, i1 + j]
            Err1[:, i] = err
        if i2 < in_f:
            acc = np.zeros((out, in_f - i2), dtype=f32)
            for k in range(count):
                acc = acc + Err1[:, k:k + 1] * Hinv[i1 + k, i2:][None, :]
            W[:, i2:] = W[:, i2:] - acc
    if in_pad != in_f:
        qall[:, in_f:] = np.clip(np.rint(zeros[:, -1]), 0, 3).astype(np.uint8)[:, None]
    qpacked = (qall[:, 0::4] | (qall[:, 1::4] << 2) | (qall[:, 2::4] << 4) | (qall[:, 3::4] << 6)).astype(np.uint8)
    return qpacked, scales, zeros, DQ


def hinv_from_h(H, percdamp: float = 0.01):
    """The reference's Cholesky stage in float64 (gptq_pack.py:128-139): dead diagonal entries set
    to 1, damping percdamp * mean(diag), cholesky -> cholesky_inverse -> upper cholesky. Returns
    (Hinv float32, dead mask) -- the caller zeroes W's dead columns."""
    H = np.array(H, dtype=np.float64, copy=True)
    dead = np.diag(H) == 0
    idx = np.nonzero(dead)[0]
    H[idx, idx] = 1.0
    damp = percdamp * float(np.mean(np.diag(H)))
    H[np.arange(H.shape[0]), np.arange(H.shape[0])] += damp
    L = np.linalg.cholesky(H)
    Hi = np.linalg.inv(L).T @ np.linalg.inv(L)
    U = np.linalg.cholesky(Hi).T
    return U.astype(f32), dead


def rtn_params_identity(Wg, grid: int = 48, maxshrink: float = 0.75):
    """The same search in float64 with np.power: the closed-form check for find_params."""
    Wg = np.asarray(Wg, dtype=np.float64)
    xmin = np.minimum(Wg.min(axis=1), 0.0)
    xmax = np.maximum(Wg.max(axis=1), 0.0)
    best = (np.full(Wg.shape[0], math.inf), np.ones(Wg.shape[0]), np.zeros(Wg.shape[0]))
    errs = []
    for k in range(int(maxshrink * grid)):
        p = 1.0 - k / grid
        s1 = np.maximum((xmax - xmin) * (p / 3.0), 1e-8)
        z1 = np.clip(np.rint(-xmin * p / s1), 0, 3)
        q = np.clip(np.rint(Wg / s1[:, None] + z1[:, None]), 0, 3)
        dq = (q - z1[:, None]) * s1[:, None]
        err = np.power(np.abs(dq - Wg), 2.4).sum(axis=1)
        errs.append(err)
        better = err < best[0]
        best = (np.where(better, err, best[0]), np.where(better, s1, best[1]), np.where(better, z1, best[2]))
    return best[1], best[2], np.stack(errs, axis=1)
