"""Pins of the GPTQ int2 restatement (oracle/gptq.py, the reference's gptq_pack.py:78-189).

* pow24 against float64 np.power (relative error < 2e-6) and its cut-offs;
* find_params against the same search in float64 with np.power: the same candidate wherever
  the two best float64 errors are not within float32 noise of each other;
* solve with Hinv = I (no error propagation): exactly the group search's parameters and
  round-to-nearest codes, column by column;
* solve against a float64 transcription of the reference loop (torch ops): codes agree almost
  everywhere, and GPTQ's proxy loss tr((W - DQ) H (W - DQ)^T) beats round-to-nearest with the
  same parameters -- a dropped or sign-flipped propagation term fails this;
* the crumb layout (column 4 j + i in bits 2 i of byte j) and the padded tail (the last group's
  rounded zero point).
"""
import numpy as np
import pytest
import torch

from oracle import gptq as og


def test_pow24_accuracy_and_cutoffs():
    x = np.logspace(-14, 3, 20001).astype(np.float32)
    y = og.pow24(x).astype(np.float64)
    ref = np.power(x.astype(np.float64), 2.4)
    rel = np.abs(y - ref) / ref
    assert rel.max() < 2e-6, rel.max()
    assert og.pow24(np.array([0.0, 2.0 ** -51, 1e-30], np.float32)).tolist() == [0.0, 0.0, 0.0]
    assert og.pow24(np.array([1.0], np.float32))[0] == np.float32(1.0)
    assert np.isinf(og.pow24(np.array([3e30], np.float32))[0])


def test_find_params_matches_float64_search():
    r = np.random.default_rng(0)
    Wg = (r.standard_normal((400, 64)) * 0.02).astype(np.float32)
    Wg[:40] *= 50.0                                 # wide groups
    Wg[40:60, :] = np.abs(Wg[40:60, :])             # all-positive groups (xmin clamps to 0)
    s, z = og.find_params(Wg)
    s64, z64, errs = og.rtn_params_identity(Wg)
    # the winning candidate's index on each side (scales differ in the last bit between the
    # float32 and float64 products even for the same candidate)
    cand_s = np.maximum((np.maximum(Wg.max(1), 0) - np.minimum(Wg.min(1), 0))[:, None].astype(np.float64)
                        * np.array([(1 - k / 48) / 3 for k in range(36)]), 1e-8)
    k_ours = np.argmin(np.abs(cand_s - s[:, None].astype(np.float64)), axis=1)
    k_f64 = np.argmin(errs, axis=1)
    same = k_ours == k_f64
    assert same.mean() > 0.95, same.mean()
    # where they differ, the two picks' float64 errors are within float32 noise
    for row in np.nonzero(~same)[0]:
        e_ours, e_best = errs[row, k_ours[row]], errs[row].min()
        assert e_ours <= e_best * (1 + 1e-5), (row, e_ours, e_best)
    assert np.array_equal(z[same], z64[same].astype(np.float32))


def test_find_params_degenerate_groups():
    Wg = np.zeros((3, 64), np.float32)
    Wg[1, :] = 0.5
    Wg[2, :] = -0.25
    s, z = og.find_params(Wg)
    assert s[0] == np.float32(1e-8) and z[0] == 0                          # zero span -> clamped scale
    assert z[1] == 0 and np.isclose(s[1], 0.5 / 3, rtol=1e-6)             # [0, 0.5]: z 0, 3 steps
    assert z[2] == 3 and np.isclose(s[2], 0.25 / 3, rtol=1e-6)            # [-0.25, 0]: z 3


def test_solve_identity_hessian_is_round_to_nearest():
    r = np.random.default_rng(1)
    out, in_f, G = 24, 200, 64
    W = (r.standard_normal((out, in_f)) * 0.02).astype(np.float32)
    q, s, z, dq = og.solve(W, np.eye(in_f, dtype=np.float32), G)
    ng = -(-in_f // G)
    codes = np.zeros((out, ng * G), np.uint8)
    for i in range(4):
        codes[:, i::4] = (q >> (2 * i)) & 3
    for g in range(ng):
        c0, c1 = g * G, min(g * G + G, in_f)
        sg, zg = og.find_params(W[:, c0:c1])
        assert np.array_equal(s[:, g], sg) and np.array_equal(z[:, g], zg)
        qq = np.clip(np.rint(W[:, c0:c1] / sg[:, None] + zg[:, None]), 0, 3)
        assert np.array_equal(codes[:, c0:c1], qq.astype(np.uint8))
        assert np.array_equal(dq[:, c0:c1], ((qq - zg[:, None]) * sg[:, None]).astype(np.float32))
    # the padded tail (200 -> 256) holds the last group's rounded zero point
    tail = np.clip(np.rint(z[:, -1]), 0, 3).astype(np.uint8)
    assert np.array_equal(codes[:, in_f:], np.repeat(tail[:, None], ng * G - in_f, axis=1))


def _reference_loop_f64(W, Hinv, G, blocksize=128, grid=48, maxshrink=0.75):
    """gptq_pack.py:141-178 transcribed with float64 torch ops (torch.round, torch.pow)."""
    W = torch.tensor(W, dtype=torch.float64)
    Hinv = torch.tensor(Hinv, dtype=torch.float64)
    out, in_f = W.shape
    ng = -(-in_f // G)
    qall = torch.zeros((out, ng * G), dtype=torch.uint8)
    scales = torch.zeros((out, ng), dtype=torch.float64)
    zeros = torch.zeros((out, ng), dtype=torch.float64)
    DQ = torch.zeros_like(W)

    def find(Wg):
        xmin = Wg.amin(dim=1).clamp(max=0.0)
        xmax = Wg.amax(dim=1).clamp(min=0.0)
        best = (torch.full_like(xmin, float("inf")), torch.ones_like(xmin), torch.zeros_like(xmin))
        for k in range(int(maxshrink * grid)):
            p = 1.0 - k / grid
            s1 = ((xmax - xmin) * (p / 3.0)).clamp(min=1e-8)
            z1 = torch.round(-xmin * p / s1).clamp(0, 3)
            q = torch.clamp(torch.round(Wg / s1.unsqueeze(1) + z1.unsqueeze(1)), 0, 3)
            err = ((q - z1.unsqueeze(1)) * s1.unsqueeze(1) - Wg).abs().pow(2.4).sum(dim=1)
            b = err < best[0]
            best = (torch.where(b, err, best[0]), torch.where(b, s1, best[1]), torch.where(b, z1, best[2]))
        return best[1], best[2]

    for i1 in range(0, in_f, blocksize):
        i2 = min(i1 + blocksize, in_f)
        W1 = W[:, i1:i2].clone()
        Err1 = torch.zeros_like(W1)
        for i in range(i2 - i1):
            col = i1 + i
            if col % G == 0:
                scales[:, col // G], zeros[:, col // G] = find(W[:, col:min(col + G, in_f)])
            s, z = scales[:, col // G], zeros[:, col // G]
            w = W1[:, i]
            q = torch.clamp(torch.round(w / s + z), 0, 3)
            dq = (q - z) * s
            qall[:, col] = q.to(torch.uint8)
            DQ[:, col] = dq
            err = (w - dq) / Hinv[col, col]
            W1[:, i + 1:] -= err.unsqueeze(1) * Hinv[col, i1 + i + 1:i2].unsqueeze(0)
            Err1[:, i] = err
        if i2 < in_f:
            W[:, i2:] -= Err1 @ Hinv[i1:i2, i2:]
    return qall.numpy(), scales.numpy(), zeros.numpy(), DQ.numpy()


def _hessian(r, in_f, n=4096):
    base = r.standard_normal((n, in_f)).astype(np.float64)
    mix = np.eye(in_f) + 0.3 * r.standard_normal((in_f, in_f)) / np.sqrt(in_f)
    X = base @ mix
    return 2.0 / n * X.T @ X


def test_solve_against_float64_reference_loop_and_proxy_loss():
    r = np.random.default_rng(2)
    out, in_f, G = 48, 320, 64
    W = (r.standard_normal((out, in_f)) * 0.02).astype(np.float32)
    H = _hessian(r, in_f)
    Hinv, dead = og.hinv_from_h(H)
    assert not dead.any()
    q, s, z, dq = og.solve(W, Hinv, G)
    codes = np.stack([(q >> (2 * i)) & 3 for i in range(4)], axis=2).reshape(out, -1)[:, :in_f]
    q64, s64, z64, dq64 = _reference_loop_f64(W, Hinv, G)
    agree = (codes == q64[:, :in_f]).mean()
    assert agree > 0.98, agree
    assert np.isclose(s, s64, rtol=1e-3).mean() > 0.97

    def proxy(D):
        E = (W.astype(np.float64) - D)
        return float(np.einsum("ij,jk,ik->", E, H, E))

    # round-to-nearest with the same group parameters, no propagation
    rtn = np.zeros_like(dq, dtype=np.float64)
    for g in range(s.shape[1]):
        c0, c1 = g * G, min(g * G + G, in_f)
        qq = np.clip(np.rint(W[:, c0:c1] / s[:, g:g + 1] + z[:, g:g + 1]), 0, 3)
        rtn[:, c0:c1] = (qq - z[:, g:g + 1]) * s[:, g:g + 1]
    assert proxy(dq.astype(np.float64)) < 0.9 * proxy(rtn), (proxy(dq), proxy(rtn))


def test_crumb_layout():
    r = np.random.default_rng(3)
    W = (r.standard_normal((5, 64)) * 0.02).astype(np.float32)
    q, s, z, dq = og.solve(W, np.eye(64, dtype=np.float32), 64)
    assert q.shape == (5, 16) and q.dtype == np.uint8
    # byte j holds columns 4j..4j+3, lowest bits first: decoding reproduces dq
    codes = np.stack([(q >> (2 * i)) & 3 for i in range(4)], axis=2).reshape(5, 64)
    assert np.array_equal(((codes - z[:, :1]) * s[:, :1]).astype(np.float32), dq)


def test_solve_refuses_misaligned_blocks():
    with pytest.raises(ValueError):
        og.solve(np.zeros((2, 64), np.float32), np.eye(64, dtype=np.float32), 64, blocksize=96)
