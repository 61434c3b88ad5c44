"""GPU GPTQ int2 solver (imq_gptq_int2_params / imq_gptq_int2_solve, the reference's
gptq_pack.py:78-189) against its host restatement (oracle/gptq.py): bit-identical codes, scales,
zeros and dequantized weights -- both compute in float32 with every operation rounded on its own
and the same summation order. Shapes: partial last block, a padded last group (tail crumbs at the
last group's zero point), group 128, wide groups; and the _GPTQ class end to end."""
import numpy as np
import pytest

from oracle import gptq as og

pytestmark = pytest.mark.gpu


def _hessian(r, in_f, n=2048):
    X = r.standard_normal((n, in_f)) @ (np.eye(in_f) + 0.3 * r.standard_normal((in_f, in_f)) / np.sqrt(in_f))
    return 2.0 / n * X.T @ X


def _solve_gpu(dev, W, Hinv, G, blocksize=128, grid=48, maxshrink=0.75):
    import torch
    from infinitemodel_amd import _lib
    from infinitemodel_amd.ops import _ptr, _stream, call
    out, in_f = W.shape
    ng = -(-in_f // G)
    Wt = torch.from_numpy(W.copy()).to(dev)
    Ht = torch.from_numpy(np.ascontiguousarray(Hinv)).to(dev)
    q = torch.full((out, ng * G // 4), 0xAB, dtype=torch.uint8, device=dev)
    s = torch.empty((out, ng), dtype=torch.float32, device=dev)
    z = torch.empty_like(s)
    dq = torch.empty((out, in_f), dtype=torch.float32, device=dev)
    nws = int(_lib.lib().imq_gptq_int2_workspace_bytes(out, blocksize))
    ws = torch.empty(nws, dtype=torch.uint8, device=dev)
    call("imq_gptq_int2_solve", _ptr(Wt), Wt.stride(0), out, in_f, _ptr(Ht), Ht.stride(0), G, grid, maxshrink,
         blocksize, _ptr(q), q.stride(0), _ptr(s), _ptr(z), s.stride(0), _ptr(dq), dq.stride(0), _ptr(ws), nws,
         _stream(dev))
    torch.cuda.synchronize()
    return q.cpu().numpy(), s.cpu().numpy(), z.cpu().numpy(), dq.cpu().numpy()


@pytest.mark.parametrize("out,in_f,G,scale", [(96, 320, 64, 0.02), (130, 200, 64, 0.02), (64, 384, 128, 1.0),
                                              (200, 256, 64, 3.0)])
def test_gptq_solve_bit_identical_to_host(dev, out, in_f, G, scale):
    r = np.random.default_rng(out + in_f)
    W = (r.standard_normal((out, in_f)) * scale).astype(np.float32)
    W[:3] *= 40.0                                  # a few wide rows
    Hinv, _ = og.hinv_from_h(_hessian(r, in_f))
    q_h, s_h, z_h, dq_h = og.solve(W, Hinv, G)
    q_g, s_g, z_g, dq_g = _solve_gpu(dev, W, Hinv, G)
    assert np.array_equal(s_g, s_h) and np.array_equal(z_g, z_h)
    assert np.array_equal(q_g, q_h)
    assert np.array_equal(dq_g, dq_h)


def test_gptq_find_params_bit_identical(dev):
    import torch
    from infinitemodel_amd import gptq_pack as gp
    r = np.random.default_rng(7)
    Wg = (r.standard_normal((1000, 64)) * 0.02).astype(np.float32)
    Wg[:100] *= 30.0
    Wg[100:110] = 0.0
    s_h, z_h = og.find_params(Wg)
    s_g, z_g = gp._find_params(torch.from_numpy(Wg).to(dev), 48, 0.75)
    assert np.array_equal(s_g.cpu().numpy(), s_h) and np.array_equal(z_g.cpu().numpy(), z_h)


def test_gptq_class_end_to_end(dev):
    """add_batch over two batches, solve: the returned crumbs / scales decode to the weight
    written back into the Linear, in the RTN int2 packer's layout and the weight's dtype."""
    import torch
    from infinitemodel_amd import gptq_pack as gp
    torch.manual_seed(0)
    lin = torch.nn.Linear(256, 96, bias=False).to(torch.bfloat16).to(dev)
    g = gp._GPTQ(lin, dev)
    for _ in range(2):
        g.add_batch(torch.randn(4, 32, 256, device=dev, dtype=torch.bfloat16))
    assert g.n == 256
    q, s, z = g.solve(64, 48, 0.75, 0.01)
    assert q.shape == (96, 64) and q.dtype == torch.uint8
    assert s.shape == (96, 4) and s.dtype == torch.bfloat16 and z.dtype == torch.bfloat16
    codes = torch.stack([(q >> (2 * i)) & 3 for i in range(4)], dim=2).reshape(96, 256).float()
    dq = (codes - z.float().repeat_interleave(64, dim=1)) * s.float().repeat_interleave(64, dim=1)
    w = lin.weight.detach().float().cpu()
    # the solver's fp32 dequant, written back in bf16: equal to the bf16 rounding of the decode
    # from fp32 scales (s, z came back rounded to bf16, so compare with a relative bound)
    assert torch.allclose(w, dq, rtol=2e-2, atol=1e-4)
    assert torch.equal(z.float(), z.float().round()) and float(z.float().min()) >= 0 and float(z.float().max()) <= 3
