"""HIP graph replay of every kernel family, the way bench.py times them.

An op captured in a graph and replayed several times -- with eager work of the library and of
torch between the replays -- must give results bit-identical to its eager call on every replay:
no memset nodes, no state carried from one call to the next, workspaces reused correctly. The
eager result itself is checked against the oracle by the parity tests of each family."""
import numpy as np
import pytest

from oracle import moe as om
from oracle import quant as oq
from tests import _cases as C

pytestmark = pytest.mark.gpu


def _replay_check(fn, between):
    import torch
    eager = fn().clone()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    torch.cuda.synchronize()
    for i in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        between()
        torch.cuda.synchronize()
    return eager


def _x(dev, M, K, seed):
    return C.to_torch(C.bf16_normal(C.rng(seed), (M, K)), "bf16", dev)


@pytest.mark.parametrize("M", [1, 8, 64, 512])
def test_graph_linear_w4(dev, M):
    """Line kernel (M 1), K-split kernel + reduce launch (M 8), prefill GEMM (M 64, 512)."""
    from infinitemodel_amd import ops
    c = C.int4_case(1024, 2048, 128, seed=31)
    q, s, z = C.u8(c["q"], dev), C.to_torch(c["s"], "bf16", dev), C.to_torch(c["z"], "bf16", dev)
    x, x2 = _x(dev, M, 2048, 1), _x(dev, 16, 2048, 2)
    _replay_check(lambda: ops.linear_w4(x, q, 128, (s, z)),
                  lambda: (ops.linear_w4(x2, q, 128, (s, z)), x2.float().sum()))


@pytest.mark.parametrize("M", [1, 8, 64])
def test_graph_linear_w2(dev, M):
    from infinitemodel_amd import ops
    c = C.int2_case(512, 2048, 64, seed=32, dt="fp16")
    q, s, z = C.u8(c["q"], dev), C.to_torch(c["s"], "fp16", dev), C.to_torch(c["z"], "fp16", dev)
    x, x2 = _x(dev, M, 2048, 3), _x(dev, 4, 2048, 4)
    _replay_check(lambda: ops.linear_w2(x, q, 64, (s, z)),
                  lambda: (ops.linear_w2(x2, q, 64, (s, z)), x2.float().sum()))


@pytest.mark.parametrize("M", [1, 64])
def test_graph_linear_w8(dev, M):
    from infinitemodel_amd import ops
    c = C.int8_case(768, 1024, seed=33)
    q, s = C.u8(c["q"], dev), C.to_torch(c["s"], "bf16", dev)
    x, x2 = _x(dev, M, 1024, 5), _x(dev, 3, 1024, 6)
    _replay_check(lambda: ops.linear_w8(x, q, s), lambda: (ops.linear_w8(x2, q, s), x2.float().sum()))


@pytest.mark.parametrize("bits,M", [(4, 1), (4, 3), (4, 16), (4, 600), (2, 2), (2, 8), (8, 1), (8, 8), (8, 600)])
def test_graph_linear_line_tiled(dev, bits, M):
    """The line-tiled entry points under graph replay: line kernels, the K-split kernels with their
    workspace and reduce launch (int4 M 16, int2 M 2..8 on tiled weights), the int8 skinny kernel and
    the prefill GEMMs; each replay equal to the eager call."""
    import torch
    from infinitemodel_amd import ops
    K = 4096
    if bits == 4:
        c = C.int4_case(1024, K, 128, seed=35)
        q, s, z = C.u8(c["q"], dev), C.to_torch(c["s"], "bf16", dev), C.to_torch(c["z"], "bf16", dev)
        t = ops.line_tile(q)
        fn = lambda x: ops.linear_w4_tiled(x, t, 128, (s, z))      # noqa: E731
    elif bits == 2:
        c = C.int2_case(1024, K, 64, seed=36, dt="fp16")
        q, s, z = C.u8(c["q"], dev), C.to_torch(c["s"], "fp16", dev), C.to_torch(c["z"], "fp16", dev)
        t = ops.line_tile(q)
        fn = lambda x: ops.linear_w2_tiled(x, t, 64, (s, z))       # noqa: E731
    else:
        c = C.int8_case(1024, K, seed=37)
        q, s = torch.from_numpy(c["q"].astype(np.int8)).to(dev), C.to_torch(c["s"], "bf16", dev)
        t = ops.line_tile(q)
        fn = lambda x: ops.linear_w8_tiled(x, t, s)                # noqa: E731
    x, x2 = _x(dev, M, K, 7 + M), _x(dev, 5, K, 8)
    _replay_check(lambda: fn(x), lambda: (fn(x2), x2.float().sum()))


def test_graph_dequant_w4(dev):
    from infinitemodel_amd import ops
    c = C.int4_case(256, 1024, 128, seed=34)
    q, s, z = C.u8(c["q"], dev), C.to_torch(c["s"], "bf16", dev), C.to_torch(c["z"], "bf16", dev)
    out = _replay_check(lambda: ops.dequant_w4(q, s, z, 1024, 128), lambda: None)
    assert np.array_equal(C.t2np(out), c["Wd"])


@pytest.mark.parametrize("E,H,I,k,T,act", [
    (32, 512, 256, 4, 1, "silu_glu"),      # decode: the two-launch line path
    (8, 512, 256, 2, 20, "silu_glu"),      # token-sorted line kernels, sort + combine launches
    (4, 512, 256, 2, 400, "silu_glu"),     # grouped GEMM (block list built by the sort)
    (4, 512, 256, 2, 400, "gptoss"),
])
def test_graph_moe_experts(dev, E, H, I, k, T, act):
    import torch
    from infinitemodel_amd import ops
    r = C.rng(35 + T)
    gu = oq.pack_linear_int4_3d(C.bf16_normal(r, (E, 2 * I, H), 0.02), 128, "bf16")
    dn = oq.pack_linear_int4_3d(C.bf16_normal(r, (E, H, I), 0.02), 128, "bf16")
    t = lambda a: C.to_torch(a, "bf16", dev)  # noqa: E731
    gut = (C.u8(gu[0], dev), t(gu[1]), t(gu[2]), H)
    dnt = (C.u8(dn[0], dev), t(dn[1]), t(dn[2]), I)
    kw = {}
    if act == "gptoss":
        kw = dict(act="gptoss", gu_bias=t(C.bf16_normal(r, (E, 2 * I), 0.02)),
                  dn_bias=t(C.bf16_normal(r, (E, H), 0.02)))

    def routed(seed, n):
        idx, w = om.route_topk(C.rng(seed).standard_normal((n, E)).astype(np.float32), k)
        return torch.from_numpy(idx).to(dev), t(w), _x(dev, n, H, seed + 1)

    idx, w, x = routed(36, T)
    idx2, w2, x2 = routed(37, max(1, T // 2))
    _replay_check(lambda: ops.moe_experts_w4(x, idx, w, gut, dnt, 128, **kw),
                  lambda: (ops.moe_experts_w4(x2, idx2, w2, gut, dnt, 128, **kw), x2.float().sum()))


def test_graph_survives_workspace_growth(dev):
    """A graph captured with the cached K-split workspace of its capture stream keeps replaying
    correctly after eager calls on that same stream need a larger workspace: the old buffer is
    retired, never freed, so the graph's baked-in address stays valid and no later allocation can
    land on it."""
    import torch
    from infinitemodel_amd import _lib, ops
    c = C.int4_case(1024, 2048, 128, seed=38)
    q, s, z = C.u8(c["q"], dev), C.to_torch(c["s"], "bf16", dev), C.to_torch(c["z"], "bf16", dev)
    x = _x(dev, 8, 2048, 7)
    g = torch.Generator(device=dev)
    g.manual_seed(39)
    N2, K2 = 8192, 8192
    q2 = torch.randint(0, 256, (N2, K2 // 2), dtype=torch.uint8, device=dev, generator=g)
    s2 = (torch.rand((N2, K2 // 128), device=dev, generator=g) * 0.004 + 0.001).to(torch.bfloat16)
    z2 = torch.randint(0, 16, (N2, K2 // 128), device=dev, generator=g).to(torch.bfloat16)
    x2 = _x(dev, 16, K2, 8)
    L = _lib.lib()
    assert L.imq_linear_workspace_bytes(16, N2, K2) > 4 * L.imq_linear_workspace_bytes(8, 1024, 2048) > 0

    eager = ops.linear_w4(x, q, 128, (s, z)).clone()
    cs = torch.cuda.Stream(dev)
    cs.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(cs):
        ops.linear_w4(x, q, 128, (s, z))           # warm-up: the capture stream's workspace exists
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cs):
        out = ops.linear_w4(x, q, 128, (s, z))
    torch.cuda.synchronize(dev)
    ref2 = None
    for i in range(3):
        with torch.cuda.stream(cs):
            out.zero_()
            graph.replay()
        torch.cuda.synchronize(dev)
        assert torch.equal(out, eager), i
        with torch.cuda.stream(cs):
            y2 = ops.linear_w4(x2, q2, 128, (s2, z2))   # grows this stream's workspace
            junk = torch.full((1 << 22,), 7.0, device=dev)
            junk.add_(1.0)
        torch.cuda.synchronize(dev)
        if ref2 is None:
            ref2 = y2.clone()
        assert torch.equal(y2, ref2), i
