"""GPU parity of the fused MoE experts forward (imq_moe_experts_w4) against the oracle's
restatement of the eager experts loop, at the OLMoE shape (BASELINE C5) and small ragged ones.

Tolerance: normwise max relative error <= 1e-2 and mean relative error <= 5e-3 against the exact
(float64, no intermediate rounding) MoE over the bit-exact dequantized experts; against the
reference's bf16 eager loop, the reference's own fused-MoE self-check bounds."""
import functools

import numpy as np
import pytest

from oracle import moe as om
from oracle import quant as oq
from tests import _cases as C

pytestmark = pytest.mark.gpu

MAX_REL = 1e-2
MEAN_REL = 5e-3


@functools.lru_cache(maxsize=2)
def _layer(E, H, I, G, seed):
    r = C.rng(seed)
    Wgu = C.bf16_normal(r, (E, 2 * I, H), 0.02)
    Wdn = C.bf16_normal(r, (E, H, I), 0.02)
    gu = oq.pack_linear_int4_3d(Wgu, G, "bf16")
    dn = oq.pack_linear_int4_3d(Wdn, G, "bf16")
    Dgu = np.stack([oq.dequant_int4_3d(gu[0], gu[1], gu[2], e, H, G) for e in range(E)])
    Ddn = np.stack([oq.dequant_int4_3d(dn[0], dn[1], dn[2], e, I, G) for e in range(E)])
    return gu, dn, Dgu, Ddn


def _run(dev, E, H, I, k, T, seed, G=128, sdt="bf16"):
    import torch
    from infinitemodel_amd import ops
    gu, dn, Dgu, Ddn = _layer(E, H, I, G, seed)
    if sdt != "bf16":
        # stored scale / zero in another dtype; the kernels round them to bf16 like the reference
        gu = (gu[0], oq.round_to(gu[1], sdt), oq.round_to(gu[2], sdt))
        dn = (dn[0], oq.round_to(dn[1], sdt), oq.round_to(dn[2], sdt))
    r = C.rng(seed + 1)
    logits = r.standard_normal((T, E)).astype(np.float32)
    idx, w = om.route_topk(logits, k)
    x = C.bf16_normal(r, (T, H))
    t = lambda a: C.to_torch(a, "bf16", dev)  # noqa: E731
    ts = lambda a: C.to_torch(a, sdt, dev)  # noqa: E731
    out = ops.moe_experts_w4(t(x), torch.from_numpy(idx).to(dev), t(w),
                             (C.u8(gu[0], dev), ts(gu[1]), ts(gu[2]), H),
                             (C.u8(dn[0], dev), ts(dn[1]), ts(dn[2]), I), G)
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == (T, H)
    y = C.t2np(out)
    exact = om.moe_exact_grouped(x, idx, w, Dgu, Ddn)
    assert np.isfinite(y).all()
    mr, me = oq.max_rel(y, exact), oq.mean_rel(y, exact)
    assert mr <= MAX_REL and me <= MEAN_REL, (T, mr, me)
    # against the reference's bf16 eager loop (which itself carries several bf16 roundings per
    # stage and a bf16 index_add): the reference's own fused-MoE self-check bounds,
    # mean rel < 0.03 and max rel < 0.1 (worker_quant.py:2193-2231)
    eager = om.moe_eager_bf16(x, idx, w, Dgu, Ddn)
    assert oq.mean_rel(y, eager) < 0.03 and oq.max_rel(y, eager) < 0.1
    return y


@pytest.mark.parametrize("T", [1, 3, 16])
def test_moe_small(dev, T):
    _run(dev, E=8, H=256, I=128, k=2, T=T, seed=10 + T)


def test_moe_ragged_intermediate(dev):
    """I not a multiple of the group: down's K pads 200 -> 256 and h's pad lanes must be zero."""
    _run(dev, E=5, H=384, I=200, k=3, T=7, seed=3)


@pytest.mark.parametrize("T", [1, 10, 11, 16])
def test_moe_olmoe_shape(dev, T):
    """BASELINE C5: E=64, top-8, H=2048, I=1024. T = 10 (80 routed rows, 1.25 per expert) is the
    last decode-kernel call, T = 11 the first token-sorted one."""
    _run(dev, E=64, H=2048, I=1024, k=8, T=T, seed=3000)


@pytest.mark.parametrize("T,k,E", [(1, 2, 8), (9, 2, 8), (64, 2, 4), (40, 3, 6)])
def test_moe_token_sorted_path(dev, T, k, E):
    """Shapes of the token-sorted grouped path (G 128, H and I_pad multiples of 256, I % 32 == 0):
    a few tokens, and experts with more than 16 routed rows (several MFMA passes); one token runs
    the direct decode kernels."""
    _run(dev, E=E, H=512, I=256, k=k, T=T, seed=40 + T)


def test_moe_token_sorted_h_pad(dev):
    """I = 160 < I_pad = 256: h's pad columns are zeroed before the down projection."""
    _run(dev, E=6, H=512, I=160, k=2, T=9, seed=8)


@pytest.mark.parametrize("sdt", ["fp16", "fp32"])
def test_moe_token_sorted_scale_dtypes(dev, sdt):
    _run(dev, E=4, H=512, I=256, k=2, T=20, seed=9, sdt=sdt)


@pytest.mark.parametrize("T", [64, 256, 384])
def test_moe_olmoe_shape_prefill(dev, T):
    """BASELINE C5 at T = 64 (~8 rows per expert: the token-sorted line kernels), T = 256 (every
    expert hit, ~32 rows each) and T = 384 (~48 rows): the register-B grouped GEMM."""
    _run(dev, E=64, H=2048, I=1024, k=8, T=T, seed=3000)


@pytest.mark.parametrize("T", [1, 16, 300])
def test_moe_int32_and_int64_ids_identical(dev, T):
    """The kernels read the routing ids as int64 (torch's top-k output, as the reference's fused
    op reads them) or int32: the same routing gives bit-identical outputs on every dispatch path
    (T = 1 direct decode, T = 16 token-sorted line kernels, T = 300 the register-B grouped GEMM),
    and the int64 call launches no conversion kernel of its own."""
    import torch
    from infinitemodel_amd import ops
    E, H, I, k, G = 64, 2048, 1024, 8, 128
    gu, dn, _, _ = _layer(E, H, I, G, 3000)
    t = lambda a: C.to_torch(a, "bf16", dev)  # noqa: E731
    r = C.rng(77 + T)
    idx, w = om.route_topk(r.standard_normal((T, E)).astype(np.float32), k)
    x, wt = t(C.bf16_normal(r, (T, H))), t(w)
    a = (C.u8(gu[0], dev), t(gu[1]), t(gu[2]), H)
    b = (C.u8(dn[0], dev), t(dn[1]), t(dn[2]), I)
    i64 = torch.from_numpy(idx).to(dev)
    assert i64.dtype == torch.int64
    y64 = ops.moe_experts_w4(x, i64, wt, a, b, G, check_ids=False)
    y32 = ops.moe_experts_w4(x, i64.to(torch.int32), wt, a, b, G, check_ids=False)
    torch.cuda.synchronize()
    assert torch.equal(y64.view(torch.int16), y32.view(torch.int16)), T


def test_moe_repeat_identical(dev):
    import torch
    from infinitemodel_amd import ops
    E, H, I, G = 8, 256, 128, 128
    gu, dn, _, _ = _layer(E, H, I, G, 5)
    t = lambda a: C.to_torch(a, "bf16", dev)  # noqa: E731
    idx = torch.tensor([[0, 3], [3, 7], [1, 0]], device=dev)
    w = t(np.full((3, 2), 0.5, np.float32))
    x = t(C.bf16_normal(C.rng(2), (3, H)))
    a = (C.u8(gu[0], dev), t(gu[1]), t(gu[2]), H)
    b = (C.u8(dn[0], dev), t(dn[1]), t(dn[2]), I)
    ys = [ops.moe_experts_w4(x, idx, w, a, b, G) for _ in range(3)]
    assert all(torch.equal(ys[0], y) for y in ys[1:])


# ---- gpt-oss experts (imq_moe_experts_w4_ex, act gptoss) ------------------------------------
@functools.lru_cache(maxsize=2)
def _gptoss_layer(E, H, I, seed, bias_std):
    """gpt-oss stores its experts in-major ([E, H, 2I], [E, I, H]); they are transpose-packed."""
    r = C.rng(seed)
    Wgu_in = C.bf16_normal(r, (E, H, 2 * I), 0.02)
    Wdn_in = C.bf16_normal(r, (E, I, H), 0.02)
    bgu = C.bf16_normal(r, (E, 2 * I), bias_std)
    bdn = C.bf16_normal(r, (E, H), 0.02)
    gu = oq.pack_linear_int4_3d(Wgu_in, 128, "bf16", in_major=True)
    dn = oq.pack_linear_int4_3d(Wdn_in, 128, "bf16", in_major=True)
    Dgu = np.stack([oq.dequant_int4_3d(gu[0], gu[1], gu[2], e, H, 128) for e in range(E)])
    Ddn = np.stack([oq.dequant_int4_3d(dn[0], dn[1], dn[2], e, I, 128) for e in range(E)])
    return gu, dn, bgu, bdn, Dgu, Ddn


def _run_gptoss(dev, E, H, I, k, T, seed, bias_std=0.02, pad_to_256=False):
    import torch
    from infinitemodel_amd import ops
    gu, dn, bgu, bdn, Dgu, Ddn = _gptoss_layer(E, H, I, seed, bias_std)
    r = C.rng(seed + 1)
    idx, w = om.route_topk(r.standard_normal((T, E)).astype(np.float32), k)
    x = C.bf16_normal(r, (T, H))
    t = lambda a: C.to_torch(a, "bf16", dev)  # noqa: E731

    def hold(p):
        q, s, z = C.u8(p[0], dev), t(p[1]), t(p[2])
        if pad_to_256 and (q.shape[2] * 2) % 256:
            # the kernel layout of a holder: K padded with zero codes and zero scales
            k2 = -(-q.shape[2] * 2 // 256) * 256
            q2 = torch.zeros((*q.shape[:2], k2 // 2), dtype=torch.uint8, device=dev)
            q2[:, :, :q.shape[2]] = q
            s2 = torch.zeros((*s.shape[:2], k2 // 128), dtype=s.dtype, device=dev)
            z2 = torch.zeros_like(s2)
            s2[:, :, :s.shape[2]], z2[:, :, :z.shape[2]] = s, z
            q, s, z = q2, s2, z2
        return q, s, z

    out = ops.moe_experts_w4(t(x), torch.from_numpy(idx).to(dev), t(w), (*hold(gu), H), (*hold(dn), I), 128,
                             act="gptoss", gu_bias=t(bgu), dn_bias=t(bdn))
    y = C.t2np(out)
    exact = om.gptoss_exact(x, idx, w, Dgu, bgu, Ddn, bdn)
    assert np.isfinite(y).all()
    mr, me = oq.max_rel(y, exact), oq.mean_rel(y, exact)
    assert mr <= MAX_REL and me <= MEAN_REL, (T, mr, me)
    return y, exact


@pytest.mark.parametrize("T", [1, 9, 40])
def test_gptoss_token_sorted(dev, T):
    """Token-sorted path (H, I multiples of 256): interleaved gate / up row pairs, biases."""
    _run_gptoss(dev, E=8, H=512, I=256, k=2, T=T, seed=70 + T)


def test_gptoss_clamps_active(dev):
    """Gate-up biases of std 6 push many gate values above +limit and up values past +-limit."""
    _, exact = _run_gptoss(dev, E=6, H=256, I=128, k=2, T=24, seed=77, bias_std=6.0)
    assert np.isfinite(exact).all()


@pytest.mark.parametrize("pad", [False, True])
def test_gptoss_width_2880(dev, pad):
    """gpt-oss-20b's widths H = I = 2880 (K_pad 2944, 23 groups): the per-row path as packed,
    the token-sorted path once K is padded to 3072 with zero codes and scales."""
    _run_gptoss(dev, E=4, H=2880, I=2880, k=2, T=3, seed=90, pad_to_256=pad)


def test_gptoss_per_row_path(dev):
    """H % 64 != 0 takes the per-row kernels with the gpt-oss activation and biases."""
    _run_gptoss(dev, E=5, H=200, I=96, k=3, T=6, seed=91)


def test_gptoss_module_install(dev):
    """transformers GptOssExperts quantized by _quantize_experts4_ (transpose-pack, dedicated
    forward, kernel layout after placement) against the oracle over its own packed weights."""
    import torch
    from transformers import GptOssConfig
    from transformers.models.gpt_oss.modeling_gpt_oss import GptOssExperts
    from infinitemodel_amd import worker_quant as wq
    E, H, I, k, T = 6, 320, 160, 2, 9
    cfg = GptOssConfig(hidden_size=H, intermediate_size=I, num_local_experts=E, num_experts_per_tok=k,
                       num_hidden_layers=1, num_attention_heads=4, num_key_value_heads=4, head_dim=16)
    mod = GptOssExperts(cfg).to(torch.bfloat16)
    r = C.rng(93)
    with torch.no_grad():
        for p, std in ((mod.gate_up_proj, 0.02), (mod.down_proj, 0.02), (mod.gate_up_proj_bias, 0.5),
                       (mod.down_proj_bias, 0.02)):
            p.copy_(torch.from_numpy(C.bf16_normal(r, tuple(p.shape), std)))
    bgu = mod.gate_up_proj_bias.detach().float().numpy()
    bdn = mod.down_proj_bias.detach().float().numpy()
    wq._quantize_experts4_(mod)
    assert getattr(mod, "_gptoss_fused_installed", False)
    gu, dn = mod.gate_up_proj, mod.down_proj
    Dgu = np.stack([oq.dequant_int4_3d(gu.qweight.numpy(), gu.scale.float().numpy(), gu.zero.float().numpy(),
                                       e, H, 128) for e in range(E)])
    Ddn = np.stack([oq.dequant_int4_3d(dn.qweight.numpy(), dn.scale.float().numpy(), dn.zero.float().numpy(),
                                       e, I, 128) for e in range(E)])
    mod.to(dev)
    wq.finalize_placement(mod)
    assert gu._kernel_tensors()[0].shape[2] * 2 == 512       # K_pad 384 -> kernel layout 512
    idx, w = om.route_topk(r.standard_normal((T, E)).astype(np.float32), k)
    x = C.bf16_normal(r, (T, H))
    with torch.no_grad():
        y = C.t2np(mod(C.to_torch(x, "bf16", dev), torch.from_numpy(idx).to(dev), C.to_torch(w, "bf16", dev)))
    exact = om.gptoss_exact(x, idx, w, Dgu, bgu, Ddn, bdn)
    assert oq.max_rel(y, exact) <= MAX_REL and oq.mean_rel(y, exact) <= MEAN_REL


@pytest.mark.parametrize("kernel_layout", [False, True])
def test_moe_unpadded_hidden_and_pad_codes(dev, kernel_layout):
    """Hidden rows of exactly H columns (H % 8 == 0 < K_pad) give bit-identical results to
    zero-padded rows, on the per-row path (K_pad 384) and the token-sorted path (kernel layout
    512); arbitrary codes in the packed pad columns change nothing (they meet zero activations,
    as in the reference's zero-padded x)."""
    import torch
    from infinitemodel_amd import ops
    E, H, I, k, T, G = 6, 320, 160, 2, 7, 128
    gu, dn, Dgu, Ddn = _layer(E, H, I, G, 17)
    t = lambda a: C.to_torch(a, "bf16", dev)  # noqa: E731

    def hold(p, junk):
        q, s, z = C.u8(p[0], dev).clone(), t(p[1]), t(p[2])
        if kernel_layout:
            k2 = -(-q.shape[2] * 2 // 256) * 256
            q2 = torch.zeros((*q.shape[:2], k2 // 2), dtype=torch.uint8, device=dev)
            q2[:, :, :q.shape[2]] = q
            s2 = torch.zeros((*s.shape[:2], k2 // G), dtype=s.dtype, device=dev)
            z2 = torch.zeros_like(s2)
            s2[:, :, :s.shape[2]], z2[:, :, :z.shape[2]] = s, z
            q, s, z = q2, s2, z2
        if junk is not None:
            q[:, :, junk // 2:] = torch.randint(0, 256, q[:, :, junk // 2:].shape, dtype=torch.uint8,
                                                 generator=torch.Generator(device=dev).manual_seed(5), device=dev)
        return q, s, z

    r = C.rng(18)
    idx, w = om.route_topk(r.standard_normal((T, E)).astype(np.float32), k)
    x = t(C.bf16_normal(r, (T, H)))
    ti = torch.from_numpy(idx).to(dev)
    a = (*hold(gu, None), H)
    b = (*hold(dn, None), I)
    y_un = ops.moe_experts_w4(x, ti, t(w), a, b, G)
    xp = torch.nn.functional.pad(x, (0, a[0].shape[2] * 2 - H))
    y_pad = ops.moe_experts_w4(xp, ti, t(w), a, b, G)
    assert torch.equal(y_un, y_pad)
    y_junk = ops.moe_experts_w4(x, ti, t(w), (*hold(gu, H), H), (*hold(dn, I), I), G)
    assert torch.equal(y_un, y_junk)
    exact = om.moe_exact_grouped(C.t2np(x), idx, w, Dgu, Ddn)
    assert oq.max_rel(C.t2np(y_un), exact) <= MAX_REL


@pytest.mark.parametrize("T,E,k", [(1, 16, 2), (2, 16, 2), (14, 32, 4), (15, 32, 4)])
def test_gptoss_decode_gpt20b_widths(dev, T, E, k):
    """Decode rows at gpt-oss-20b widths in the kernel layout (K 2880 padded to 3072): the
    two-launch line path with unpadded hidden rows and h read as zero past I. At E = 32, top-4,
    T = 14 (56 routed rows, 1.75 per expert) is the last decode-kernel call, T = 15 the first
    token-sorted one."""
    _run_gptoss(dev, E=E, H=2880, I=2880, k=k, T=T, seed=95 + T, pad_to_256=True)


@pytest.mark.parametrize("sdt", ["bf16", "fp16", "fp32"])
def test_moe_decode_line_path(dev, sdt):
    """SiLU-GLU decode through the two-launch line path: one token, 4 of 32 experts, kernel
    layout K (H 320 -> 512), scale / zero dtypes."""
    _run(dev, E=32, H=512, I=256, k=4, T=1, seed=97, sdt=sdt)
    _run(dev, E=32, H=1024, I=512, k=8, T=1, seed=98, sdt=sdt)


class _LazyExact:
    """[E, N, K] view of random-code experts, dequantized exactly per expert on access (only the
    hit experts are ever read by moe_exact_grouped)."""

    def __init__(self, q, s, z, K, G):
        self.q, self.s, self.z, self.K, self.G = q, s, z, K, G
        self.shape = (q.shape[0], q.shape[1], K)

    def __getitem__(self, e):
        return oq.dequant_exact(oq.unpack_int4(self.q[e]), self.s[e], self.z[e], self.G, self.K)


def test_moe_decode_down_over_lds_declines_before_launch(dev):
    """Top-8 decode (4 B <= E: the direct two-launch form) with the down projection's K 3584 at
    H 512: the paired down form would need 16 waves x 4.7 KB > 64 KiB of LDS, so the plan checks
    both launches' LDS before the first and the call runs on the token-sorted path instead of
    launching a gate_up whose down then declines. Random codes (the RTN search at this size would
    take minutes on the host); results against the exact oracle."""
    import torch
    from infinitemodel_amd import ops
    E, H, I, k, T, G = 32, 512, 3584, 8, 1, 128
    r = C.rng(99)
    def experts(N, K):
        q = r.integers(0, 256, size=(E, N, K // 2), dtype=np.uint8)
        s = oq.round_to(r.uniform(0.0005, 0.005, size=(E, N, K // G)).astype(np.float32), "bf16")
        z = r.integers(0, 16, size=(E, N, K // G)).astype(np.float32)
        return q, s, z
    gu, dn = experts(2 * I, H), experts(H, I)
    logits = r.standard_normal((T, E)).astype(np.float32)
    idx, w = om.route_topk(logits, k)
    x = C.bf16_normal(r, (T, H))
    t = lambda a: C.to_torch(a, "bf16", dev)  # noqa: E731
    out = ops.moe_experts_w4(t(x), torch.from_numpy(idx).to(dev), t(w),
                             (C.u8(gu[0], dev), t(gu[1]), t(gu[2]), H),
                             (C.u8(dn[0], dev), t(dn[1]), t(dn[2]), I), G)
    y = C.t2np(out)
    exact = om.moe_exact_grouped(x, idx, w, _LazyExact(*gu, H, G), _LazyExact(*dn, I, G))
    assert np.isfinite(y).all()
    mr, me = oq.max_rel(y, exact), oq.mean_rel(y, exact)
    assert mr <= MAX_REL and me <= MEAN_REL, (mr, me)


@pytest.mark.parametrize("T", [64, 80])
def test_moe_many_rows_per_expert(dev, T):
    """16+ routed rows per expert on average: 32-row blocks with passes of 32 rows (a partial last
    pass at T 80); SiLU-GLU and gpt-oss."""
    _run(dev, E=8, H=512, I=256, k=2, T=T, seed=140 + T)
    _run_gptoss(dev, E=8, H=512, I=256, k=2, T=T, seed=150 + T)


@pytest.mark.parametrize("E,H,I,k,T,sdt", [
    (4, 512, 256, 2, 400, "bf16"),     # ~200 rows per expert: several 64-row blocks, partial last ones
    (4, 512, 192, 2, 330, "bf16"),     # I_pad 256 > I: h's pad columns zeroed before down
    (6, 768, 320, 3, 220, "fp16"),
    (6, 512, 256, 2, 480, "fp32"),
])
def test_moe_grouped_gemm_path(dev, E, H, I, k, T, sdt):
    """Prefill rows ((B / E) * K >= 81920): the grouped dequant-GEMM over 64-row blocks of each hit
    expert, SwiGLU in gate_up's epilogue, the scatter to routed order in down's."""
    _run(dev, E=E, H=H, I=I, k=k, T=T, seed=160 + T, sdt=sdt)


@pytest.mark.parametrize("E,H,I,k,T,bias_std,pad", [
    (4, 512, 256, 2, 330, 0.02, False),
    (6, 256, 128, 2, 960, 6.0, False),      # clamps active
    (4, 2880, 2880, 2, 64, 0.02, True),     # gpt-oss-20b widths, K padded to 3072
])
def test_gptoss_grouped_gemm_path(dev, E, H, I, k, T, bias_std, pad):
    """gpt-oss prefill rows through the grouped GEMM: interleaved (gate, up) columns in adjacent
    lanes of the epilogue, its clamped GLU, both biases."""
    _run_gptoss(dev, E=E, H=H, I=I, k=k, T=T, seed=170 + T, bias_std=bias_std, pad_to_256=pad)


@pytest.mark.parametrize("gpt,E,H,I,k,T", [(True, 4, 2880, 2880, 2, 64), (False, 4, 640, 384, 2, 64)])
def test_grouped_gemm_k_pad_128(dev, gpt, E, H, I, k, T):
    """K_pad a multiple of 128 but not of the line kernels' 256 (gpt-oss-20b's 2944, a 640 x 384
    SiLU layer): the grouped register-B GEMM; at I = 2880 the last gate_up tile holds half a
    group of h columns, the rest of that group reading as zeros in down's group sums."""
    if gpt:
        _run_gptoss(dev, E=E, H=H, I=I, k=k, T=T, seed=185)
    else:
        _run(dev, E=E, H=H, I=I, k=k, T=T, seed=186)


@pytest.mark.parametrize("E,H,I,k,T", [(4, 4608, 256, 2, 24), (4, 512, 4352, 2, 24)])
def test_moe_grouped_gemm_wide_k(dev, E, H, I, k, T):
    """K beyond the line kernels' 4096 (gate_up K 4608, down K 4352): prefill rows take the grouped
    GEMM whatever their number per expert."""
    _run(dev, E=E, H=H, I=I, k=k, T=T, seed=180 + H)


@pytest.mark.parametrize("k,T", [(3, 1), (5, 2), (2, 4)])
def test_moe_decode_slot_pairs(dev, k, T):
    """Decode down with two routed slots per 16-row MFMA tile (8 output rows per workgroup while
    T * H / 8 fits the CUs): odd k leaves the last pair one slot; T 4 at H 1024 takes 16-row tiles."""
    _run(dev, E=64, H=1024 if T == 4 else 512, I=256, k=k, T=T, seed=190 + 10 * k + T)


@pytest.mark.parametrize("bad", [8, -1])
def test_moe_out_of_range_expert_ids_raise(dev, bad):
    """Routing ids outside [0, E) raise ValueError (the reference's eager loop raises in
    one_hot(num_classes=E)) in both MoE ops, before any launch."""
    import torch
    from infinitemodel_amd import ops
    E, H, I, k, G = 8, 256, 128, 2, 128
    gu, dn, _, _ = _layer(E, H, I, G, 77)
    t = lambda a: C.to_torch(a, "bf16", dev)  # noqa: E731
    gut = (C.u8(gu[0], dev), t(gu[1]), t(gu[2]), H)
    dnt = (C.u8(dn[0], dev), t(dn[1]), t(dn[2]), I)
    x = t(C.bf16_normal(C.rng(78), (3, H)))
    idx = torch.tensor([[0, 1], [2, bad], [4, 5]], dtype=torch.int32, device=dev)
    w = torch.full((3, k), 0.5, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="expert ids"):
        ops.moe_experts_w4(x, idx, w, gut, dnt, G)
    with pytest.raises(ValueError, match="expert ids"):
        ops.moe_rows_w4(x[:1].expand(6, H).contiguous(), idx.reshape(-1), gut[0], gut[1], gut[2], G, H)
    ok = ops.moe_experts_w4(x, idx.clamp(0, E - 1), w, gut, dnt, G)
    torch.cuda.synchronize()
    assert torch.isfinite(ok.float()).all()
