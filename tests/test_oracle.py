"""Pins of the CPU oracle (oracle/quant.py, oracle/moe.py) by checks that do not restate it:
hand-derived known-answer vectors, torch's own bf16/fp16 arithmetic, torch's tinygemm int4
consumer, and transformers' OlmoeExperts / OlmoeTopKRouter. Each check is chosen so that a
plausible oracle mistake (swapped nibbles, min/max before padding, fp32 instead of in-dtype
int8 arithmetic, dropped rounding, gate/up order) fails it.
"""
import numpy as np
import pytest

from oracle import moe as om
from oracle import quant as oq
from tests import _cases as C


# --------------------------------------------------------------------------------------------
# bf16 rounding emulation
# --------------------------------------------------------------------------------------------
def test_bf16_rne_known_answers():
    f = lambda bits: np.array([bits], np.uint32).view(np.float32)
    assert oq.f32_to_bf16_bits(f(0x3F808000))[0] == 0x3F80      # 1 + 2^-8: tie -> even (down)
    assert oq.f32_to_bf16_bits(f(0x3F818000))[0] == 0x3F82      # 1 + 3*2^-8: tie -> even (up)
    assert oq.f32_to_bf16_bits(f(0x3F808001))[0] == 0x3F81      # just above the tie
    assert oq.f32_to_bf16_bits(np.float32([-2.5]))[0] == 0xC020
    assert oq.f32_to_bf16_bits(f(0x7F7FFFFF))[0] == 0x7F80      # FLT_MAX rounds to +inf
    assert np.isnan(oq.round_to(np.float32([np.nan]), "bf16")[0])


def test_bf16_rounding_matches_torch():
    import torch
    hi = np.arange(0, 1 << 16, dtype=np.uint32)
    hi = hi[(hi & 0x7F80) != 0x7F80]                           # finite high halves
    lows = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF], np.uint32)
    bits = ((hi[:, None] << 16) | lows[None, :]).ravel()
    x = bits.view(np.float32)
    t = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oq.f32_to_bf16_bits(x), t)


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
def test_dequant_rounding_matches_torch_arithmetic(dt):
    """Exhaustive (q, z) x sampled scales (and non-integer zeros): the oracle's two-rounding
    dequant equals torch's own (qf - z.to(dt)) * s.to(dt) in dtype dt."""
    import torch
    tdt = {"bf16": torch.bfloat16, "fp16": torch.float16}[dt]
    r = C.rng(7)
    N = 256
    zs = np.concatenate([np.arange(16, dtype=np.float32), r.uniform(0, 15, 16).astype(np.float32)])
    s = oq.round_to(r.uniform(1e-4, 0.1, size=(N, 1)).astype(np.float32), dt)
    codes = np.tile(np.arange(16, dtype=np.uint8), (N, 8))                    # 128 codes / row
    q = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    for zv in zs:
        z = oq.round_to(np.full((N, 1), zv, np.float32), dt)
        ours = oq.dequant_int4(q, s, z, 128, 128, dt)
        qf = torch.from_numpy(codes.astype(np.int16)).to(tdt)
        ref = ((qf - torch.from_numpy(z).to(tdt)) * torch.from_numpy(s).to(tdt)).float().numpy()
        assert np.array_equal(ours, ref), zv


# --------------------------------------------------------------------------------------------
# packed layouts and RTN packers
# --------------------------------------------------------------------------------------------
def test_int4_layout_known_bytes():
    """W = (c - 8) / 16 for a ramp c gives scale 1/16, zero 8, codes c exactly; the packed bytes
    are written out by hand: low nibble = even column (shard_compile.py:93)."""
    c = np.array(list(range(16)) + list(range(15, -1, -1)) + [0] * 96, np.float32)
    W = ((c - 8.0) / 16.0).reshape(1, 128).astype(np.float32)
    q, s, z, in_f = oq.pack_linear_int4(W, 128, "bf16")
    assert s[0, 0] == np.float32(0.0625) and z[0, 0] == 8.0 and in_f == 128
    expect = [0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE,
              0xEF, 0xCD, 0xAB, 0x89, 0x67, 0x45, 0x23, 0x01] + [0x00] * 48
    assert q.tolist() == [expect]
    assert oq.unpack_int4(q)[0, :32].tolist() == c[:32].astype(int).tolist()


def test_int2_layout_known_bytes():
    """W = (c - 2) / 4 for codes c in 0..3 -> scale 0.25, zero 2; crumb i of byte j = column 4j+i."""
    c = np.array([0, 1, 2, 3, 3, 2, 1, 0] + [0, 3] * 28, np.float32)
    W = ((c - 2.0) / 4.0).reshape(1, 64)
    q, s, z, _ = oq.pack_linear_int2(W, 64, "bf16")
    assert s[0, 0] == np.float32(0.25) and z[0, 0] == 2.0
    assert q[0, :2].tolist() == [0xE4, 0x1B]                   # 0b11_10_01_00, 0b00_01_10_11
    assert q[0, 2] == 0b11001100                                # codes 0,3,0,3


def test_nibble_and_crumb_roundtrip_all_bytes():
    b = np.arange(256, dtype=np.uint8).reshape(1, 256)
    c4 = oq.unpack_int4(b).reshape(256, 2)
    assert np.array_equal(c4[:, 0] | (c4[:, 1] << 4), b[0])
    c2 = oq.unpack_int2(b).reshape(256, 4)
    assert np.array_equal(c2[:, 0] | (c2[:, 1] << 2) | (c2[:, 2] << 4) | (c2[:, 3] << 6), b[0])


def test_rtn_constant_group_quirk():
    """A constant group has max-min = 0 -> scale = clamp(0, 1e-8) = 1e-8, zero = clamp(round(-c/1e-8))
    and the codes saturate: the reference dequantizes c > 0 to 15 * bf16(1e-8), not c."""
    W = np.full((3, 128), 0.0, np.float32)
    W[0] = 0.30078125          # bf16 value
    W[1] = -0.30078125
    q, s, z, _ = oq.pack_linear_int4(W, 128, "bf16")
    e8 = oq.round_to(np.float32(1e-8), "bf16")
    assert np.all(s == e8)
    assert z[:, 0].tolist() == [0.0, 15.0, 0.0]
    assert np.all(q[0] == 0xFF) and np.all(q[1] == 0x00) and np.all(q[2] == 0x00)
    d = oq.dequant_int4(q, s, z, 128, 128, "bf16")
    assert np.all(d[0] == oq.round_to(np.float32(15.0) * e8, "bf16"))
    assert np.all(d[1] == oq.round_to(np.float32(-15.0) * e8, "bf16"))


def test_rtn_padding_participates_in_minmax():
    """in_features=100 < G: the zero pad is in the group before min/max (shard_compile.py:80-84),
    so a constant positive row gets wmin = 0 -> scale = c/15, zero 0, codes 15 (no quirk)."""
    W = np.full((1, 100), 0.9375, np.float32)
    q, s, z, in_f = oq.pack_linear_int4(W, 128, "bf16")
    assert in_f == 100 and q.shape == (1, 64)
    assert s[0, 0] == np.float32(0.0625) and z[0, 0] == 0.0
    assert np.all(q[0, :50] == 0xFF) and np.all(q[0, 50:] == 0x00)
    assert np.all(oq.dequant_int4(q, s, z, 100, 128, "bf16") == np.float32(0.9375))


@pytest.mark.parametrize("bits,G", [(4, 128), (2, 64), (4, 32)])
def test_rtn_invariants(bits, G):
    r = C.rng(bits * 100 + G)
    W = C.bf16_normal(r, (64, 3 * G + 17), 0.02)
    pack = oq.pack_linear_int4 if bits == 4 else oq.pack_linear_int2
    deq = oq.dequant_int4 if bits == 4 else oq.dequant_int2
    q, s, z, in_f = pack(W, G, "bf16")
    qmax = (1 << bits) - 1
    codes = (oq.unpack_int4 if bits == 4 else oq.unpack_int2)(q)
    assert codes.max() <= qmax and z.min() >= 0 and z.max() <= qmax and np.all(z == np.rint(z))
    d32 = deq(q, s, z, in_f, G, "fp32")
    ng = s.shape[1]
    Wp = np.zeros((64, ng * G), np.float32)
    Wp[:, :in_f] = W
    # with wmin <= 0 <= wmax every value is within half a (bf16-rounded) step of its code
    err = np.abs(Wp[:, :in_f] - d32)
    bound = np.repeat(s, G, axis=1)[:, :in_f] * (0.5 + 16 * 2.0 ** -9) + 1e-7   # + |q-z| * bf16(s) error
    assert np.all(err <= bound)


def test_int8_known_answers():
    """in-dtype (bf16) arithmetic: scale = bf16(1/127); 0.99609375/scale = 126.51 rounds via bf16
    126.5 to 126 (fp32 arithmetic would give 127); an all-zero row gets bf16(1e-8) and zeros."""
    W = np.zeros((2, 4), np.float32)
    W[0] = [1.0, 0.99609375, -0.5, 0.0]
    q, s = oq.pack_linear_int8(W, "bf16")
    assert s[0, 0] == np.float32(0.00787353515625)
    assert q[0].tolist() == [127, 126, -64, 0]
    assert s[1, 0] == oq.round_to(np.float32(1e-8), "bf16") and q[1].tolist() == [0, 0, 0, 0]


def test_int8_invariants():
    for dt in ("bf16", "fp16"):
        W = C.bf16_normal(C.rng(3), (128, 999), 0.05, dt)
        q, s = oq.pack_linear_int8(W, dt)
        assert np.abs(q.astype(int)).max() <= 127
        amax_pos = np.abs(W).argmax(axis=1)
        assert np.all(np.abs(q[np.arange(128), amax_pos].astype(int)) >= 126)
        # |W/s - q| <= 1/2 + the in-dtype rounding of W/s (<= 2^-8 relative)
        assert np.all(np.abs(W - q * s) <= s * 0.5 + np.abs(W) * 2.0 ** -8 + 1e-7)


def test_int8_dequant_promotion():
    q = np.array([[1, -2]], np.int8)
    s = oq.round_to(np.float32([[0.1]]), "fp16")
    w, res = oq.dequant_int8(q, s, "fp16", "bf16")
    assert res == "fp32" and w.tolist() == [[float(s[0, 0]), float(-2 * s[0, 0])]]
    w2, res2 = oq.dequant_int8(q, s, "fp16", "fp16")
    assert res2 == "fp16"


# --------------------------------------------------------------------------------------------
# dequantize-then-matmul vs an independent int4 consumer (torch tinygemm, CPU)
# --------------------------------------------------------------------------------------------
def _tinygemm(c, x):
    import torch
    from oracle import cpu_path
    q = torch.from_numpy(c["q"])
    s = torch.from_numpy(c["s"]).to(torch.bfloat16)
    z = torch.from_numpy(c["z"]).to(torch.bfloat16)
    mat2, sz = cpu_path.tinygemm_prepare(q, s, z, c["G"])
    return cpu_path.tinygemm_linear(torch.from_numpy(x).to(torch.bfloat16), mat2, c["G"], sz).float().numpy()


def test_linear_ref_matches_tinygemm():
    c = C.int4_case(512, 1024, 128, seed=42)
    x = C.bf16_normal(C.rng(43), (4, 1024))
    ref = oq.linear_ref(x, c["Wd"])
    tg = _tinygemm(c, x)
    assert oq.max_rel(tg, ref) < 1e-2 and oq.mean_rel(tg, ref) < 5e-3


def test_linear_ref_tinygemm_negative_control():
    """Swapping the nibble order in the oracle's view of the weight must break the agreement."""
    c = C.int4_case(256, 512, 128, seed=44)
    x = C.bf16_normal(C.rng(45), (2, 512))
    swapped = ((c["q"] >> 4) | (c["q"] << 4)).astype(np.uint8)
    bad = oq.dequant_int4(swapped, c["s"], c["z"], c["in_f"], 128, "bf16")
    assert oq.max_rel(_tinygemm(c, x), oq.linear_ref(x, bad)) > 0.2


def test_linear_ref_one_hot():
    c = C.int4_case(32, 256, 128, seed=46)
    x = np.zeros((1, 256), np.float32)
    x[0, 77] = 1.0
    assert np.array_equal(oq.linear_ref(x, c["Wd"])[0], c["Wd"][:, 77].astype(np.float64))


# --------------------------------------------------------------------------------------------
# MoE semantics vs transformers' OlmoeExperts / OlmoeTopKRouter
# --------------------------------------------------------------------------------------------
def _olmoe_cfg(E, H, I, k):
    from transformers import OlmoeConfig
    cfg = OlmoeConfig(hidden_size=H, intermediate_size=I, num_experts=E, num_experts_per_tok=k,
                      hidden_act="silu", norm_topk_prob=True, num_hidden_layers=1,
                      num_attention_heads=4, num_key_value_heads=4)
    cfg._experts_implementation = "eager"
    return cfg


def _moe_case(E=8, H=256, I=128, k=2, T=5, seed=50):
    r = C.rng(seed)
    Wg = C.bf16_normal(r, (E, 2 * I, H), 0.02)
    Wd = C.bf16_normal(r, (E, H, I), 0.02)
    gq, gs, gz, _, _ = oq.pack_linear_int4_3d(Wg, 128, "bf16")
    dq, ds, dz, _, _ = oq.pack_linear_int4_3d(Wd, 128, "bf16")
    Wgd = np.stack([oq.dequant_int4(gq[e], gs[e], gz[e], H, 128, "bf16") for e in range(E)])
    Wdd = np.stack([oq.dequant_int4(dq[e], ds[e], dz[e], I, 128, "bf16") for e in range(E)])
    x = C.bf16_normal(r, (T, H))
    idx, w = om.route_topk(r.standard_normal((T, E)).astype(np.float32), k)
    return x, idx, w, Wgd, Wdd


def test_moe_eager_matches_transformers_olmoe_experts():
    import torch
    from transformers.models.olmoe.modeling_olmoe import OlmoeExperts
    E, H, I, k = 8, 256, 128, 2
    x, idx, w, Wgd, Wdd = _moe_case(E, H, I, k)
    mod = OlmoeExperts(_olmoe_cfg(E, H, I, k)).to(torch.bfloat16)
    with torch.no_grad():
        mod.gate_up_proj.copy_(torch.from_numpy(Wgd).to(torch.bfloat16))
        mod.down_proj.copy_(torch.from_numpy(Wdd).to(torch.bfloat16))
        ref = mod(torch.from_numpy(x).to(torch.bfloat16), torch.from_numpy(idx),
                  torch.from_numpy(w).to(torch.bfloat16)).float().numpy()
    ours = om.moe_eager_bf16(x, idx, w, Wgd, Wdd)
    assert oq.max_rel(ours, ref) < 1e-2 and oq.mean_rel(ours, ref) < 3e-3
    exact = om.moe_exact(x, idx, w, Wgd, Wdd)
    assert oq.max_rel(exact, ref) < 2e-2
    # negative control: up/gate swapped must not match
    swapped = np.concatenate([Wgd[:, I:], Wgd[:, :I]], axis=1)
    assert oq.max_rel(om.moe_exact(x, idx, w, swapped, Wdd), ref) > 0.2


def test_route_topk_matches_transformers_router():
    import torch
    from transformers.models.olmoe.modeling_olmoe import OlmoeTopKRouter
    E, k, T = 16, 4, 9
    cfg = _olmoe_cfg(E, E, 32, k)
    r = C.rng(60)
    logits = r.standard_normal((T, E)).astype(np.float32)
    router = OlmoeTopKRouter(cfg)
    with torch.no_grad():
        router.weight.copy_(torch.eye(E))
        _, scores, ridx = router(torch.from_numpy(logits))
    idx, w = om.route_topk(logits, k, out_dt="fp32")
    assert np.array_equal(np.sort(idx, axis=1), np.sort(ridx.numpy(), axis=1))
    np.testing.assert_allclose(np.sort(w, axis=1), np.sort(scores.float().numpy(), axis=1), rtol=2e-6, atol=1e-7)


def test_moe_single_token_brute_force():
    E, H, I, k = 4, 128, 128, 2
    x, idx, w, Wgd, Wdd = _moe_case(E, H, I, k, T=1, seed=61)
    out = om.moe_exact(x, idx, w, Wgd, Wdd)
    acc = np.zeros(H)
    for j in range(k):
        e = idx[0, j]
        g = Wgd[e].astype(np.float64) @ x[0]
        h = g[:I] / (1 + np.exp(-g[:I])) * g[I:]
        acc += float(w[0, j]) * (Wdd[e].astype(np.float64) @ h)
    np.testing.assert_allclose(out[0], acc, rtol=1e-12, atol=1e-12)


def test_moe_exact_grouped_matches_per_token_loop():
    """The grouped evaluation (used by the GPU tests at large T) is the per-token float64 sum."""
    r = np.random.default_rng(5)
    E, H, I, k, T = 6, 32, 16, 3, 11
    Wgu = r.standard_normal((E, 2 * I, H)).astype(np.float32) * 0.1
    Wdn = r.standard_normal((E, H, I)).astype(np.float32) * 0.1
    x = r.standard_normal((T, H)).astype(np.float32)
    idx, w = om.route_topk(r.standard_normal((T, E)).astype(np.float32), k)
    a = om.moe_exact(x, idx, w, Wgu, Wdn)
    b = om.moe_exact_grouped(x, idx, w, Wgu, Wdn)
    assert np.allclose(a, b, rtol=1e-12, atol=1e-12)
    # negative control: dropping one slot's contribution is visible
    w2 = np.array(w, copy=True)
    w2[0, 0] = 0
    assert not np.allclose(om.moe_exact_grouped(x, idx, w2, Wgu, Wdn), a, rtol=1e-6, atol=1e-9)


# --------------------------------------------------------------------------------------------
# gpt-oss experts vs transformers' GptOssExperts
# --------------------------------------------------------------------------------------------
def _gptoss_case(E=6, H=64, I=48, k=2, T=7, seed=70, wscale=0.3):
    r = np.random.default_rng(seed)
    Wgu = r.standard_normal((E, 2 * I, H)) * wscale / np.sqrt(H)     # transpose-packed [E, 2I, H]
    Wdn = r.standard_normal((E, H, I)) * 0.2 / np.sqrt(I)
    bgu = r.standard_normal((E, 2 * I)) * 0.5
    bdn = r.standard_normal((E, H)) * 0.5
    x = r.standard_normal((T, H)) * 2.0
    idx, w = om.route_topk(r.standard_normal((T, E)).astype(np.float32), k, out_dt="fp32")
    return x, idx, w.astype(np.float64), Wgu, bgu, Wdn, bdn


def _gptoss_module(E, H, I, k, Wgu, bgu, Wdn, bdn):
    import torch
    from transformers import GptOssConfig
    from transformers.models.gpt_oss.modeling_gpt_oss import GptOssExperts
    cfg = GptOssConfig(hidden_size=H, intermediate_size=I, num_local_experts=E, num_experts_per_tok=k,
                       num_hidden_layers=1, num_attention_heads=4, num_key_value_heads=4, head_dim=16)
    mod = GptOssExperts(cfg).to(torch.float64)
    with torch.no_grad():
        mod.gate_up_proj.copy_(torch.from_numpy(np.ascontiguousarray(Wgu.transpose(0, 2, 1))))   # in-major
        mod.gate_up_proj_bias.copy_(torch.from_numpy(bgu))
        mod.down_proj.copy_(torch.from_numpy(np.ascontiguousarray(Wdn.transpose(0, 2, 1))))
        mod.down_proj_bias.copy_(torch.from_numpy(bdn))
    return mod


@pytest.mark.parametrize("wscale", [0.3, 6.0])
def test_gptoss_exact_matches_transformers_gptoss_experts(wscale):
    """float64 agreement with a live GptOssExperts fed the in-major transpose of the oracle's
    weights; wscale 6 drives gate / up past +-limit so both clamps take part."""
    import torch
    E, H, I, k = 6, 64, 48, 2
    x, idx, w, Wgu, bgu, Wdn, bdn = _gptoss_case(E, H, I, k, wscale=wscale)
    mod = _gptoss_module(E, H, I, k, Wgu, bgu, Wdn, bdn)
    with torch.no_grad():
        ref = mod(torch.from_numpy(x), torch.from_numpy(idx), torch.from_numpy(w)).numpy()
    ours = om.gptoss_exact(x, idx, w, Wgu, bgu, Wdn, bdn, mod.alpha, mod.limit)
    np.testing.assert_allclose(ours, ref, rtol=1e-10, atol=1e-12)
    gu = np.einsum("th,eoh->teo", x, Wgu) + bgu[None]
    clamped = (gu[..., 0::2] > mod.limit).any() and (np.abs(gu[..., 1::2]) > mod.limit).any()
    assert clamped == (wscale > 1)
    # negative controls: gate / up swapped, a dropped bias, and (when active) no clamp
    sw = np.empty_like(Wgu)
    sw[:, 0::2], sw[:, 1::2] = Wgu[:, 1::2], Wgu[:, 0::2]
    bsw = np.empty_like(bgu)
    bsw[:, 0::2], bsw[:, 1::2] = bgu[:, 1::2], bgu[:, 0::2]
    assert oq.max_rel(om.gptoss_exact(x, idx, w, sw, bsw, Wdn, bdn), ref) > 0.05
    assert oq.max_rel(om.gptoss_exact(x, idx, w, Wgu, bgu, Wdn, 0 * bdn), ref) > 0.05
    if clamped:
        assert oq.max_rel(om.gptoss_exact(x, idx, w, Wgu, bgu, Wdn, bdn, limit=1e30), ref) > 0.05


def test_gptoss_glu_hand_cases():
    """(up + 1) * gate * sigmoid(alpha * gate) with gate clamped above at limit and up clamped to
    [-limit, limit], evaluated by hand."""
    a, L = 1.702, 7.0
    sig = lambda v: 1.0 / (1.0 + np.exp(-v))
    cases = [(0.5, 0.25, 1.25 * 0.5 * sig(a * 0.5)), (9.0, 2.0, 3.0 * 7.0 * sig(a * 7.0)),
             (-9.0, 20.0, 8.0 * -9.0 * sig(-a * 9.0)), (1.0, -8.0, -6.0 * 1.0 * sig(a)), (0.0, 3.0, 0.0)]
    for g, u, want in cases:
        assert om.gptoss_glu64(g, u, a, L) == pytest.approx(want, rel=1e-15, abs=1e-300)


# ---------------------------------------------------------------------------------------------
# int8_gemm_ref: the kernel form s * (x @ q.T) (worker_quant.py:977-980, 1019-1020)
# ---------------------------------------------------------------------------------------------
def test_int8_gemm_ref_known_answer():
    """Hand-computed: x = [1, 2], rows q0 = [3, -4] (s 0.5), q1 = [127, -127] (s 2)."""
    x = np.array([[1.0, 2.0]], np.float32)
    q = np.array([[3, -4], [127, -127]], np.int8)
    s = np.array([[0.5], [2.0]], np.float32)
    assert np.array_equal(oq.int8_gemm_ref(x, q, s), np.array([[-2.5, -254.0]]))


@pytest.mark.parametrize("sdt", ["bf16", "fp16"])
def test_int8_gemm_ref_matches_torch_dequant_then_linear(sdt):
    """The scale factored out of K equals torch's dequantize-then-matmul in float64 (the
    reference's naive path, worker_quant.py:411-417, without its final rounding): the weight
    q.double() * s.double() per row, then F.linear. A scale applied per input column instead of
    per output row (wrong axis) must not match."""
    import torch
    import torch.nn.functional as F
    c = C.int8_case(48, 96, seed=21, dt=sdt)
    x = C.bf16_normal(C.rng(22), (5, 96))
    ref = F.linear(torch.from_numpy(x).double(),
                   torch.from_numpy(c["q"]).double() * torch.from_numpy(c["s"]).double()).numpy()
    got = oq.int8_gemm_ref(x, c["q"], c["s"])
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)
    # oracle's own int8 dequant (pinned by the promotion tests) then linear_ref: same product
    Wd, res = oq.dequant_int8(c["q"], c["s"], sdt, "bf16")
    assert np.allclose(oq.linear_ref(x, Wd), got, rtol=1e-12, atol=1e-12) or res != "fp32"
    # negative control: scale broadcast over K instead of N
    x2 = C.bf16_normal(C.rng(23), (5, 48))
    q2 = np.ascontiguousarray(c["q"][:, :48])
    wrong = F.linear(torch.from_numpy(x2).double(),
                     torch.from_numpy(q2).double() * torch.from_numpy(c["s"]).double().reshape(1, -1)).numpy()
    assert not np.allclose(oq.int8_gemm_ref(x2, q2, c["s"]), wrong, rtol=1e-3, atol=1e-6)


# ---------------------------------------------------------------------------------------------
# dequant_exact: un-rounded (q - bf16(z)) * bf16(s) (worker_quant.py:1176-1177, 646-647)
# ---------------------------------------------------------------------------------------------
def test_dequant_exact_known_answer():
    """Codes 15 / 0 with zero 8 and scale 0.1 (bf16(0.1) = 0.10009765625): (15-8)*0.10009765625 and
    (0-8)*0.10009765625, exactly; a non-integer fp16 zero 1.3 is first taken to bf16 (1.296875)."""
    codes = np.array([[15, 0]], np.uint8)
    s = np.array([[0.1]], np.float32)
    z = np.array([[8.0]], np.float32)
    got = oq.dequant_exact(codes, s, z, 2, 2)
    assert np.array_equal(got, np.array([[7 * 0.10009765625, -8 * 0.10009765625]]))
    z2 = np.array([[1.3]], np.float32)
    got2 = oq.dequant_exact(np.array([[3, 1]], np.uint8), s, z2, 2, 2)
    assert np.array_equal(got2, np.array([[(3 - 1.296875) * 0.10009765625, (1 - 1.296875) * 0.10009765625]]))


@pytest.mark.parametrize("bits,G", [(4, 128), (2, 64)])
def test_dequant_exact_matches_torch_and_rounds_to_reference(bits, G):
    """Against torch float64 over torch's own bf16 casts of scale/zero (independent of the oracle's
    bf16 emulation); rounded once to bf16 it is bit-identical to the reference dequant for the
    integer zeros every reference packer writes; the K tail past in_features is dropped."""
    import torch
    mk = C.int4_case if bits == 4 else C.int2_case
    c = mk(40, 2 * G + 24, G, seed=24)
    codes = oq.unpack_int4(c["q"]) if bits == 4 else oq.unpack_int2(c["q"])
    N, Kp = codes.shape
    zt = torch.from_numpy(c["z"]).to(torch.bfloat16).double()
    st = torch.from_numpy(c["s"]).to(torch.bfloat16).double()
    want = ((torch.from_numpy(codes.astype(np.int64)).double().reshape(N, -1, G) - zt[:, :, None])
            * st[:, :, None]).reshape(N, Kp)[:, :c["in_f"]].numpy()
    got = oq.dequant_exact(codes, c["s"], c["z"], G, c["in_f"])
    assert got.shape == (N, c["in_f"]) and np.array_equal(got, want)
    assert np.array_equal(oq.round_to(got.astype(np.float32), "bf16"), c["Wd"])


def test_dequant_exact_non_integer_zero_within_one_rounding():
    """C3's fp16 non-integer zeros: the reference rounds (q - z) before the product; the exact
    form differs from it by at most that one bf16 rounding of (q - z) times s plus the final one."""
    c = C.int2_random_case(32, 256, 64, seed=2000, dt="fp16")
    codes = oq.unpack_int2(c["q"])
    ex = oq.dequant_exact(codes, c["s"], c["z"], 64, 256)
    s_b = np.repeat(oq.round_to(c["s"], "bf16"), 64, axis=1).astype(np.float64)
    err = np.abs(c["Wd"].astype(np.float64) - ex)
    assert (err <= 2.0 ** -8 * 4.0 * s_b + 2.0 ** -9 * np.abs(ex)).all()
    assert (err > 0).any()     # the two roundings are visible (not the integer-zero case)


# ---------------------------------------------------------------------------------------------
# cpu_path helpers (the timed CPU comparator) against the pinned oracle
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("bits,G,dt", [(4, 128, "bf16"), (4, 128, "fp16"), (4, 64, "fp32"), (2, 64, "bf16"),
                                       (2, 64, "fp16")])
def test_cpu_path_dequant_g_is_the_reference_dequant(bits, G, dt):
    import torch
    from oracle import cpu_path as cp
    c = (C.int4_case if bits == 4 else C.int2_case)(24, 3 * G - 8, G, seed=25)
    tdt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[dt]
    w = cp.dequant_g(torch.from_numpy(c["q"]), torch.from_numpy(c["s"]).to(torch.bfloat16),
                     torch.from_numpy(c["z"]).to(torch.bfloat16), c["in_f"], G, tdt, bits)
    ref = (oq.dequant_int4 if bits == 4 else oq.dequant_int2)(c["q"], c["s"], c["z"], c["in_f"], G, dt)
    assert w.dtype == tdt and np.array_equal(w.float().numpy(), ref)


@pytest.mark.parametrize("rows", [1, 15, 16, 40])
def test_cpu_path_naive_linear_rows_rule(rows):
    """rows < 16: bf16 F.linear over the bf16 dequant; rows >= 16: fp32 dequant + fp32 GEMM, then
    bf16 (worker_quant.py:847-853). Each within one bf16 rounding (+ fp32 accumulation) of the
    exact product over its own dequant: the bf16 dequant below 16 rows, the un-rounded fp32
    dequant ``(q - z) * s`` from 16 rows."""
    import torch
    from oracle import cpu_path as cp
    c = C.int4_case(64, 256, 128, seed=26)
    x = C.bf16_normal(C.rng(27), (rows, 256))
    y = cp.naive_linear(torch.from_numpy(x).to(torch.bfloat16), torch.from_numpy(c["q"]),
                        torch.from_numpy(c["s"]).to(torch.bfloat16), torch.from_numpy(c["z"]).to(torch.bfloat16),
                        c["in_f"], 128, 4)
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (rows, 64)
    Wd = c["Wd"] if rows < 16 else oq.dequant_int4(c["q"], c["s"], c["z"], c["in_f"], 128, "fp32")
    assert oq.max_rel(y.float().numpy(), oq.linear_ref(x, Wd)) <= 2.0 ** -8 + 1e-6


@pytest.mark.parametrize("rows,sdt", [(2, "bf16"), (16, "fp16"), (24, "bf16")])
def test_cpu_path_naive_linear_int8(rows, sdt):
    import torch
    from oracle import cpu_path as cp
    c = C.int8_case(32, 128, seed=28, dt=sdt)
    x = C.bf16_normal(C.rng(29), (rows, 128))
    tdt = torch.bfloat16 if sdt == "bf16" else torch.float16
    y = cp.naive_linear_int8(torch.from_numpy(x).to(torch.bfloat16), torch.from_numpy(c["q"]),
                             torch.from_numpy(c["s"]).to(tdt))
    assert y.dtype == torch.bfloat16
    assert oq.max_rel(y.float().numpy(), oq.int8_gemm_ref(x, c["q"], c["s"])) <= 2.0 ** -7


def test_cpu_path_moe_eager_matches_oracle_loop():
    """The torch eager experts loop against the oracle's bf16 eager loop (pinned against
    transformers' OlmoeExperts) and the exact MoE."""
    import torch
    from oracle import cpu_path as cp
    E, H, I, k, T, G = 8, 256, 128, 2, 6, 128
    r = C.rng(30)
    gu = oq.pack_linear_int4_3d(C.bf16_normal(r, (E, 2 * I, H), 0.02), G, "bf16")
    dn = oq.pack_linear_int4_3d(C.bf16_normal(r, (E, H, I), 0.02), G, "bf16")
    Dgu = np.stack([oq.dequant_int4_3d(gu[0], gu[1], gu[2], e, H, G) for e in range(E)])
    Ddn = np.stack([oq.dequant_int4_3d(dn[0], dn[1], dn[2], e, I, G) for e in range(E)])
    idx, w = om.route_topk(r.standard_normal((T, E)).astype(np.float32), k)
    x = C.bf16_normal(r, (T, H))
    b = lambda a: torch.from_numpy(a).to(torch.bfloat16)  # noqa: E731
    y = cp.moe_eager_cpu(b(x), torch.from_numpy(idx), b(w), (torch.from_numpy(gu[0]), b(gu[1]), b(gu[2]), H),
                         (torch.from_numpy(dn[0]), b(dn[1]), b(dn[2]), I), G).float().numpy()
    assert oq.max_rel(y, om.moe_eager_bf16(x, idx, w, Dgu, Ddn)) <= 2e-2
    assert oq.max_rel(y, om.moe_exact_grouped(x, idx, w, Dgu, Ddn)) <= 3e-2
