"""CPU model of the global-memory address ranges of the int4 skinny GEMV kernel.

The model restates the host dispatch in csrc/gemv.hip (skinny_dispatch / skinny_resident) and
the kernel's per-lane address arithmetic (load_round, the strip loads and the x staging), then
checks that every byte a launch can touch lies inside its buffer, for a matrix of shapes,
scale dtypes, the de-alias padded row view and the exact-fit (no slack) allocation. It guards
against out-of-bounds reads that a generous allocator would hide on the GPU.

The restated launch plans are checked against the compiled dispatcher's own (imq_launch_plan,
host code of libimq.so that needs no device) at the end of the file, so the model cannot drift
from the kernels' real launch shapes unnoticed.
"""
import math

import pytest

STEP = 128


def _dispatch(Kpad, N=16, bf16=True):
    """skinny_dispatch in csrc/gemv.hip."""
    KS = Kpad // STEP
    NT = -(-N // 16)
    if NT >= 1024 and KS >= 16 and (bf16 or -(-KS // 8) <= 8):
        S, W = 8, -(-KS // 8)
    else:
        S, W = 4, -(-KS // 4)
    return KS, S, max(1, min(16, W))


def _strip_ok(G, KS, S, ssg, szb, ssn_elems, base_align=256):
    return G == STEP and KS % S == 0 and ssg == 1 and (ssn_elems * szb) % 16 == 0 and base_align % 16 == 0


def skinny_ranges(N, Kpad, M, G, szb, sqn, ssn, strip_bytes=None, bf16=True):
    """Max exclusive byte offset touched in (qweight, scale, x) for one launch."""
    KS, S, W = _dispatch(Kpad, N, bf16)
    R = -(-KS // (W * S))
    gsh = int(math.log2(G // STEP))
    strip = _strip_ok(G, KS, S, 1, szb, ssn)
    q_hi = s_hi = 0
    for row in range(N):
        for rnd in range(R):
            for wave in range(W):
                sbase = (rnd * W + wave) * S
                for i in range(S):
                    s = min(sbase + i, KS - 1)
                    for jl in range(4):
                        q_hi = max(q_hi, row * sqn + 16 * jl + s * 64 + 16)
                    if not strip:
                        s_hi = max(s_hi, (row * ssn + (s >> gsh)) * szb + szb)
                if strip:
                    g0 = sbase if sbase < KS else 0
                    s_hi = max(s_hi, row * ssn * szb + g0 * szb + (strip_bytes or S * szb))
        if row > 2:      # rows are independent and affine: first rows + last row suffice
            break
    # last row (clamped rows read row N-1)
    row = N - 1
    for rnd in range(R):
        for wave in range(W):
            sbase = (rnd * W + wave) * S
            for i in range(S):
                s = min(sbase + i, KS - 1)
                q_hi = max(q_hi, row * sqn + 48 + s * 64 + 16)
                if not strip:
                    s_hi = max(s_hi, (row * ssn + (s >> gsh)) * szb + szb)
            if strip:
                g0 = sbase if sbase < KS else 0
                s_hi = max(s_hi, row * ssn * szb + g0 * szb + (strip_bytes or S * szb))
    nblk = KS * (STEP // 8)
    x_hi = (M - 1) * Kpad * 2 + (nblk - 1) * 16 + 16
    return q_hi, s_hi, x_hi, strip


SHAPES = [(4096, 4096), (28672, 4096), (28672, 8192), (16384, 4224), (4096, 14336), (6144, 4096), (37, 384), (1000, 256),
          (16, 128), (17, 1152), (2048, 1024), (2048, 2048), (80, 384), (96, 1024), (33, 512)]


@pytest.mark.parametrize("N,K", SHAPES)
@pytest.mark.parametrize("szb", [2, 4])
@pytest.mark.parametrize("pad", [0, 64])
def test_skinny_reads_in_bounds(N, K, szb, pad):
    G = 128
    Kpad = -(-K // G) * G
    ng = Kpad // G
    row_bytes = Kpad // 2
    sqn = row_bytes + pad
    q_bytes = (N - 1) * sqn + row_bytes          # exact fit: the last row has no padding after it
    s_bytes = N * ng * szb
    for M in (1, 4, 16):
        q_hi, s_hi, x_hi, _ = skinny_ranges(N, Kpad, M, G, szb, sqn, ng, bf16=(szb == 2))
        assert q_hi <= q_bytes, (N, K, M, q_hi, q_bytes)
        assert s_hi <= s_bytes, (N, K, M, s_hi, s_bytes)
        assert x_hi <= M * Kpad * 2


@pytest.mark.parametrize("G", [256, 512])
def test_skinny_reads_in_bounds_wide_groups(G):
    for (N, K) in [(64, 1024), (96, 4096)]:
        Kpad = -(-K // G) * G
        ng = Kpad // G
        q_hi, s_hi, _, strip = skinny_ranges(N, Kpad, 1, G, 2, Kpad // 2, ng)
        assert not strip
        assert q_hi <= (N - 1) * (Kpad // 2) + Kpad // 2
        assert s_hi <= N * ng * 2


def test_strip_size_is_exact():
    """The strip load reads exactly S values: S=4 bf16 is an 8-byte load, not 16."""
    for KS, szb in [(4, 2), (8, 2), (16, 2), (32, 4)]:
        _, S, _ = _dispatch(KS * STEP)
        assert S * szb in (8, 16, 32)


def test_model_catches_oversized_strip_load():
    """Negative control: a 16-byte load of an 8-byte strip (S=4, bf16) reads past the last row."""
    N, K = 33, 1024          # 8 groups: 16-byte scale rows, S=4 strips of 8 bytes
    _, s_hi, _, strip = skinny_ranges(N, K, 1, 128, 2, K // 2, K // 128, strip_bytes=16)
    assert strip and s_hi > N * (K // 128) * 2


# ---- prefill GEMM (csrc/gemm.hip): 128 x 128 tiles, K steps of 64 ------------------------------
def gemm_cfg(M, N):
    """launch_gemm in csrc/gemm.hip: (BM, threads) -- 256 x 128 tiles with 512 threads once M
    exceeds 128 rows, else 128 x 128 with 256 threads."""
    return (256, 512) if M > 128 else (128, 256)


def split_plan(T, KT, cus=256):
    """split_plan in csrc/gemm.hip."""
    if 4 * T >= 3 * cus:
        return 1
    s = 1
    while s < 8 and T * s < cus and KT // (2 * s) >= 8:
        s *= 2
    return s


def gemm_ranges(M, N, K, bits, G, sxm, sqn, ssn, sym):
    """Max exclusive offsets read from x (elements), q (bytes), scale (elements) and written to y
    (elements), from the kernel's clamped row indices and per-thread K offsets."""
    BM, NTHR = gemm_cfg(M, N)
    BN = 128
    BK = 64
    WC = BN * BK // NTHR
    KT = K // BK
    tm, tn = -(-M // BM), -(-N // BN)
    x_hi = q_hi = s_hi = y_hi = 0
    for t_m in (0, tm - 1):
        for row in range(BM):
            gm = min(t_m * BM + row, M - 1)
            for c in range(8):
                x_hi = max(x_hi, gm * sxm + c * 8 + (KT - 1) * BK + 8)
    step_bytes = BK * bits // 8
    per_part = WC * bits // 8
    load_bytes = WC * bits // 8
    for t_n in (0, tn - 1):
        for wrow in range(BN):
            gn = min(t_n * BN + wrow, N - 1)
            for part in range(BK // WC):
                q_hi = max(q_hi, gn * sqn + part * per_part + (KT - 1) * step_bytes + load_bytes)
                if bits != 8:
                    g = ((KT - 1) * BK + WC * part) // G
                    s_hi = max(s_hi, gn * ssn + g + 1)
                else:
                    s_hi = max(s_hi, gn * ssn + 1)
    # stores are masked to m < M, n < N
    y_hi = (M - 1) * sym + N
    return x_hi, q_hi, s_hi, y_hi


@pytest.mark.parametrize("M,N,K,bits,G", [(17, 256, 512, 4, 128), (300, 1000, 4096, 4, 128), (129, 200, 1024, 4, 64),
                                          (40, 1792, 2048, 2, 64), (512, 1000, 1024, 8, 0), (2048, 14336, 4096, 4, 128),
                                          (512, 4096, 14336, 8, 0), (100, 96, 448, 2, 64)])
@pytest.mark.parametrize("pad", [0, 64])
def test_gemm_reads_in_bounds(M, N, K, bits, G, pad):
    if K % 64:
        pytest.skip("K not a multiple of 64 goes to the generic kernel")
    row_bytes = K * bits // 8
    sqn = row_bytes + pad
    ng = K // G if G else 1
    x_hi, q_hi, s_hi, y_hi = gemm_ranges(M, N, K, bits, G, K, sqn, ng, N)
    assert x_hi <= M * K
    assert q_hi <= (N - 1) * sqn + row_bytes
    assert s_hi <= N * ng
    assert y_hi <= M * N


def test_gemm_model_catches_unclamped_rows():
    """Negative control: without the row clamp the last tile would read past x."""
    M, K = 130, 256
    rows_unclamped = (-(-M // 128)) * 128
    assert (rows_unclamped - 1) * K + K > M * K


# ---- int2 decode kernel (csrc/gemv.hip w2_skinny_kernel / w2_dispatch) ------------------------
def w2_plan(M, Kpad, max_lds=160 * 1024, bf16=False):
    """w2_dispatch: (S, W, chunk steps, LDS bytes) or None when nothing fits."""
    KS = Kpad // 64
    S = 8 if (not bf16 and -(-KS // 16) > 8) else 16
    W = max(1, min(16, -(-KS // S)))
    need = lambda cs: M * (cs * 64 + 8) * 2 + cs * 64 + 2 * W * 256 * 4  # noqa: E731
    cs = KS
    if need(cs) > max_lds:
        cs = (-(-KS // (W * S))) * W * S
        while cs > W * S and need(cs) > max_lds:
            cs -= W * S
        while cs > S and need(cs) > max_lds:
            cs -= S
        if need(cs) > max_lds:
            return None
    return S, W, cs, need(cs)


@pytest.mark.parametrize("N,K", [(28672, 8192), (8192, 28672), (512, 1024), (96, 448), (1792, 2048)])
@pytest.mark.parametrize("M", [1, 4, 8, 16])
@pytest.mark.parametrize("szb", [2, 4])
def test_w2_reads_in_bounds(N, K, M, szb):
    G = 64
    Kpad = -(-K // G) * G
    if (Kpad // 64) % 4:
        pytest.skip("K_pad not a multiple of 256 codes: the generic kernel serves it")
    plan = w2_plan(M, Kpad)
    assert plan is not None
    S, W, CS, lds = plan
    KS = Kpad // 64
    assert lds <= 160 * 1024 and (CS % S == 0 or CS == KS)
    ng = Kpad // G
    sqn = Kpad // 4
    strip = KS % S == 0 and CS % S == 0
    q_hi = s_hi = 0
    nchunks = -(-KS // CS)
    for row in (0, N - 1):
        for c in range(nchunks):
            c0, c1 = c * CS, min(KS, (c + 1) * CS)
            R = -(-(c1 - c0) // (W * S))
            for rnd in range(R):
                for wave in range(W):
                    sbase = c0 + (rnd * W + wave) * S
                    for t in range(S // 4):
                        sb4 = min(sbase + 4 * t, c1 - 4)
                        q_hi = max(q_hi, row * sqn + 16 * 3 + 16 * sb4 + 16)
                    for i in range(S):
                        st = min(sbase + i, c1 - 1)
                        if not strip:
                            s_hi = max(s_hi, (row * ng + st) * szb + szb)
                    if strip:
                        g0 = sbase if sbase < c1 else c0
                        s_hi = max(s_hi, (row * ng + g0) * szb + S * szb)
            # staging reads x[m, c0*64 + 16*pr .. +16] for pr < 4*(c1-c0)
            assert c0 * 64 + 16 * (4 * (c1 - c0) - 1) + 16 <= Kpad
    assert q_hi <= (N - 1) * sqn + Kpad // 4
    assert s_hi <= N * ng * szb


# ---- int8 decode kernel (csrc/gemv.hip w8_skinny_kernel / w8_dispatch) ------------------------
def w8_plan(M, K, max_lds=160 * 1024):
    S = 8
    KS = K // 64
    W = max(1, min(16, -(-KS // S)))
    need = lambda cs: M * (cs * 64 + 8) * 2 + cs * 64 + 64 + 2 * W * 256 * 4  # noqa: E731
    cs = KS
    if need(cs) > max_lds:
        cs = (-(-KS // (W * S))) * W * S
        while cs > W * S and need(cs) > max_lds:
            cs -= W * S
        while cs > S and need(cs) > max_lds:
            cs -= S
        if need(cs) > max_lds:
            return None
    return S, W, cs, need(cs)


@pytest.mark.parametrize("N,K", [(14336, 4096), (4096, 14336), (320, 14336), (1000, 4096), (1792, 4096)])
@pytest.mark.parametrize("M", [1, 5, 16])
def test_w8_reads_in_bounds(N, K, M):
    plan = w8_plan(M, K)
    assert plan is not None
    S, W, CS, lds = plan
    KS = K // 64
    assert lds <= 160 * 1024 and (CS % S == 0 or CS == KS)
    q_hi = 0
    for row in (0, N - 1):
        for c in range(-(-KS // CS)):
            c0, c1 = c * CS, min(KS, (c + 1) * CS)
            R = -(-(c1 - c0) // (W * S))
            for rnd in range(R):
                for wave in range(W):
                    sbase = c0 + (rnd * W + wave) * S
                    for i in range(S):
                        st = min(sbase + i, c1 - 1)
                        q_hi = max(q_hi, row * K + 16 * 3 + 64 * st + 16)
            assert c0 * 64 + 8 * (8 * (c1 - c0) - 1) + 8 <= K
    assert q_hi <= N * K


# ---- int4 line kernel (csrc/gemv.hip w4_line_kernel / line_plan) ------------------------------
LINE = 256


def line_plan(M, Kpad, G, N, sqn, sxm, ssn, vb, max_lds=160 * 1024):
    """line_plan in csrc/gemv.hip: (S2, W, LDS bytes) or None when the line kernel declines."""
    if not (1 <= M <= 4) or G != 128 or Kpad % LINE or N < 1:
        return None
    if (ssn * vb) % 4:
        return None
    if 16 * sqn >= 2 ** 31 or M * sxm * 2 >= 2 ** 31 or 16 * ssn * vb >= 2 ** 31:
        return None
    KL = Kpad // LINE
    S2 = 2
    if -(-KL // S2) > 16:
        S2 = 4
    W = -(-KL // S2)
    if W > 16:
        return None
    wave_lds = M * (S2 * LINE + 8) * 2 + 2 * S2 * 16 * 4 + 2 * 16 * S2 * vb // 2 * 4
    rc = M if M <= 2 else 4              # M = 3 runs the 4-row instantiation
    lds = W * wave_lds + W * rc * 16 * 4
    if lds > max_lds:
        return None
    return S2, W, lds


def line_ranges(M, Kpad, N, sqn, sxm, ssn, vb, S2, W, sz_dword=None):
    """Max exclusive byte offsets read from qweight / scale (= zero) / x and written to y, from
    the kernel's per-lane arithmetic with its clamps. sz_dword(ls0, dw) overrides the scale dword
    index (negative controls)."""
    KL = Kpad // LINE
    DPR = S2 * vb // 2
    ngd = Kpad // 128 * vb // 4
    q_hi = s_hi = x_hi = y_hi = 0
    NT = -(-N // 16)
    for tile in sorted({0, NT - 1}):
        row0 = tile * 16
        rlast = N - 1 - row0
        for wave in range(W):
            ls0 = wave * S2
            # x: idx -> (m, b), kb = min(8b, Kpad - ls0*256 - 8), 8 elements
            XB = 32 * S2
            xtot = M * XB
            xlim = Kpad - ls0 * LINE - 8
            for idx in range(xtot):
                m, b = divmod(idx, XB)
                kb = min(8 * b, xlim)
                assert kb >= 0
                x_hi = max(x_hi, (ls0 * LINE + m * sxm + kb + 8) * 2)
            # scale / zero dwords
            for d in range(32 * DPR):
                arr, rem = divmod(d, 16 * DPR)
                r, dw = divmod(rem, DPR)
                r = min(r, rlast)
                gd = sz_dword(ls0, dw) if sz_dword else ls0 * (vb // 2) + dw
                gd = min(gd, ngd - 1)
                s_hi = max(s_hi, (row0 + r) * ssn * vb + 4 * gd + 4)
            # weights: two full-line loads per line-step
            for c in range(16):
                for ar in range(4):
                    lo8 = c < 8
                    rr0 = min(c & 7, rlast)
                    rr1 = min(8 + (c & 7), rlast)
                    for i in range(S2):
                        l = min(ls0 + i, KL - 1)
                        q_hi = max(q_hi, (row0 + rr0) * sqn + 16 * ar + (0 if lo8 else 64) + 128 * l + 16)
                        q_hi = max(q_hi, (row0 + rr1) * sqn + 16 * ar + (64 if lo8 else 0) + 128 * l + 16)
        for n in range(16):
            if n <= rlast:
                y_hi = max(y_hi, row0 + n + 1)
    return q_hi, s_hi, x_hi, y_hi


def line_lds_reads(M, S2):
    """Max exclusive element offsets of a wave's A-operand reads (bf16, in its staged x strip of M
    rows) and group-sum reads (fp32, in its 2 * S2 * 16 sums) for the launched row class: M <= 2
    pairs the two groups of a line-step in A rows [0, M) / [M, 2M); M 3..4 puts group 2l in A rows
    0-3 and group 2l+1 in rows 4-7 (lanes 16-31 read their own group's sums); rows past M repeat an
    existing row."""
    xrow = S2 * LINE + 8
    xa = xs = 0
    for c in range(16):
        for ar in range(4):
            if M <= 2:
                row = c % M if c < 2 * M else 0
                off = 128 if M <= c < 2 * M else 0
                sums = [(2 * i) * 16 + 4 * ar + 4 for i in range(S2)] + [(2 * i + 1) * 16 + 4 * ar + 4 for i in range(S2)]
            else:
                row = (c & 3) if (c & 3) < M else M - 1
                off = 128 if c & 4 else 0
                sums = [(2 * i + (1 if ar == 1 else 0)) * 16 + 4 for i in range(S2)]
            for i in range(S2):
                xa = max(xa, row * xrow + 32 * ar + i * LINE + off + 8 * 3 + 8)
            xs = max(xs, *sums)
    return xa, xs, M * xrow, 2 * S2 * 16


LINE_SHAPES = [(4096, 4096), (6144, 4096), (28672, 4096), (4096, 14336), (37, 512), (100, 768), (17, 256),
               (48, 16384), (1000, 256)]


@pytest.mark.parametrize("N,K", LINE_SHAPES)
@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("vb", [2, 4])
@pytest.mark.parametrize("pad", [0, 64])
def test_line_reads_in_bounds(N, K, M, vb, pad):
    Kpad = K
    ng = Kpad // 128
    sqn = Kpad // 2 + pad
    plan = line_plan(M, Kpad, 128, N, sqn, Kpad, ng, vb)
    assert plan is not None
    S2, W, lds = plan
    assert W * S2 * LINE >= Kpad and (W - 1) * S2 * LINE < Kpad
    assert lds <= 160 * 1024
    q_hi, s_hi, x_hi, y_hi = line_ranges(M, Kpad, N, sqn, Kpad, ng, vb, S2, W)
    # LDS: the reduction area of the launched row class (M = 3 -> 4 rows) lies inside the launch
    rc = M if M <= 2 else 4
    xrow = S2 * LINE + 8
    wave_lds = M * xrow * 2 + 2 * S2 * 16 * 4 + 2 * 16 * S2 * vb // 2 * 4
    assert W * wave_lds + W * rc * 16 * 4 <= lds
    xa, xs, xa_lim, xs_lim = line_lds_reads(M, S2)
    assert xa <= xa_lim and xs <= xs_lim
    assert q_hi <= (N - 1) * sqn + Kpad // 2          # exact fit: no padding after the last row
    assert s_hi <= N * ng * vb
    assert x_hi <= ((M - 1) * Kpad + Kpad) * 2
    assert y_hi <= N


def test_line_plan_declines():
    """Shapes the line kernel leaves to the skinny kernel."""
    assert line_plan(5, 4096, 128, 4096, 2048, 4096, 32, 2) is None      # M > 4
    assert line_plan(1, 4096, 64, 4096, 2048, 4096, 64, 2) is None       # G != 128
    assert line_plan(1, 384, 128, 37, 192, 384, 3, 2) is None            # K_pad % 256
    assert line_plan(1, 16640, 128, 64, 8320, 16640, 130, 2) is None     # K_pad > 16384 (W > 16)
    assert line_plan(1, 16384, 128, 64, 8192, 16384, 128, 2) is not None


def test_line_model_catches_wrong_scale_index():
    """Negative control for the scale dword index: line-steps * dwords-per-row (instead of the
    dwords of one line-step) stays inside the array only because of the in-kernel clamp, and
    then hands every wave but the first the groups of another K range."""
    N, K, M, vb = 64, 4096, 1, 2
    S2, W, _ = line_plan(M, K, 128, N, K // 2, K, K // 128, vb)
    DPR = S2 * vb // 2
    wrong = lambda ls0, dw: ls0 * DPR + dw     # noqa: E731
    # with the clamp to the row the wrong index stays inside the array but reads other groups:
    # compare the group each wave would use for its first line-step
    for wave in range(1, W):
        assert wrong(wave * S2, 0) != wave * S2 * (vb // 2)




# ---- int4 K-split decode kernel (csrc/gemv.hip w4_ksplit_kernel / ksplit_plan) -----------------
KS_S2 = 4


def ksplit_plan(M, Kpad, G, N, sqn, sxm, ssn, vb, max_lds=160 * 1024, cus=256):
    """ksplit_plan in csrc/gemv.hip: (splits, NW, LDS bytes, line-steps per split) or None when
    the K-split kernel declines."""
    if not (4 < M <= 16) or G != 128 or Kpad % LINE or Kpad <= 0 or N < 1:
        return None
    if N % 4 or sxm % 8 or (ssn * vb) % 4:
        return None
    if 16 * sqn >= 2 ** 31 or M * sxm * 2 >= 2 ** 31 or 16 * ssn * vb >= 2 ** 31:
        return None
    splits4 = -(-(Kpad // LINE) // KS_S2)
    nw = 8 if splits4 * -(-N // 128) >= cus else 4
    s2 = 2 if nw == 4 and splits4 * -(-N // 64) <= 2 * cus else KS_S2     # short grids: 512-code splits
    splits = -(-(Kpad // LINE) // s2)
    lds = M * (s2 * LINE + 8) * 2 + 2 * s2 * 16 * 4 + nw * 2 * 16 * (s2 * vb // 2) * 4
    if lds > max_lds:
        return None
    return splits, nw, lds, s2


def ksplit_ranges(M, Kpad, N, sqn, sxm, ssn, vb):
    """Max exclusive offsets the K-split kernel reads (qweight bytes, scale bytes, x elements) and
    writes (partials, LDS x elements / xs floats / s-z dwords), per the kernel's index arithmetic
    and clamps, over the first and last split and row block; plus the set of (split, m, n) partial
    elements written over every workgroup."""
    splits, NW, _, S2 = ksplit_plan(M, Kpad, 128, N, sqn, sxm, ssn, vb)
    MC = 8 if M <= 8 else 16
    NT = 64 * NW
    KL = Kpad // LINE
    RB = -(-N // (16 * NW))
    DPR = S2 * vb // 2
    ngd = Kpad // 128 * vb // 4
    XB = 32 * S2
    XU = -(-(MC * XB) // NT)
    xrow = S2 * LINE + 8
    r = dict(q=0, s=0, x=0, part=0, lds_x=0, lds_xs=0, lds_sz=0, lds_xa=0)
    written = set()
    for split in range(splits):
        ls0 = split * S2
        xlim = Kpad - ls0 * LINE - 8
        for rb in range(RB):
            full = split in (0, splits - 1) and rb in (0, RB - 1)
            if full:
                xtot = M * XB
                for t in range(NT):
                    for u in range(XU):
                        idx = min(t + NT * u, xtot - 1)
                        m, b = divmod(idx, XB)
                        kb = min(8 * b, xlim)
                        assert kb >= 0
                        r["x"] = max(r["x"], ls0 * LINE + m * sxm + kb + 8)
                        if t + NT * u < xtot:
                            r["lds_x"] = max(r["lds_x"], m * xrow + 8 * b + 8)
                            if b % 16 == 0:
                                r["lds_xs"] = max(r["lds_xs"], (b >> 4) * 16 + m + 1)
            for wave in range(NW):
                row0 = (rb * NW + wave) * 16
                tile_ok = row0 < N
                rowa = row0 if tile_ok else 0
                rlast = N - 1 - rowa
                assert rlast >= 0
                if full:
                    for d in range(32 * DPR):
                        arr, rem = divmod(d, 16 * DPR)
                        rr, dw = divmod(rem, DPR)
                        rr = min(rr, rlast)
                        gd = min(ls0 * (vb // 2) + dw, ngd - 1)
                        r["s"] = max(r["s"], (rowa + rr) * ssn * vb + 4 * gd + 4)
                        r["lds_sz"] = max(r["lds_sz"], wave * 2 * 16 * DPR + d + 1)
                    for c in range(16):
                        for ar in range(4):
                            lo8 = c < 8
                            rr0 = min(c & 7, rlast)
                            rr1 = min(8 + (c & 7), rlast)
                            mrow = c if c < M else M - 1
                            for i in range(S2):
                                l = min(ls0 + i, KL - 1)
                                r["q"] = max(r["q"], (rowa + rr0) * sqn + 16 * ar + (0 if lo8 else 64) + 128 * l + 16)
                                r["q"] = max(r["q"], (rowa + rr1) * sqn + 16 * ar + (64 if lo8 else 0) + 128 * l + 16)
                                r["lds_xa"] = max(r["lds_xa"], mrow * xrow + 32 * ar + i * LINE + 128 + 8 * 3 + 8)
                for c in range(16):
                    for ar in range(4):
                        for rr in range(4):
                            m = 4 * ar + rr
                            if tile_ok and m < M and c <= rlast:
                                off = split * M * N + m * N + row0 + c
                                r["part"] = max(r["part"], off + 1)
                                written.add(off)
    return splits, r, written


KS_SHAPES = [(4096, 4096), (6144, 4096), (28672, 4096), (4096, 14336), (36, 768), (100, 1280), (20, 256),
             (80, 512)]


@pytest.mark.parametrize("N,K", KS_SHAPES)
@pytest.mark.parametrize("M", [5, 8, 9, 16])
@pytest.mark.parametrize("vb", [2, 4])
@pytest.mark.parametrize("pad", [0, 64])
def test_ksplit_in_bounds_and_covering(N, K, M, vb, pad):
    """Every K-split read lies inside its operand, every LDS access inside the launch's dynamic
    LDS, the partials stay inside the workspace the host sizes (splits * M * N fp32), and the
    kernel writes every partial element the reduction reads."""
    Kpad = K
    ng = Kpad // 128
    sqn = Kpad // 2 + pad
    plan = ksplit_plan(M, Kpad, 128, N, sqn, Kpad, ng, vb)
    assert plan is not None
    splits, nw, lds, s2 = plan
    if N == 28672:
        assert nw == 8
    if (N, K) in ((4096, 4096), (6144, 4096)):
        assert nw == 4 and s2 == 2                    # short grids: 512-code splits
    assert splits * s2 * LINE >= Kpad and (splits - 1) * s2 * LINE < Kpad
    _, r, written = ksplit_ranges(M, Kpad, N, sqn, Kpad, ng, vb)
    assert r["q"] <= (N - 1) * sqn + Kpad // 2
    assert r["s"] <= N * ng * vb
    assert r["x"] <= (M - 1) * Kpad + Kpad
    assert r["part"] <= splits * M * N
    assert len(written) == splits * M * N            # complete: the reduction reads no stale value
    xrow = s2 * LINE + 8
    x_bytes = M * xrow * 2
    assert r["lds_x"] * 2 <= x_bytes and r["lds_xa"] * 2 <= x_bytes
    assert r["lds_xs"] <= 2 * s2 * 16
    sz_off = x_bytes + 2 * s2 * 16 * 4
    assert sz_off + r["lds_sz"] * 4 <= lds


def test_ksplit_plan_declines():
    assert ksplit_plan(4, 4096, 128, 4096, 2048, 4096, 32, 2) is None     # M <= 4: line kernel
    assert ksplit_plan(17, 4096, 128, 4096, 2048, 4096, 32, 2) is None    # prefill rows
    assert ksplit_plan(8, 4096, 64, 4096, 2048, 4096, 64, 2) is None      # G != 128
    assert ksplit_plan(8, 384, 128, 36, 192, 384, 3, 2) is None           # K_pad % 256
    assert ksplit_plan(8, 512, 128, 37, 256, 512, 4, 2) is None           # N % 4 (vector reduction)
    assert ksplit_plan(16, 14336, 128, 4096, 7168, 14336, 112, 2) is not None


# ---- int4 wave-split decode kernel (csrc/gemv.hip w4_wsplit_kernel / wsplit_plan) --------------
WS_NW = 8


def wsplit_lds(R, NW=WS_NW):
    """wsplit_lds in csrc/gemv.hip: per-wave activation slices and group sums, the double-buffered
    partials, 8 tiles of buffered bf16 results."""
    return NW * (16 * (R * LINE + 8) * 2 + 2 * R * 16 * 4) + 2 * NW * 256 * 4 + 8 * 256 * 2


def wsplit_plan(M, Kpad, G, N, sqn, sxm, ssn, vb, cus=256, max_lds=160 * 1024):
    """wsplit_plan in csrc/gemv.hip: R (line-steps per wave) or None when the kernel declines."""
    if not (4 < M <= 16) or G != 128 or Kpad not in (WS_NW * LINE, 2 * WS_NW * LINE):
        return None
    if N < 1 or sxm % 8 or (ssn * vb) % 4:
        return None
    if 16 * sqn >= 2 ** 31 or M * sxm * 2 >= 2 ** 31:
        return None
    R = Kpad // (WS_NW * LINE)
    if wsplit_lds(R) > max_lds or -(-N // 16) < cus:
        return None
    return R


def wsplit_ranges(M, Kpad, N, sqn, sxm, ssn, vb, cus=256, clamp=True):
    """Max exclusive offsets the wave-split kernel reads (x elements, qweight bytes, scale
    elements), its wave-private LDS offsets (staged x, A-operand reads, group sums), and the y
    elements it writes (with multiplicity), from its index arithmetic: every lane of every wave
    for the first and last tile of each workgroup (the prefetch past the last tile re-reads it),
    and every tile for y."""
    R = wsplit_plan(M, Kpad, 128, N, sqn, sxm, ssn, vb, cus)
    T = -(-N // 16)
    G = min(T, cus)
    r = dict(x=0, q=0, s=0, red=0, lds_x=0, lds_xa=0, lds_sum=0)
    ywrites = {}
    CPR = 32 * R
    XROW = R * LINE + 8
    for wave in range(WS_NW):
        ls0 = wave * R
        for lane in range(64):
            c, ar = lane & 15, lane >> 4
            for u in range(16 * CPR // 64):
                m, ch = divmod(64 * u + lane, CPR)
                r["x"] = max(r["x"], min(m, M - 1) * sxm + ls0 * LINE + 8 * ch + 8)
                if m < M:
                    r["lds_x"] = max(r["lds_x"], m * XROW + 8 * ch + 8)
                    if ch % 16 == 0:
                        r["lds_sum"] = max(r["lds_sum"], (ch >> 4) * 16 + m + 1)
            row = c if c < M else 0
            for i in range(R):
                for k in range(4):
                    r["lds_xa"] = max(r["lds_xa"], row * XROW + 32 * ar + i * LINE + 128 + 8 * k + 8)
                r["lds_sum"] = max(r["lds_sum"], (2 * i + 1) * 16 + 4 * ar + 4)
    tiles = set()
    for b in range(G):
        ts = list(range(b, T, G))
        tiles.update(ts)
        for t in (ts[0], ts[-1]):
            row0 = t * 16
            rlast = N - 1 - row0
            assert rlast >= 0
            for wave in range(WS_NW):
                ls0 = wave * R
                for lane in range(64):
                    c, ar = lane & 15, lane >> 4
                    lo8 = c < 8
                    rr0 = min(c & 7, rlast) if clamp else c & 7
                    rr1 = min(8 + (c & 7), rlast) if clamp else 8 + (c & 7)
                    rc = min(c, rlast) if clamp else c
                    for i in range(R):
                        r["q"] = max(r["q"], (row0 + rr0) * sqn + ls0 * 128 + 16 * ar + (0 if lo8 else 64) + 128 * i + 16)
                        r["q"] = max(r["q"], (row0 + rr1) * sqn + ls0 * 128 + 16 * ar + (64 if lo8 else 0) + 128 * i + 16)
                    nwords = 2 * R if vb == 4 else R
                    per = 1 if vb == 4 else 2        # scale elements per dword
                    r["s"] = max(r["s"], (row0 + rc) * ssn + 2 * ls0 + nwords * per)
                    for rr in range(4):
                        r["red"] = max(r["red"], (4 * ar + rr) * 16 + c + 1)
    assert tiles == set(range(T))
    for t in range(T):
        for e in range(64 * WS_NW):
            m, col = e >> 4, e & 15
            if e < 256 and m < M and t * 16 + col < N:
                key = (m, t * 16 + col)
                ywrites[key] = ywrites.get(key, 0) + 1
    return R, r, ywrites


@pytest.mark.parametrize("N,K,cus", [(28672, 4096, 256), (16400, 2048, 256), (100, 2048, 1), (68, 4096, 1),
                                     (4100, 2048, 64), (72, 2048, 1), (1000, 4096, 8)])
@pytest.mark.parametrize("M", [5, 9, 16])
@pytest.mark.parametrize("vb", [2, 4])
@pytest.mark.parametrize("pad", [0, 64])
def test_wsplit_in_bounds_and_covering(N, K, cus, M, vb, pad):
    """Every wave-split read lies inside its operand (exact-fit allocations, the +64-byte row
    view), the LDS partials stay inside one wave's 256 floats, the persistent grid visits every
    tile once, and every y element is written exactly once. Small CU counts put short grids,
    partial last tiles and uneven tiles per workgroup under the plan's 4-tiles-per-CU rule."""
    Kpad, ng = K, K // 128
    sqn = Kpad // 2 + pad
    ssn = ng + (pad // 2 if vb == 2 else pad // 4)
    R, r, yw = wsplit_ranges(M, Kpad, N, sqn, Kpad, ssn, vb, cus)
    assert R in (1, 2)
    assert r["x"] <= (M - 1) * Kpad + Kpad
    assert r["q"] <= (N - 1) * sqn + Kpad // 2
    assert r["s"] <= (N - 1) * ssn + ng
    assert r["red"] <= 256
    xrow = R * LINE + 8
    assert r["lds_x"] <= 16 * xrow and r["lds_xa"] <= 16 * xrow and r["lds_sum"] <= 2 * R * 16
    lds = WS_NW * (16 * xrow * 2 + 2 * R * 16 * 4) + 2 * WS_NW * 256 * 4 + 8 * 256 * 2
    assert lds <= 160 * 1024
    assert len(yw) == M * N and set(yw.values()) == {1}


def test_wsplit_model_catches_missing_row_clamp():
    """Negative control: without the row clamps a partial last tile (N % 16) would read weight and
    scale rows past N."""
    N, K, M = 100, 2048, 8
    _, r, _ = wsplit_ranges(M, K, N, K // 2, K, K // 128, 2, cus=1, clamp=False)
    assert r["q"] > (N - 1) * (K // 2) + K // 2 or r["s"] > (N - 1) * (K // 128) + K // 128


def test_wsplit_plan_declines():
    assert wsplit_plan(4, 4096, 128, 4096, 2048, 4096, 32, 2) is None     # M <= 4: line kernel
    assert wsplit_plan(8, 14336, 128, 4096, 7168, 14336, 112, 2) is None  # K_pad not 2048 / 4096
    assert wsplit_plan(8, 4096, 64, 4096, 2048, 4096, 64, 2) is None      # G != 128
    assert wsplit_plan(8, 4096, 128, 4096, 2048, 4096, 33, 2) is None     # odd bf16 scale row stride
    assert wsplit_plan(16, 4096, 128, 2048, 2048, 4096, 32, 2) is None    # < 1 tile per CU: K-split
    assert wsplit_plan(16, 4096, 128, 4096, 2048, 4096, 32, 2) == 2       # o: 1 tile per CU
    assert wsplit_plan(16, 4096, 128, 6144, 2048, 4096, 32, 2) == 2       # qkv: 1.5 tiles per CU
    assert wsplit_plan(16, 4096, 128, 28672, 2048, 4096, 32, 2) == 2      # gate_up: 7 tiles per CU
    assert wsplit_plan(8, 2048, 128, 16384, 1024, 2048, 16, 2) == 1


def test_ksplit_model_catches_missing_row_clamp():
    """Negative control: without the idle-wave clamp (rowa = row0 for every wave), a partial last
    row block would address rows past N."""
    N, K, M = 100, 1024, 8
    _, NW, _, _ = ksplit_plan(M, K, 128, N, K // 2, K, K // 128, 2)
    RB = -(-N // (16 * NW))
    row0 = ((RB - 1) * NW + NW - 1) * 16
    assert row0 >= N and N - 1 - row0 < 0



# ---- int2 line kernel (csrc/gemv.hip w2_line_kernel / line2_plan) -----------------------------
LINE2 = 512


def sz2_row(ngw):
    """Row stride (floats) of the staged (s, -(128 + z) * s) pairs of NGW groups."""
    return 2 * ngw + 2


def sz2_bytes(ngw):
    return 16 * sz2_row(ngw) * 4


def sz2_ranges(r, lds_base, row0, rlast, ssn, szn, vb, ngw, gd0, ngd):
    """SzPairs::load / store of csrc/gemv.hip: the scale and zero bytes read for 16 rows x NGW
    groups (row clamp rlast, dword clamp ngd) and the LDS bytes the pairs occupy."""
    GPD = 4 // vb
    DPR = ngw // GPD
    for d in range(16 * DPR):
        rr, dw = divmod(d, DPR)
        rc = min(rr, rlast)
        gd = min(gd0 + dw, ngd - 1)
        r["s"] = max(r["s"], (row0 + rc) * ssn * vb + 4 * gd + 4)
        r["z"] = max(r["z"], (row0 + rc) * szn * vb + 4 * gd + 4)
        for e in range(GPD):
            g = dw * GPD + e
            assert g < ngw
            r["lds"] = max(r["lds"], lds_base + (rr * sz2_row(ngw) + 2 * g + 2) * 4)


def line2_plan(M, Kpad, G, N, sqn, sxm, ssn, vb, max_lds=160 * 1024):
    """line2_plan in csrc/gemv.hip: (S2, W, LDS bytes) or None when the int2 line kernel declines."""
    if not (1 <= M <= 2) or G != 64 or Kpad % LINE2 or N < 1:
        return None
    if (ssn * vb) % 4:
        return None
    if 16 * sqn >= 2 ** 31 or M * sxm * 2 >= 2 ** 31 or 16 * ssn * vb >= 2 ** 31:
        return None
    KL = Kpad // LINE2
    S2 = 4 if M == 1 else 2
    W = -(-KL // S2)
    if W > 16:
        return None
    wave_lds = M * (S2 * LINE2 + 8) * 2 + S2 * 8 * 16 * 4 + sz2_bytes(S2 * 8)
    lds = W * wave_lds + W * M * 16 * 4
    if lds > max_lds:
        return None
    return S2, W, lds


def line2_ranges(M, Kpad, N, sqn, sxm, ssn, vb, S2, W):
    """Max exclusive offsets the int2 line kernel reads from qweight (bytes), scale (bytes) and x
    (elements) and the LDS bytes its wave areas touch, from its per-lane arithmetic and clamps."""
    KL = Kpad // LINE2
    GPL = 8
    NGW = S2 * GPL
    ngd = Kpad // 64 * vb // 4
    XP = 32 * S2
    xrow = S2 * LINE2 + 8
    wave_lds = M * xrow * 2 + S2 * GPL * 16 * 4 + sz2_bytes(NGW)
    szo = M * xrow * 2 + S2 * GPL * 16 * 4
    r = dict(q=0, s=0, z=0, x=0, lds=0)
    NT = -(-N // 16)
    for tile in sorted({0, NT - 1}):
        row0 = tile * 16
        rlast = N - 1 - row0
        for wave in range(W):
            ls0 = wave * S2
            base = wave * wave_lds
            plim = Kpad - ls0 * LINE2 - 16
            for idx in range(M * XP):
                m, p = divmod(idx, XP)
                kb = min(16 * p, plim)
                assert kb >= 0
                r["x"] = max(r["x"], ls0 * LINE2 + m * sxm + kb + 16)
                r["lds"] = max(r["lds"], base + (m * xrow + 16 * p + 16) * 2)
                if p % 4 == 0:
                    r["lds"] = max(r["lds"], base + M * xrow * 2 + ((p >> 2) * 16 + m + 1) * 4)
            sz2_ranges(r, base + szo, row0, rlast, ssn, ssn, vb, NGW, ls0 * (GPL * vb // 4), ngd)
            for c in range(16):
                lo8 = c < 8
                rr0 = min(c & 7, rlast)
                rr1 = min(8 + (c & 7), rlast)
                mrow = c if c < M else M - 1
                for ar in range(4):
                    for i in range(S2):
                        l = min(ls0 + i, KL - 1)
                        r["q"] = max(r["q"], (row0 + rr0) * sqn + 16 * ar + (0 if lo8 else 64) + 128 * l + 16)
                        r["q"] = max(r["q"], (row0 + rr1) * sqn + 16 * ar + (64 if lo8 else 0) + 128 * l + 16)
                        for k in range(8):        # A reads: groups gA = 8i + k (k < 4), gB = 8i + 4 + k
                            g = GPL * i + k
                            r["lds"] = max(r["lds"], base + (mrow * xrow + 16 * ar + 64 * g + 16) * 2)
                            r["lds"] = max(r["lds"], base + M * xrow * 2 + (g * 16 + 4 * ar + M) * 4)
                            row = c if k < 4 else c ^ 8
                            r["lds"] = max(r["lds"], base + szo + (row * sz2_row(NGW) + 2 * g + 2) * 4)
    return r


LINE2_SHAPES = [(28672, 8192), (8192, 28672), (36, 512), (100, 1536), (17, 1024), (64, 16384)]


@pytest.mark.parametrize("N,K", LINE2_SHAPES)
@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("vb", [2, 4])
@pytest.mark.parametrize("pad", [0, 64])
def test_line2_reads_in_bounds(N, K, M, vb, pad):
    Kpad = K
    ng = Kpad // 64
    sqn = Kpad // 4 + pad
    plan = line2_plan(M, Kpad, 64, N, sqn, Kpad, ng, vb)
    if M == 2 and Kpad > 16384:
        assert plan is None            # M = 2 with K_pad > 16384 takes the skinny kernel
        return
    assert plan is not None
    S2, W, lds = plan
    assert W * S2 * LINE2 >= Kpad and (W - 1) * S2 * LINE2 < Kpad
    r = line2_ranges(M, Kpad, N, sqn, Kpad, ng, vb, S2, W)
    assert r["q"] <= (N - 1) * sqn + Kpad // 4
    assert r["s"] <= N * ng * vb and r["z"] <= N * ng * vb
    assert r["x"] <= (M - 1) * Kpad + Kpad
    assert r["lds"] <= lds - W * M * 16 * 4          # wave areas end where the reduction area starts


def test_line2_plan_declines():
    assert line2_plan(3, 4096, 64, 4096, 1024, 4096, 64, 2) is None      # M > 2
    assert line2_plan(1, 4096, 128, 4096, 1024, 4096, 32, 2) is None     # G != 64
    assert line2_plan(1, 448, 64, 96, 112, 448, 7, 2) is None            # K_pad % 512
    assert line2_plan(1, 33280, 64, 64, 8320, 33280, 520, 2) is None     # W > 16
    assert line2_plan(1, 32768, 64, 64, 8192, 32768, 512, 2) is None     # 16 waves exceed LDS
    assert line2_plan(1, 30720, 64, 64, 7680, 30720, 480, 4) is not None


# ---- int8 line kernel (csrc/gemv.hip w8_line_kernel / line8_plan) -----------------------------
LINE8 = 128


def line8_plan(M, K, N, sqn, sxm, max_lds=160 * 1024):
    """line8_plan in csrc/gemv.hip: (S2, W, LDS bytes) or None when the int8 line kernel declines."""
    if not (1 <= M <= 4) or K <= 0 or K % LINE8 or N < 1:
        return None
    if 16 * sqn >= 2 ** 31 or M * sxm * 2 >= 2 ** 31:
        return None
    KL = K // LINE8
    S2 = 4 if -(-KL // 4) <= 16 else 8
    W = -(-KL // S2)
    if W > 16:
        return None
    rc = M if M <= 2 else 4
    lds = W * (M * (S2 * LINE8 + 8) * 2 + 2 * S2 * 16 * 4) + W * rc * 16 * 4
    if lds > max_lds:
        return None
    return S2, W, lds


def line8_ranges(M, K, N, sqn, sxm, S2, W):
    """Max exclusive offsets the int8 line kernel reads (qweight bytes, x elements, scale rows)
    and the LDS bytes its wave areas touch, from its per-lane arithmetic and clamps."""
    KL = K // LINE8
    XB = 16 * S2
    xrow = S2 * LINE8 + 8
    wave_lds = M * xrow * 2 + 2 * S2 * 16 * 4
    r = dict(q=0, x=0, s=0, lds=0)
    NT = -(-N // 16)
    for tile in sorted({0, NT - 1}):
        row0 = tile * 16
        rlast = N - 1 - row0
        for wave in range(W):
            ls0 = wave * S2
            base = wave * wave_lds
            xlim = K - ls0 * LINE8 - 8
            assert xlim >= 0
            for idx in range(M * XB):
                m, b = divmod(idx, XB)
                kb = min(8 * b, xlim)
                r["x"] = max(r["x"], ls0 * LINE8 + m * sxm + kb + 8)
                r["lds"] = max(r["lds"], base + (m * xrow + 8 * b + 8) * 2)
                if b % 8 == 0:
                    r["lds"] = max(r["lds"], base + M * xrow * 2 + ((b >> 3) * 16 + m + 1) * 4)
            for c in range(16):
                lo8 = c < 8
                rr0 = min(c & 7, rlast)
                rr1 = min(8 + (c & 7), rlast)
                mrow = c if c < M else M - 1
                for ar in range(4):
                    for i in range(S2):
                        l = min(ls0 + i, KL - 1)
                        r["q"] = max(r["q"], (row0 + rr0) * sqn + 16 * ar + (0 if lo8 else 64) + LINE8 * l + 16)
                        r["q"] = max(r["q"], (row0 + rr1) * sqn + 16 * ar + (64 if lo8 else 0) + LINE8 * l + 16)
                        r["lds"] = max(r["lds"], base + (mrow * xrow + 16 * ar + i * LINE8 + 72 + 8) * 2)
                        r["lds"] = max(r["lds"], base + M * xrow * 2 + ((2 * i + 1) * 16 + 4 * ar + 4) * 4)
        for n in range(16):
            if n <= rlast:
                r["s"] = max(r["s"], row0 + n + 1)
    return r


@pytest.mark.parametrize("N,K", [(152064, 3584), (4096, 14336), (14336, 4096), (37, 128), (100, 384), (17, 1280),
                                 (64, 16384)])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("pad", [0, 64])
def test_line8_reads_in_bounds(N, K, M, pad):
    sqn = K + pad
    plan = line8_plan(M, K, N, sqn, K)
    assert plan is not None
    S2, W, lds = plan
    assert W * S2 * LINE8 >= K and (W - 1) * S2 * LINE8 < K
    r = line8_ranges(M, K, N, sqn, K, S2, W)
    assert r["q"] <= (N - 1) * sqn + K
    assert r["x"] <= (M - 1) * K + K
    assert r["s"] <= N
    rc = M if M <= 2 else 4
    assert r["lds"] <= lds - W * rc * 16 * 4          # wave areas end where the reduction area starts


def test_line8_plan_declines():
    assert line8_plan(5, 4096, 64, 4096, 4096) is None         # M > 4: the skinny int8 kernel
    assert line8_plan(1, 4032, 64, 4032, 4032) is None         # K % 128
    assert line8_plan(1, 8 * 16 * 128 + 128, 64, 20000, 20000) is None   # more than 16 waves of 8
    assert line8_plan(4, 16384, 64, 16384, 16384) is not None


# ---- int2 K-split decode kernel (csrc/gemv.hip w2_ksplit_kernel / ksplit2_plan) --------------
KS2_S2 = 2


def ksplit2_plan(M, Kpad, G, N, sqn, sxm, ssn, vb, max_lds=160 * 1024, cus=256):
    """ksplit2_plan in csrc/gemv.hip: (splits, NW, LDS bytes) or None when it declines."""
    if not (4 < M <= 16) or G != 64 or Kpad % LINE2 or Kpad <= 0 or N < 1:
        return None
    if N % 4 or sxm % 8 or (ssn * vb) % 4:
        return None
    if 16 * sqn >= 2 ** 31 or M * sxm * 2 >= 2 ** 31 or 16 * ssn * vb >= 2 ** 31:
        return None
    splits = -(-(Kpad // LINE2) // KS2_S2)
    nw = 4
    lds = M * (KS2_S2 * LINE2 + 8) * 2 + KS2_S2 * 8 * 16 * 4 + nw * sz2_bytes(KS2_S2 * 8)
    if lds > max_lds:
        return None
    return splits, nw, lds


def ksplit2_ranges(M, Kpad, N, sqn, sxm, ssn, vb):
    """Max exclusive offsets the int2 K-split kernel reads and writes (qweight / scale bytes, x
    elements, partials, LDS bytes), from its index arithmetic and clamps, over the first and last
    split and row block; plus the set of partial elements written over every workgroup."""
    splits, NW, _ = ksplit2_plan(M, Kpad, 64, N, sqn, sxm, ssn, vb)
    S2, GPL = KS2_S2, 8
    MC = 8 if M <= 8 else 16
    NT = 64 * NW
    KL = Kpad // LINE2
    RB = -(-N // (16 * NW))
    NGW = S2 * GPL
    ngd = Kpad // 64 * vb // 4
    XP = 32 * S2
    XU = -(-(MC * XP) // NT)
    xrow = S2 * LINE2 + 8
    xs_off = M * xrow * 2
    sz_off = xs_off + S2 * GPL * 16 * 4
    r = dict(q=0, s=0, z=0, x=0, part=0, lds=0)
    written = set()
    for split in range(splits):
        ls0 = split * S2
        plim = Kpad - ls0 * LINE2 - 16
        for rb in range(RB):
            full = split in (0, splits - 1) and rb in (0, RB - 1)
            if full:
                xtot = M * XP
                for t in range(NT):
                    for u in range(XU):
                        idx = min(t + NT * u, xtot - 1)
                        m, p = divmod(idx, XP)
                        kb = min(16 * p, plim)
                        assert kb >= 0
                        r["x"] = max(r["x"], ls0 * LINE2 + m * sxm + kb + 16)
                        if t + NT * u < xtot:
                            r["lds"] = max(r["lds"], (m * xrow + 16 * p + 16) * 2)
                            if p % 4 == 0:
                                r["lds"] = max(r["lds"], xs_off + ((p >> 2) * 16 + m + 1) * 4)
            for wave in range(NW):
                row0 = (rb * NW + wave) * 16
                tile_ok = row0 < N
                rowa = row0 if tile_ok else 0
                rlast = N - 1 - rowa
                assert rlast >= 0
                if full:
                    wbase = sz_off + wave * sz2_bytes(NGW)
                    sz2_ranges(r, wbase, rowa, rlast, ssn, ssn, vb, NGW, ls0 * (GPL * vb // 4), ngd)
                    for c in range(16):
                        lo8 = c < 8
                        rr0 = min(c & 7, rlast)
                        rr1 = min(8 + (c & 7), rlast)
                        mrow = c if c < M else M - 1
                        for ar in range(4):
                            for i in range(S2):
                                l = min(ls0 + i, KL - 1)
                                r["q"] = max(r["q"], (rowa + rr0) * sqn + 16 * ar + (0 if lo8 else 64) + 128 * l + 16)
                                r["q"] = max(r["q"], (rowa + rr1) * sqn + 16 * ar + (64 if lo8 else 0) + 128 * l + 16)
                                for k in range(8):
                                    g = GPL * i + k
                                    r["lds"] = max(r["lds"], (mrow * xrow + 16 * ar + 64 * g + 16) * 2)
                                    r["lds"] = max(r["lds"], xs_off + (g * 16 + 4 * ar + 4) * 4)
                                    row = c if k < 4 else c ^ 8
                                    r["lds"] = max(r["lds"], wbase + (row * sz2_row(NGW) + 2 * g + 2) * 4)
                for c in range(16):
                    for ar in range(4):
                        for rr in range(4):
                            m = 4 * ar + rr
                            if tile_ok and m < M and c <= rlast:
                                off = split * M * N + m * N + row0 + c
                                r["part"] = max(r["part"], off + 1)
                                written.add(off)
    return splits, r, written


KS2_SHAPES = [(28672, 8192), (8192, 28672), (4096, 4096), (36, 512), (100, 1536), (20, 1024), (80, 2560)]


@pytest.mark.parametrize("N,K", KS2_SHAPES)
@pytest.mark.parametrize("M", [5, 8, 16])
@pytest.mark.parametrize("vb", [2, 4])
@pytest.mark.parametrize("pad", [0, 64])
def test_ksplit2_in_bounds_and_covering(N, K, M, vb, pad):
    """Every int2 K-split read lies inside its operand, every LDS access inside the launch's
    dynamic LDS, the partials inside the workspace the host sizes (ceil(K_pad / 1024) * M * N fp32,
    the int4 K-split's formula), and every partial the reduction reads is written."""
    Kpad = K
    ng = Kpad // 64
    sqn = Kpad // 4 + pad
    plan = ksplit2_plan(M, Kpad, 64, N, sqn, Kpad, ng, vb)
    assert plan is not None
    splits, nw, lds = plan
    assert splits == -(-Kpad // 1024)
    splits_, r, written = ksplit2_ranges(M, Kpad, N, sqn, Kpad, ng, vb)
    assert r["q"] <= (N - 1) * sqn + Kpad // 4
    assert r["s"] <= N * ng * vb and r["z"] <= N * ng * vb
    assert r["x"] <= (M - 1) * Kpad + Kpad
    assert r["part"] <= splits * M * N
    assert len(written) == splits * M * N
    assert r["lds"] <= lds


def test_ksplit2_plan_declines():
    assert ksplit2_plan(4, 4096, 64, 4096, 1024, 4096, 64, 2) is None     # M <= 4
    assert ksplit2_plan(17, 4096, 64, 4096, 1024, 4096, 64, 2) is None    # prefill rows
    assert ksplit2_plan(8, 4096, 128, 4096, 1024, 4096, 32, 2) is None    # G != 64
    assert ksplit2_plan(8, 768, 64, 36, 192, 768, 12, 2) is None          # K_pad % 512
    assert ksplit2_plan(8, 512, 64, 37, 128, 512, 8, 2) is None           # N % 4
    assert ksplit2_plan(16, 28672, 64, 8192, 7168, 28672, 448, 4) is not None


@pytest.mark.parametrize("M,N,K", [(40, 256, 2048), (300, 512, 4096), (512, 4096, 14336), (150, 1000, 8192),
                                   (512, 14336, 4096), (2048, 4096, 14336), (17, 64, 256)])
def test_gemm_split_k_ranges(M, N, K):
    """Every split owns >= 1 K step, the splits tile [0, K/64) exactly, and the [split][M][N]
    partials fit the workspace the host sized."""
    BM, NTHR = gemm_cfg(M, N)
    BN, BK = 128, 64
    T = (-(-M // BM)) * (-(-N // BN))
    KT = K // BK
    S = split_plan(T, KT)
    kps = -(-KT // S)
    covered = []
    for sp in range(S):
        kt0 = sp * kps
        n = min(KT - kt0, kps)
        assert n >= 1, (sp, kt0, n)
        covered += list(range(kt0, kt0 + n))
    assert covered == list(range(KT))
    if S > 1:
        # stores are masked to m < M, n < N: the last partial element is ((S-1)*M + M-1)*N + N-1
        assert (((S - 1) * M + M - 1) * N + N - 1 + 1) * 4 == S * M * N * 4


# ---- grouped MoE GEMM (csrc/gemm.hip gemm_wq_kernel MOE 1-3, csrc/moe.hip moe_sort_kernel) ----
MOE_BM, MOE_BN, MOE_BK = 64, 128, 64


def moe_blocks(idx, E, bm=MOE_BM):
    """moe_sort_kernel's sorted offsets and its block list: wave 0's lanes own ceil(E / 64)
    experts each; exclusive scans of the per-lane row and block counts place each lane's blocks."""
    import numpy as np
    e_of = np.where((idx >= 0) & (idx < E), idx, 0)
    cnt = np.bincount(e_of, minlength=E)
    per = -(-E // 64)
    rows_l, blks_l = [], []
    for lane in range(64):
        e0, e1 = lane * per, min(lane * per + per, E)
        rows_l.append(int(cnt[e0:e1].sum()) if e0 < E else 0)
        blks_l.append(sum(-(-int(c) // bm) for c in cnt[e0:e1]) if e0 < E else 0)
    run, brun = 0, 0
    off = [0] * (E + 1)
    mtl = {}
    for lane in range(64):
        e0, e1 = lane * per, min(lane * per + per, E)
        b = brun
        for e in range(e0, e1):
            off[e] = run
            for r0 in range(0, int(cnt[e]), bm):
                mtl[b] = (e, run + r0)
                b += 1
            run += int(cnt[e])
        brun += blks_l[lane]
        assert b == brun
    off[E] = run
    perm = np.argsort(e_of, kind="stable")
    return off, perm, [mtl[i] for i in range(brun)]


def moe_gemm_ranges(mode, idx, E, k, K, N, I, sxm, xrows, sqe, sqn, sse, ssn, hs):
    """Max exclusive element / byte offsets of one grouped launch and the written cells."""
    B = len(idx)
    off, perm, blocks = moe_blocks(idx, E)
    max_mt = -(-B // MOE_BM) + min(E, B)
    assert len(blocks) <= max_mt
    half = MOE_BN // 2                                  # mode 1: gate rows per tile (then as many up rows)
    tiles_n = I // half if mode == 1 else -(-N // MOE_BN)
    x_hi = q_hi = s_hi = 0
    written = set()
    for e, p0 in blocks:
        cnt = min(off[e + 1] - p0, MOE_BM)
        assert cnt >= 1
        for row in range(MOE_BM):
            p = p0 + min(row, cnt - 1)
            r = p if mode == 3 else int(perm[p]) // k
            assert 0 <= r < xrows
            x_hi = max(x_hi, r * sxm + K)              # last step: chunk 7 of columns K-64 .. K
        for tn in range(tiles_n):
            for wrow in range(MOE_BN):
                gn = tn * MOE_BN + wrow
                if mode == 1:
                    gn = tn * half + wrow if wrow < half else I + tn * half + wrow - half
                gn = min(gn, N - 1)
                q_hi = max(q_hi, e * sqe + gn * sqn + 16 + (K // MOE_BK - 1) * 32 + 16)
                s_hi = max(s_hi, e * sse + gn * ssn + (K - 1) // 128 + 1)
            for m in range(cnt):
                if mode == 1:
                    for col in range(half):
                        written.add(((p0 + m) * hs + tn * half + col))
                elif mode == 2:
                    for n in range(tn * MOE_BN, min(tn * MOE_BN + MOE_BN, N), 2):
                        written.add((p0 + m) * hs + n // 2)
                else:
                    for n in range(tn * MOE_BN, min(tn * MOE_BN + MOE_BN, N)):
                        written.add(int(perm[p0 + m]) * N + n)
    return x_hi, q_hi, s_hi, written


@pytest.mark.parametrize("mode,E,T,k,H,I", [
    (1, 4, 150, 2, 512, 256), (1, 6, 96, 3, 768, 320), (2, 4, 40, 2, 3072, 2880), (3, 4, 150, 2, 512, 256),
    (3, 70, 40, 8, 256, 128), (1, 4, 24, 2, 4608, 256), (3, 4, 24, 2, 512, 4352),
])
def test_moe_gemm_in_bounds_and_covering(mode, E, T, k, H, I):
    """Every read of the grouped GEMM stays in its exact-fit buffer and the writes cover exactly
    the sorted h cells (gate_up) or the routed fp32 rows (down), for routings with empty experts,
    more than 64 rows per expert and E > 64 (several experts per lane of the sort's scan)."""
    import numpy as np
    rng = np.random.default_rng(mode * 100 + E)
    B = T * k
    idx = rng.integers(0, max(1, E - 1), size=B)         # expert E-1 never hit
    Ip = -(-I // 128) * 128
    hw = -(-Ip // 256) * 256
    if mode == 3:
        K, N, sxm, xrows = Ip, H, hw, B
    else:
        K, N, sxm, xrows = H, 2 * I, H, T
    sqn, ssn = K // 2, K // 128
    sqe, sse = N * sqn, N * ssn
    x_hi, q_hi, s_hi, written = moe_gemm_ranges(mode, idx, E, k, K, N, I, sxm, xrows, sqe, sqn, sse, ssn, hw)
    assert x_hi <= xrows * sxm
    assert q_hi <= E * sqe
    assert s_hi <= E * sse
    if mode == 3:
        assert written == {b * N + n for b in range(B) for n in range(N)}
    else:
        assert written == {p * hw + c for p in range(B) for c in range(I)}


def test_moe_blocks_model_catches_block_overlap():
    """A block list built with a wrong block size (rows of 64-row blocks counted as 32) overlaps."""
    import numpy as np
    idx = np.repeat(np.arange(3), 100)
    off, _, blocks = moe_blocks(idx, 3, bm=32)
    spans = [(p0, min(off[e + 1] - p0, MOE_BM)) for e, p0 in blocks]
    cover = sorted(p for p0, c in spans for p in range(p0, p0 + c))
    assert len(cover) != len(set(cover))


# ---- MoE decode line kernels (csrc/moe.hip dec_tile_partial, moe_dn_line_kernel) -------------
DLINE = 256


def dec_shape(Kpad, groups):
    """dec_shape in csrc/moe.hip."""
    if Kpad % DLINE:
        return None
    KL = Kpad // DLINE
    for s in (2, 4):
        w = -(-KL // s)
        if w * groups <= 16:
            return s, w
    return None


def dec_ranges(pair, E, H, Kpad, vb, sqe, sqn, sse, ssn, e_list, rbase_rows, scale_index=None):
    """Max exclusive byte offsets of the weight and scale reads of every wave, and the largest
    output row, for a down launch (pair) or a 16-row tile form; `scale_index` overrides the scale
    element formula (for the negative control)."""
    S2, Wk = dec_shape(Kpad, 1)
    KL = Kpad // DLINE
    DPR = S2 * vb // 2
    ngd = Kpad // 128 * vb // 4
    q_hi = s_hi = 0
    idx = scale_index or (lambda ex, row: ex * sse + row * ssn)
    for e, e2 in e_list:
        for rbase in rbase_rows:
            for wk in range(-(-KL // S2)):
                ls0 = wk * S2
                for lane in range(64):
                    c, ar = lane & 15, lane >> 4
                    lo8 = c < 8
                    r0 = rbase + (c & 7)
                    r1 = rbase + (c & 7) if pair else rbase + 8 + (c & 7)
                    e1 = e2 if pair else e
                    for i in range(S2):
                        l = min(ls0 + i, KL - 1)
                        q_hi = max(q_hi, e * sqe + r0 * sqn + 16 * ar + (0 if lo8 else 64) + 128 * l + 16,
                                   e1 * sqe + r1 * sqn + 16 * ar + (64 if lo8 else 0) + 128 * l + 16)
                    for u in range(-(-(32 * DPR) // 64)):
                        d = min(lane + 64 * u, 32 * DPR - 1)
                        rem = d % (16 * DPR)
                        r, dw = rem // DPR, rem % DPR
                        gd = min(ls0 * (vb // 2) + dw, ngd - 1)
                        second = pair and r >= 8
                        el = idx(e2 if second else e, rbase + (r - 8 if second else r))
                        s_hi = max(s_hi, el * vb + 4 * gd + 4)
    return q_hi, s_hi


@pytest.mark.parametrize("pair,H,Kpad,vb", [(True, 2048, 1024, 2), (True, 2880, 3072, 2), (True, 512, 512, 4),
                                             (False, 2048, 2048, 2)])
def test_dec_reads_in_bounds(pair, H, Kpad, vb):
    """Both forms read inside exact-fit weight and scale buffers of E experts, for the first and
    last experts and row tiles (every other tile lies between them)."""
    E = 5
    sqn, ssn = Kpad // 2, Kpad // 128
    sqe, sse = H * sqn, H * ssn
    step = 8 if pair else 16
    rows = [0, H - step]
    q_hi, s_hi = dec_ranges(pair, E, H, Kpad, vb, sqe, sqn, sse, ssn, [(0, E - 1), (E - 1, 0), (E - 1, E - 1)], rows)
    assert q_hi <= E * sqe
    assert s_hi <= E * sse * vb


def test_dec_model_catches_expert_stride_times_row_stride():
    """The scale element (e sse + row) ssn -- the expert stride scaled by the row stride -- is
    caught: it runs past the buffer."""
    E, H, Kpad, vb = 5, 2048, 1024, 2
    sqn, ssn = Kpad // 2, Kpad // 128
    sqe, sse = H * sqn, H * ssn
    _, s_hi = dec_ranges(True, E, H, Kpad, vb, sqe, sqn, sse, ssn, [(E - 1, E - 1)], [H - 8],
                         scale_index=lambda ex, row: (ex * sse + row) * ssn)
    assert s_hi > E * sse * vb


# ---- the restated plans against the compiled dispatcher's (imq_launch_plan) ---------------------
# Every plan above restates a host function of the library; imq_launch_plan runs those functions
# (host code, no device), so a drift between the model and the compiled dispatch fails here.

def _lib_plan(kind, M, K, G, N, sqn, sxm, ssn, vb, max_lds, cus):
    import os
    from infinitemodel_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} is not built")
    sdt = _lib.IMQ_DT_FP32 if vb == 4 else _lib.IMQ_DT_BF16
    return _lib.launch_plan(kind, M, K, G, N, sqn, sxm, ssn, sdt, max_lds, cus)


TIE_SHAPES = [(4096, 4096), (6144, 4096), (28672, 4096), (4096, 14336), (28672, 8192), (8192, 28672),
              (16400, 2048), (16392, 4096), (37, 512), (100, 1536), (20, 1024), (64, 16384), (17, 256),
              (151936, 3584), (2880, 2944), (80, 2560)]
TIE_DEVICES = [(160 * 1024, 256), (64 * 1024, 256), (160 * 1024, 80), (160 * 1024, 32)]


@pytest.mark.parametrize("max_lds,cus", TIE_DEVICES)
@pytest.mark.parametrize("vb", [2, 4])
def test_decode_plans_match_compiled_dispatch(max_lds, cus, vb):
    from infinitemodel_amd import _lib
    checked = 0
    for N, K in TIE_SHAPES:
        for M in (1, 2, 3, 4, 5, 8, 12, 16):
            for pad in (0, 64):
                sxm = K + pad
                # int4 g128
                Kp = -(-K // 128) * 128
                sqn, ssn = Kp // 2 + pad, -(-Kp // 128) + pad // 2
                args = (M, Kp, 128, N, sqn, sxm + (Kp - K), ssn, vb, max_lds, cus)
                want = line_plan(M, Kp, 128, N, sqn, sxm + (Kp - K), ssn, vb, max_lds)
                got = _lib_plan(_lib.IMQ_PLAN_W4_LINE, *args)
                assert (got and (got[0], got[1], got[3])) == want, ("w4 line", N, K, M, pad)
                want = ksplit_plan(M, Kp, 128, N, sqn, sxm + (Kp - K), ssn, vb, max_lds, cus)
                got = _lib_plan(_lib.IMQ_PLAN_W4_KSPLIT, *args)
                assert (got and (got[0], got[1], got[3], got[2])) == want, ("w4 ksplit", N, K, M, pad)
                want = wsplit_plan(M, Kp, 128, N, sqn, sxm + (Kp - K), ssn, vb, cus, max_lds)
                got = _lib_plan(_lib.IMQ_PLAN_W4_WSPLIT, *args)
                assert (got and got[0]) == want, ("w4 wsplit", N, K, M, pad)
                _, S, W = _dispatch(Kp, N, vb == 2)
                got = _lib_plan(_lib.IMQ_PLAN_W4_SKINNY, *args)
                assert got[:2] == (S, W), ("w4 skinny", N, K, M)
                # int2 g64
                K2 = -(-K // 64) * 64
                sqn2, ssn2 = K2 // 4 + pad, K2 // 64 + pad // 2
                args2 = (M, K2, 64, N, sqn2, K2 + pad, ssn2, vb, max_lds, cus)
                want = line2_plan(M, K2, 64, N, sqn2, K2 + pad, ssn2, vb, max_lds)
                got = _lib_plan(_lib.IMQ_PLAN_W2_LINE, *args2)
                assert (got and (got[0], got[1], got[3])) == want, ("w2 line", N, K, M, pad)
                want = ksplit2_plan(M, K2, 64, N, sqn2, K2 + pad, ssn2, vb, max_lds, cus)
                got = _lib_plan(_lib.IMQ_PLAN_W2_KSPLIT, *args2)
                assert (got and (got[0], got[1], got[3])) == want, ("w2 ksplit", N, K, M, pad)
                # int8 per row (K as given, no padding)
                want = line8_plan(M, K, N, K + pad, K + pad, max_lds)
                got = _lib_plan(_lib.IMQ_PLAN_W8_LINE, M, K, 0, N, K + pad, K + pad, 0, vb, max_lds, cus)
                assert (got and (got[0], got[1], got[3])) == want, ("w8 line", N, K, M, pad)
                checked += 1
    assert checked == len(TIE_SHAPES) * 8 * 2


@pytest.mark.parametrize("cus", [256, 80, 32])
def test_gemm_plans_match_compiled_dispatch(cus):
    from infinitemodel_amd import _lib
    for N, K in TIE_SHAPES:
        K64 = -(-K // 64) * 64
        for M in (17, 64, 128, 129, 512, 513, 2048, 4096):
            BM, _threads = gemm_cfg(M, N)
            T = -(-M // BM) * -(-N // 128)
            s = split_plan(T, K64 // 64, cus)
            got = _lib_plan(_lib.IMQ_PLAN_GEMM, M, K64, 128, N, 0, 0, 0, 2, 160 * 1024, cus)
            assert got[:3] == (BM, 128, s), (N, K, M)


def test_register_b_plan_at_the_prefill_shapes():
    """The register-B GEMM's plan at the C4 prefill shapes on 256 CUs, as documented: 256-row
    tiles (8 blocks per wave), one K split for 4096->14336, two for 14336->4096 (int4 and int8);
    it declines 512 rows and below."""
    from infinitemodel_amd import _lib
    for G in (128, 0):
        assert _lib_plan(_lib.IMQ_PLAN_GEMM_RB, 2048, 4096, G, 14336, 0, 0, 0, 2, 0, 256)[:2] == (8, 1)
        assert _lib_plan(_lib.IMQ_PLAN_GEMM_RB, 2048, 14336, G, 4096, 0, 0, 0, 2, 0, 256)[:2] == (8, 2)
        assert _lib_plan(_lib.IMQ_PLAN_GEMM_RB, 512, 4096, G, 14336, 0, 0, 0, 2, 0, 256) is None


# ---- register-B prefill GEMM, dense form (csrc/rb_kernel.h gemm_rb_kernel MOE 0, gemm_rb.hip) ---
# NW = 4 waves of 64 columns (BN 256), BM = 32 IB rows, K steps of 64. The model restates
# rb_plan, the launcher's split-K shape (kps = ceil(KT / s), KT_split = min(KT - kt0, kps)), the
# XCD-aware grouped tile mapping, the activation plan (row clamp to M - 1, 8 chunks of 16 bytes
# per row), the weight plan (column clamp to N - 1, 16 bytes per half-wave per step for int4, 32
# for int8), the group index of the scale / zero loads, the swizzled LDS stores and the masked
# partial / output stores, and checks every access against its buffer -- plus that the workgroups
# cover every (row tile, column tile, split) once and every output element once per split.
RB_BK, RB_NW = 64, 4


def rb_plan(M, N, K, cus=256):
    """rb_plan in csrc/gemm_rb.hip: (32-row blocks per wave, K splits)."""
    T8 = -(-M // 256) * -(-N // 256)
    T4 = -(-M // 128) * -(-N // 256)
    ib = 8 if (M > 128 and 2 * T8 >= cus) else 4
    T = T8 if ib == 8 else T4
    KT = K // RB_BK
    s = 1
    while s < 4 and 2 * T * s <= cus and KT // (2 * s) >= 16:
        s *= 2
    return ib, s


def rb_tile(b, tiles_m, tiles_n, BM, BN):
    """The dense form's tile mapping of workgroup b: (split, m0, n0)."""
    T = tiles_m * tiles_n
    split, L = divmod(b, T)
    if T % 8 == 0:
        L = (L & 7) * (T >> 3) + (L >> 3)
    per_group = 8 * tiles_n
    grp = L // per_group
    first_m = grp * 8
    gm = min(tiles_m - first_m, 8)
    in_grp = L - grp * per_group
    return split, (first_m + in_grp % gm) * BM, (in_grp // gm) * BN


def rb_swz(row, ch):
    return (row * 8 + (ch ^ ((row >> 1) & 7))) * 8


def rb_store_rows(ib):
    """Row offsets (within the tile) of the MFMA output elements a lane stores: 32 i + 8 (r >> 2) +
    4 h + (r & 3) over i < IB, r < 16, h < 2 (the 32x32 MFMA's D layout)."""
    return sorted(32 * i + 8 * (r >> 2) + 4 * h + (r & 3) for i in range(ib) for r in range(16) for h in range(2))


def rb_ranges(M, N, K, bits, G, sxm, sqn, ssn, ssg, sym, cus=256, row_clamp=True):
    """Every global element / byte range the dense register-B GEMM reads or writes, and the LDS
    range of its activation stores, as (lo, hi) pairs per buffer; with the coverage checks."""
    import numpy as np
    ib, s = rb_plan(M, N, K, cus)
    BM, BN, NTHR = 32 * ib, 64 * RB_NW, 64 * RB_NW
    tiles_m, tiles_n = -(-M // BM), -(-N // BN)
    KT = K // RB_BK
    kps = -(-KT // s)
    XC = BM * 8 // NTHR
    QV = 2 if bits == 8 else 1
    gsh = 0 if bits == 8 else int(math.log2(G))
    step = RB_BK * bits // 8
    # a lane's stored rows are each tile row once, and the activation plan's ids cover BM rows x 8 chunks
    assert rb_store_rows(ib) == list(range(BM))
    ids = np.arange(XC * NTHR)
    rows, chs = ids >> 3, ids & 7
    assert rows.max() == BM - 1
    swz = (rows * 8 + (chs ^ ((rows >> 1) & 7))) * 8
    assert len(set(swz.tolist())) == BM * 8           # the swizzle is a permutation of the chunks
    r = {"lds": [int(swz.min()), int(swz.max()) + 8]}
    cols = np.arange(BN)                               # n0 + 64 w + 32 j + c over w, j, c
    lo = {k: math.inf for k in ("x", "q", "s", "part", "y")}
    hi = {k: -math.inf for k in lo}
    cover = np.zeros((s, M, N), dtype=np.int8)
    seen = set()
    for b in range(tiles_m * tiles_n * s):
        split, m0, n0 = rb_tile(b, tiles_m, tiles_n, BM, BN)
        assert (split, m0, n0) not in seen
        seen.add((split, m0, n0))
        kt0 = split * kps
        kts = min(KT - kt0, kps)
        assert kts >= 1, (M, N, K, b)
        kt_lo, kt_hi = kt0, kt0 + kts - 1            # load_a / load_b clamp ktl to KT_split - 1
        rr = np.where((m0 + rows < M) | (not row_clamp), rows, M - 1 - m0)
        xb = (m0 + rr) * sxm + chs * 8
        lo["x"] = min(lo["x"], int(xb.min()) + kt_lo * RB_BK)
        hi["x"] = max(hi["x"], int(xb.max()) + kt_hi * RB_BK + 8)
        n = np.minimum(n0 + cols, N - 1)
        for h in range(2):
            qb = n * sqn + (32 if bits == 8 else 16) * h
            lo["q"] = min(lo["q"], int(qb.min()) + kt_lo * step)
            hi["q"] = max(hi["q"], int(qb.max()) + kt_hi * step + 16 * QV)
            if bits != 8:
                g_lo, g_hi = (kt_lo * RB_BK + 32 * h) >> gsh, (kt_hi * RB_BK + 32 * h) >> gsh
                lo["s"] = min(lo["s"], int(n.min()) * ssn + g_lo * ssg)
                hi["s"] = max(hi["s"], int(n.max()) * ssn + g_hi * ssg + 1)
            else:
                lo["s"] = min(lo["s"], int(n.min()) * ssn)
                hi["s"] = max(hi["s"], int(n.max()) * ssn + 1)
        m_hi, n_hi = min(m0 + BM, M), min(n0 + BN, N)  # stores are masked to m < M, n < N
        cover[split, m0:m_hi, n0:n_hi] += 1
        if s > 1:
            lo["part"] = min(lo["part"], split * M * N + m0 * N + n0)
            hi["part"] = max(hi["part"], split * M * N + (m_hi - 1) * N + n_hi)
        else:
            lo["y"] = min(lo["y"], m0 * sym + n0)
            hi["y"] = max(hi["y"], (m_hi - 1) * sym + n_hi)
    assert len(seen) == tiles_m * tiles_n * s
    assert (cover == 1).all(), "every output element once per split"
    for k in lo:
        r[k] = [lo[k], hi[k]]
    return r, (ib, s, BM)


RB_CASES = [(600, 1000, 14336, 4, 128), (600, 1000, 14336, 8, 0), (2100, 4000, 256, 4, 128),
            (513, 96, 512, 4, 64), (1000, 1000, 4096, 4, 32), (2048, 4096, 14336, 8, 0),
            (777, 300, 2048, 8, 0), (1030, 2600, 6144, 4, 128)]


@pytest.mark.parametrize("M,N,K,bits,G", RB_CASES)
@pytest.mark.parametrize("pad", [0, 64])
def test_register_b_in_bounds_and_covering(M, N, K, bits, G, pad):
    row_bytes = K * bits // 8
    sqn = row_bytes + pad
    ng = K // G if G else 1
    ssn = ng + (8 if pad else 0)
    sxm = K + (8 if pad else 0)
    rg, (ib, s, BM) = rb_ranges(M, N, K, bits, G, sxm, sqn, ssn, 1, N)
    assert rg["x"][0] >= 0 and rg["x"][1] <= (M - 1) * sxm + K
    assert rg["q"][0] >= 0 and rg["q"][1] <= (N - 1) * sqn + row_bytes
    assert rg["s"][0] >= 0 and rg["s"][1] <= (N - 1) * ssn + ng
    assert rg["lds"][0] >= 0 and rg["lds"][1] <= BM * RB_BK
    if s > 1:
        assert rg["part"][0] >= 0 and rg["part"][1] <= s * M * N
    else:
        assert rg["y"][0] >= 0 and rg["y"][1] <= (M - 1) * N + N


def test_register_b_ragged_split_case_is_split():
    """The GPU parity case M=600, N=1000, K=14336 runs 128-row tiles with four K splits on 256 CUs
    (partial stores of ragged tiles and the reduction's tails), as the restated and compiled plans
    both say."""
    from infinitemodel_amd import _lib
    assert rb_plan(600, 1000, 14336) == (4, 4)
    for G in (128, 0):
        assert _lib_plan(_lib.IMQ_PLAN_GEMM_RB, 600, 14336, G, 1000, 0, 0, 0, 2, 0, 256)[:2] == (4, 4)


@pytest.mark.parametrize("cus", [256, 80, 32])
def test_register_b_plans_match_compiled_dispatch(cus):
    from infinitemodel_amd import _lib
    for M, N, K, bits, G in RB_CASES + [(4096, 14336, 4096, 4, 128), (8192, 4096, 14336, 4, 128)]:
        got = _lib_plan(_lib.IMQ_PLAN_GEMM_RB, M, K, G if bits == 4 else 0, N, 0, 0, 0, 2, 0, cus)
        assert got is not None and got[:2] == rb_plan(M, N, K, cus), (M, N, K, cus)


def test_register_b_model_catches_missing_row_clamp():
    """Negative control: without the activation row clamp, the ragged last row tile would read
    past x."""
    M, N, K = 600, 1000, 14336
    rg, _ = rb_ranges(M, N, K, 4, 128, K, K // 2, K // 128, 1, N, row_clamp=False)
    assert rg["x"][1] > (M - 1) * K + K


def test_dec_a_operand_lds_reads_stay_in_the_staged_rows():
    """MoE decode (dec_tile_partial): lane (c, ar) reads its A operands at xa + i * 256 + 8 kk
    (16 bytes) with xa = row offset + 32 ar + (gate_up form, c == 1: 128, the line-step's second
    group; slot-pair form, c == 1: the second staged row). Every read stays inside the staged
    row(s) of S2 * 256 + 8 elements, for both forms and S2 2 / 4."""
    for S2 in (2, 4):
        xrowl = S2 * 256 + 8
        for pair in (False, True):
            nx = 2 if pair else 1
            for c in range(16):
                for ar in range(4):
                    base = (xrowl if (pair and c == 1) else 0) + (128 if (not pair and c == 1) else 0) + 32 * ar
                    row0 = xrowl if (pair and c == 1) else 0
                    for i in range(S2):
                        for kk in range(4):
                            lo = base + i * 256 + 8 * kk
                            assert row0 <= lo and lo + 8 <= row0 + S2 * 256 <= nx * xrowl, (S2, pair, c, ar, i, kk)
