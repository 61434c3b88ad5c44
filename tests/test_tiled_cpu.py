"""The line-tiled int4 layout (CPU): its definition is a permutation of 16-byte pieces within each
16-row tile, and a block's slots are exactly the pieces the decode kernels' full-line loads give
each lane in the row layout (lane c + 16 ar of the rows 0-7 load: row c & 7, bytes 16 ar, + 64
for c >= 8; of the rows 8-15 load: row 8 + (c & 7), + 64 for c < 8), so a kernel reading slot
16 ar + c of a tiled block sees the bytes its row-layout form loads."""
import numpy as np
import pytest

from tests import _cases as C


def test_tiling_is_a_permutation_of_pieces_within_tiles():
    N, KB = 48, 384
    ids = np.repeat(np.arange(N * KB // 16, dtype=np.int64), 16).reshape(N, KB)   # one id per piece
    tiled_ids = _tile_ids(ids)
    assert sorted(tiled_ids.tolist()) == list(range(N * KB // 16))
    for tile, blk in enumerate(tiled_ids.reshape(N // 16, -1)):
        assert set(((blk * 16) // KB) // 16) == {tile}   # every source row lies in the same tile
    # the byte-level helper moves whole pieces the same way
    q = (ids % 251).astype(np.uint8)
    assert np.array_equal(C.line_tile_np(q).reshape(-1, 16)[:, 0], (tiled_ids % 251).astype(np.uint8))


def _tile_ids(ids):
    """line_tile_np on int64 piece ids (one id per 16-byte piece)."""
    N, KB = ids.shape
    KL = KB // 128
    p = ids.reshape(N // 16, 16, KL, 8, 16)[..., 0]
    out = np.empty((N // 16, KL, 2, 64), dtype=np.int64)
    for h in range(2):
        for s in range(64):
            out[:, :, h, s] = p[:, 8 * h + (s & 7), :, 4 * (((s >> 3) & 1) ^ h) + (s >> 4)]
    return out.reshape(-1)


def test_block_slots_are_the_row_layout_lane_pieces():
    N, KB = 16, 256                    # one tile, two line-steps
    r = np.random.default_rng(5)
    q = r.integers(0, 256, size=(N, KB), dtype=np.uint8)
    t = C.line_tile_np(q)
    for l in range(KB // 128):
        blk = t.reshape(-1)[2048 * l: 2048 * (l + 1)]
        for load in range(2):
            for lane in range(64):
                c, ar = lane & 15, lane >> 4
                row = (c & 7) + 8 * load
                second = (c >= 8) if load == 0 else (c < 8)
                b0 = 128 * l + 16 * ar + (64 if second else 0)
                want = q[row, b0:b0 + 16]
                got = blk[1024 * load + 16 * lane: 1024 * load + 16 * lane + 16]
                assert np.array_equal(got, want), (l, load, lane)


def test_planted_slot_error_is_caught():
    """A tiling with the half's group swap dropped (piece (s >> 4) + 4 ((s >> 3) & 1) in both
    halves) differs from the definition in the rows 8-15 half."""
    N, KB = 16, 128
    q = np.random.default_rng(1).integers(0, 256, size=(N, KB), dtype=np.uint8)
    p = q.reshape(16, 1, 8, 16)
    bad = np.empty((1, 2, 64, 16), dtype=np.uint8)
    for h in range(2):
        for s in range(64):
            bad[0, h, s] = p[8 * h + (s & 7), 0, 4 * ((s >> 3) & 1) + (s >> 4)]
    good = C.line_tile_np(q).reshape(1, 2, 64, 16)
    assert np.array_equal(bad[0, 0], good[0, 0]) and not np.array_equal(bad[0, 1], good[0, 1])


def test_module_host_untile_inverts_the_definition():
    """The module's host-side conversion (a line-tiled module moved off the GPU) restores rows."""
    import torch
    from infinitemodel_amd import worker_quant as wq
    q = np.random.default_rng(3).integers(0, 256, size=(64, 768), dtype=np.uint8)
    back = wq._line_untile_torch(torch.from_numpy(C.line_tile_np(q)))
    assert np.array_equal(back.numpy(), q)


# ---- the kernels' tiled address formulas against the layout's definition -----------------------
# Each restates one kernel's per-lane offset arithmetic (csrc) for the line-tiled layout and checks
# that the 16 bytes it reads for (row, row-layout byte) are those line_tile_np puts there.

def _piece_ids(N, KB):
    return np.repeat(np.arange(N * KB // 16, dtype=np.int64), 16).reshape(N, KB)


def _tiled_piece_at(N, KB):
    """tiled byte offset // 16 -> row-layout piece id (row * KB/16 + byte/16)."""
    return _tile_ids(_piece_ids(N, KB))


def test_line_kernel_tiled_loads_cover_each_tile_once():
    """Line / K-split / wave-split kernels: lane l of the rows 0-7 load reads bytes 16 l of the
    tile's line-step block, the rows 8-15 load 1024 + 16 l; over a workgroup's waves and
    line-steps every piece of the tile is read once, in the lane the row-layout form reads it."""
    for KB in (128, 256, 1792, 2048):
        N = 32
        tiled = _tiled_piece_at(N, KB)
        KL = KB // 128
        for t in range(N // 16):
            seen = set()
            for l in range(KL):
                for load in range(2):
                    for lane in range(64):
                        off = t * 16 * KB + 2048 * l + 1024 * load + 16 * lane
                        assert 0 <= off < (t + 1) * 16 * KB
                        pid = int(tiled[off // 16])
                        row, piece = divmod(pid, KB // 16)
                        c, ar = lane & 15, lane >> 4
                        second = (c >= 8) if load == 0 else (c < 8)
                        assert row == 16 * t + (c & 7) + 8 * load
                        assert piece == 8 * l + ar + (4 if second else 0)
                        seen.add(pid)
            assert len(seen) == 16 * KB // 16


@pytest.mark.parametrize("bits", [4, 8])
def test_register_b_tiled_offsets(bits):
    """gemm_rb_kernel (TL): lane (column n, half h) reads at K step kt the pieces v < QV of bytes
    SB kt + (16 QV) h + 16 v of row n, SB = 32 (int4) / 64 (int8), from qto[sel] + 256 v + so."""
    KB, N = 2048, 64
    tiled = _tiled_piece_at(N, KB)
    SB, QV = (64, 2) if bits == 8 else (32, 1)
    for rr in range(N):
        hr = (rr >> 3) & 1
        for h in range(2):
            tb = (rr >> 4) * 16 * KB + 1024 * hr + 16 * (rr & 7) + (512 if bits == 8 else 256) * h
            qto = (tb + 128 * hr, tb + 128 * (1 - hr))
            for kt in range(KB // SB):
                sel = (kt & 1) if bits == 8 else ((kt >> 1) & 1)
                so = 2048 * (kt >> 1) if bits == 8 else 2048 * (kt >> 2) + 512 * (kt & 1)
                for v in range(QV):
                    off = qto[sel] + 256 * v + so
                    b = SB * kt + 16 * QV * h + 16 * v
                    assert tiled[off // 16] == rr * (KB // 16) + b // 16 and off % 16 == 0


@pytest.mark.parametrize("bits,WC", [(4, 16), (4, 32), (2, 16), (2, 32), (8, 16), (8, 32)])
def test_lds_dequant_gemm_tiled_offsets(bits, WC):
    """gemm_wq_kernel (TL): thread (row rr, part) reads WC codes = WC bits / 8 bytes at byte
    SB kt + o of its row (o = part WC bits / 8, SB = 64 bits / 8) from (sel ? wtb : wta) + step,
    a 32-byte int8 read as two pieces 256 bytes apart."""
    KB, N = 1024, 32
    tiled = _tiled_piece_at(N, KB)
    SB, nbytes = 64 * bits // 8, WC * bits // 8
    for rr in range(N):
        hr = (rr >> 3) & 1
        for part in range(SB // nbytes):
            o = part * nbytes
            tb = (rr >> 4) * 16 * KB + 1024 * hr + 16 * (rr & 7) + 256 * (o >> 4) + (o & 15)
            wta, wtb = tb + 128 * hr, tb + 128 * (1 - hr)
            for kt in range(KB // SB):
                step = (2048 * (kt >> 1) if bits == 8 else 2048 * (kt >> 2) + 512 * (kt & 1) if bits == 4
                        else 2048 * (kt >> 3) + 256 * (kt & 3))
                sel = (kt & 1) if bits == 8 else ((kt >> 1) & 1) if bits == 4 else ((kt >> 2) & 1)
                p = (wtb if sel else wta) + step
                chunks = [(p, 0)] if nbytes <= 16 else [(p, 0), (p + 256, 16)]
                for addr, boff in chunks:
                    b = SB * kt + o + boff
                    assert tiled[addr // 16] == rr * (KB // 16) + b // 16
                    assert addr % 16 == b % 16


def test_int8_skinny_tiled_offsets():
    """w8_skinny_kernel (TL): lane (nl, jl) reads at K step st (64 bytes) the piece at byte
    64 st + 16 jl of tile row nl from (st odd ? qto : qte) + 2048 (st / 2)."""
    KB, N = 1024, 32
    tiled = _tiled_piece_at(N, KB)
    for tile in range(N // 16):
        for nl in range(16):
            th = nl >> 3
            for jl in range(4):
                qtile = tile * 16 * KB + 1024 * th + 16 * (nl & 7) + 256 * jl
                qte, qto = qtile + 128 * th, qtile + 128 * (1 - th)
                for st in range(KB // 64):
                    off = (qto if st & 1 else qte) + 2048 * (st >> 1)
                    assert tiled[off // 16] == (16 * tile + nl) * (KB // 16) + (64 * st + 16 * jl) // 16
