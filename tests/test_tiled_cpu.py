"""The line-tiled int4 layout (CPU): its definition is a permutation of 16-byte pieces within each
16-row tile, and a block's slots are exactly the pieces the decode kernels' full-line loads give
each lane in the row layout (lane c + 16 ar of the rows 0-7 load: row c & 7, bytes 16 ar, + 64
for c >= 8; of the rows 8-15 load: row 8 + (c & 7), + 64 for c < 8), so a kernel reading slot
16 ar + c of a tiled block sees the bytes its row-layout form loads."""
import numpy as np

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
