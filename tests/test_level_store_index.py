"""CPU model of where the matrix-core CS pass (fa_ssim_mfma.hip, modes CS and
CSO) writes the next MS-SSIM pyramid level.

The kernel stores each level value through a buffer resource whose base is
the block's first level row (inside the chunk's plane) and whose range ends
at the last level row the chunk writes; the lane's byte offset is fixed (row
2g + q of the block, its column) or 0x80000000 for lanes that store nothing,
and the hardware drops every store whose offset is not below the range.  This
model replays that arithmetic for every workgroup, wave, block and lane of a
launch -- every uniform chunk height the host may pick, and the big-then-small
chunk lists it builds from them -- and checks that each element of each
plane's level is written, and only from inside that plane, and that the
stores of the steps past a chunk's last block write nothing.
"""

from __future__ import annotations

import numpy as np
import pytest

MT, WPB = 16, 4  # block size, waves per workgroup (fa_ssim_mfma.hip)


def chunk_rows(Hout, TH, nbig=None, THs=None):
    """(r0, r_lim) of each chunk of a column: nbig chunks of TH rows, then
    chunks of THs rows (uniform when nbig is None), as the kernel derives them
    from its chunk index (fa_ssim_mfma.hip)."""
    if nbig is None:
        nbig, THs = (Hout + TH - 1) // TH, TH
    out, k = [], 0
    while True:
        r0 = k * TH if k < nbig else nbig * TH + (k - nbig) * THs
        if r0 >= Hout:
            return out
        out.append((r0, r0 + (TH if k < nbig else THs)))
        k += 1


def big_small(blocks, chunks):
    """The host's big-then-small list for a uniform count of ``chunks``:
    (TH, nbig, THs) in rows, or None where it keeps the uniform list."""
    if chunks < 2:
        return None
    nb = (chunks + 1) // 2
    ns = chunks - nb
    big = int(np.floor(blocks / (nb + 0.4 * ns) + 0.5))
    if big * nb >= blocks:
        return None
    small = (blocks - big * nb + ns - 1) // ns
    if small >= big:
        return None
    return MT * big, nb, MT * small


def level_writes(N, C, H, W, K, TH, eb, short_rows=0, col_shift=0, nbig=None, THs=None):
    """Counts of writes per level element, and whether any store left its plane.
    ``short_rows`` / ``col_shift`` plant mistakes (a range that ends early, a
    lane offset one column off) for the negative controls."""
    Hout, Wout = H - K + 1, W - K + 1
    strips = (Wout + WPB * MT - 1) // (WPB * MT)
    Hd, Wd = H // 2, W // 2
    rstep = Wd * eb
    count = np.zeros(N * C * Hd * Wd, dtype=np.int64)
    g = np.arange(4)[:, None]
    n = np.arange(16)[None, :]
    for plane in range(N * C):
        for r0, r_lim in chunk_rows(Hout, TH, nbig, THs):
            r_end = min(r_lim, Hout)
            nb = (r_end - r0 + MT - 1) // MT
            row_end = 2 * (H // 2) if r_lim >= Hout else r_lim
            rows = row_end // 2 - r0 // 2
            first = (plane * Hd + r0 // 2) * Wd  # element index of the chunk's base
            for strip in range(strips):
                for wave in range(WPB):
                    c0 = (strip * WPB + wave) * MT
                    if c0 >= Wout:
                        continue
                    last_wave = c0 + MT >= Wout
                    lane_on = ((wave % 2 == 0) or last_wave) & (c0 // 2 + n < Wd)
                    lo = np.where(lane_on, (2 * g * Wd + c0 // 2 + n + col_shift) * eb,
                                  0x80000000)
                    lo = np.broadcast_to(lo, (4, 16))
                    # H blocks 0 .. nb, and the two steps past the last
                    # block, whose stores the float16 / float32 level passes
                    # issue anyway (with the previous block's values): the
                    # range check must drop every one of those
                    for j in range(nb + 3):
                        row = MT // 2 * j
                        rng = max(rows - short_rows - row, 0) * rstep
                        for q in range(2):
                            o = lo + q * rstep
                            kept = o < rng  # the range check (unsigned offsets)
                            if not kept.any():
                                continue
                            if j > nb:
                                return count, False
                            assert np.all(o[kept] % eb == 0)
                            elem = first + row * Wd + o[kept] // eb
                            lo_plane, hi_plane = plane * Hd * Wd, (plane + 1) * Hd * Wd
                            if np.any(elem < lo_plane) or np.any(elem >= hi_plane):
                                return count, False
                            np.add.at(count, elem, 1)
    return count, True


@pytest.mark.parametrize("eb", [2, 4])  # float16 or float32 level
@pytest.mark.parametrize("N,C,H,W", [(1, 1, 32, 32), (1, 2, 44, 72), (2, 1, 61, 136),
                                     (1, 1, 90, 200), (1, 1, 127, 264), (1, 1, 176, 176)])
def test_every_level_element_written_inside_its_plane(eb, N, C, H, W):
    K = 11
    Hout = H - K + 1
    blocks = (Hout + MT - 1) // MT
    for m in range(1, blocks + 1):  # every chunk height the host may choose
        count, inside = level_writes(N, C, H, W, K, MT * m, eb)
        assert inside, (N, C, H, W, MT * m)
        assert count.min() >= 1, (N, C, H, W, MT * m, int(np.argmin(count)))
        bs = big_small(blocks, (blocks + m - 1) // m)
        if bs is not None:
            TH, nbig, THs = bs
            count, inside = level_writes(N, C, H, W, K, TH, eb, nbig=nbig, THs=THs)
            assert inside, (N, C, H, W, bs)
            assert count.min() >= 1, (N, C, H, W, bs, int(np.argmin(count)))


def test_big_small_lists_cover_the_column():
    # every big-then-small list covers blocks 0 .. blocks-1 once, big chunks
    # first, the configs[1] column (67 blocks, 4 chunks) as 24, 24, 10, 9
    for blocks in range(2, 140):
        for chunks in range(2, blocks + 1):
            bs = big_small(blocks, chunks)
            if bs is None:
                continue
            TH, nbig, THs = bs
            rows = chunk_rows(blocks * MT, TH, nbig, THs)
            assert rows[0][0] == 0 and all(a[1] == b[0] for a, b in zip(rows, rows[1:]))
            assert rows[-1][1] >= blocks * MT > rows[-1][0]
            assert TH > THs and len(rows) >= 2
    TH, nbig, THs = big_small(67, 4)
    assert [(r1 - r0) // MT for r0, r1 in chunk_rows(67 * MT, TH, nbig, THs)] == [24, 24, 10, 10]


def test_model_has_teeth():
    # a range one level row short leaves rows unwritten; a lane offset one
    # column off leaves the first element unwritten (and spills each row's last
    # column into the next row)
    N, C, H, W, K, TH, eb = 1, 1, 64, 64, 11, 32, 2
    count, inside = level_writes(N, C, H, W, K, TH, eb)
    assert inside and count.min() >= 1
    count, _ = level_writes(N, C, H, W, K, TH, eb, short_rows=1)
    assert count.min() == 0
    count, _ = level_writes(N, C, H, W, K, TH, eb, col_shift=1)
    assert count.reshape(H // 2, W // 2)[0, 0] == 0
