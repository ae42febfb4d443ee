"""CPU model of the packed Prewitt arithmetic of the uint8 GMSD kernel
(fa_gmsd.hip: SrcU8Wide::samples_xy, prewitt_xy).

The kernel keeps the x and y samples of a sample column in one 32-bit
register (x in the low, y in the high 16 bits), forms the column sums with a
32-bit add and the row differences, gradients and their neighbour sums with
packed int16 operations that wrap per lane, then regathers [gx, gy] of each
tensor by a byte permute and takes its dot product with itself.  This model
replays exactly those operations with numpy's wrapping integer types and
checks the magnitudes against the direct Prewitt of 2x2 sums, on random and
extreme windows (every intermediate must stay inside int16 for the lanes not
to wrap into wrong values).
"""

from __future__ import annotations

import itertools

import numpy as np

M16 = 0xFFFF


def lanes(v):
    """uint32 -> (lo, hi) as int16."""
    v = np.asarray(v, dtype=np.uint32)
    return (v & M16).astype(np.uint16).view(np.int16), (v >> 16).astype(np.uint16).view(np.int16)


def pack(lo, hi):
    lo = np.asarray(lo).astype(np.int16).view(np.uint16).astype(np.uint32)
    hi = np.asarray(hi).astype(np.int16).view(np.uint16).astype(np.uint32)
    return lo | (hi << 16)


def pk_add(a, b):
    (al, ah), (bl, bh) = lanes(a), lanes(b)
    with np.errstate(over="ignore"):
        return pack(al + bl, ah + bh)


def pk_sub(a, b):
    (al, ah), (bl, bh) = lanes(a), lanes(b)
    with np.errstate(over="ignore"):
        return pack(al - bl, ah - bh)


def perm_lo(hi_src, lo_src):
    """v_perm_b32(hi_src, lo_src, 0x05040100): low halves of both."""
    return (np.asarray(lo_src, np.uint32) & M16) | ((np.asarray(hi_src, np.uint32) & M16) << 16)


def perm_hi(hi_src, lo_src):
    """v_perm_b32(hi_src, lo_src, 0x07060302): high halves of both."""
    return (np.asarray(lo_src, np.uint32) >> 16) | ((np.asarray(hi_src, np.uint32) >> 16) << 16)


def sdot2_self(v):
    lo, hi = lanes(v)
    return lo.astype(np.int64) ** 2 + hi.astype(np.int64) ** 2


def packed_magnitudes(sx, sy):
    """sx, sy: [..., 3 rows, 4 sample columns] 2x2 sums (the lane's two columns
    and the next lane's two).  Returns m1, m2 of the lane's two columns as the
    kernel forms them."""
    sx = np.asarray(sx, np.int64)
    sy = np.asarray(sy, np.int64)
    p = (sx + (sy << 16)).astype(np.uint64) & 0xFFFFFFFF
    p = p.astype(np.uint32)
    a, b, c = p[..., 0, :], p[..., 1, :], p[..., 2, :]
    cs = (a.astype(np.uint64) + b + c).astype(np.uint64) & 0xFFFFFFFF
    cs = cs.astype(np.uint32)
    rd = pk_sub(a, c)
    gx = [pk_sub(cs[..., 0], cs[..., 2]), pk_sub(cs[..., 1], cs[..., 3])]
    t = pk_add(rd[..., 1], rd[..., 2])
    gy = [pk_add(rd[..., 0], t), pk_add(t, rd[..., 3])]
    m1 = np.stack([sdot2_self(perm_lo(gy[k], gx[k])) for k in range(2)], -1)
    m2 = np.stack([sdot2_self(perm_hi(gy[k], gx[k])) for k in range(2)], -1)
    return m1, m2


def direct_magnitudes(s):
    s = np.asarray(s, np.int64)
    cs = s.sum(-2)                       # column sums over the three rows
    rd = s[..., 0, :] - s[..., 2, :]     # top minus bottom
    gx = cs[..., 0:2] - cs[..., 2:4]
    gy = rd[..., 0:2] + rd[..., 1:3] + rd[..., 2:4]
    return gx ** 2 + gy ** 2


def samples_from_bytes(img):
    """[..., 6 input rows, 8 input columns] uint8 -> [..., 3, 4] 2x2 sums, as
    the kernel forms them (byte dot products for x; for y the byte permute of
    two rows' pairs and the sum of its four bytes)."""
    img = np.asarray(img, np.int64)
    return img.reshape(img.shape[:-2] + (3, 2, 4, 2)).sum(axis=(-3, -1))


def test_packed_matches_direct_random():
    rng = np.random.default_rng(7)
    xb = rng.integers(0, 256, size=(20000, 6, 8))
    yb = rng.integers(0, 256, size=(20000, 6, 8))
    sx, sy = samples_from_bytes(xb), samples_from_bytes(yb)
    m1, m2 = packed_magnitudes(sx, sy)
    assert np.array_equal(m1, direct_magnitudes(sx))
    assert np.array_equal(m2, direct_magnitudes(sy))


def test_packed_matches_direct_extremes():
    # every sample at 0 or 1020 in each of a 3x4 window's positions (4096 x / y
    # combinations, paired in both orders): the largest gradients and row
    # differences of either sign
    pts = np.array(list(itertools.product([0, 1020], repeat=12)), np.int64).reshape(-1, 3, 4)
    rng = np.random.default_rng(3)
    other = pts[rng.permutation(len(pts))]
    for sx, sy in ((pts, other), (other, pts), (pts, pts)):
        m1, m2 = packed_magnitudes(sx, sy)
        assert np.array_equal(m1, direct_magnitudes(sx))
        assert np.array_equal(m2, direct_magnitudes(sy))
    # the largest magnitude stays below 2^24 (exact in float32)
    assert direct_magnitudes(pts).max() == 3060 ** 2 + 1020 ** 2 < 2 ** 24


def test_model_has_teeth():
    # samples beyond 16 bits would carry between the halves and wrap the int16
    # lanes: the model then disagrees with the direct form
    rng = np.random.default_rng(11)
    sx = rng.integers(30000, 60000, size=(1000, 3, 4))
    sy = rng.integers(0, 1021, size=(1000, 3, 4))
    m1, m2 = packed_magnitudes(sx, sy)
    assert not (np.array_equal(m1, direct_magnitudes(sx)) and np.array_equal(m2, direct_magnitudes(sy)))
