"""Pins the float64 oracle before anything is compared against it.

Every function of oracle/reference.py is checked here against something that
does not share its code: a direct 121-tap correlation, scipy, brute-force
per-pixel loops, torch library routines, float64 autograd, central differences,
closed forms, and the reference's own CPU C++ kernels (oracle/_ref, compiled
from the reference sources; golden values they produced are committed under
tests/golden/ for runs where the library is not built).
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ref_cpu
from oracle import reference as ref
from tests.conftest import natural_pair, u8_pair

GOLDEN = Path(__file__).resolve().parent / "golden" / "ref_cpu_vectors.json"


# --------------------------------------------------------------------------- #
# windows and correlation
# --------------------------------------------------------------------------- #


@pytest.mark.parametrize("k,s", [(11, 1.5), (7, 2.0), (3, 0.5), (5, 1.0)])
def test_window_2d_is_outer_product_and_normalised(k, s):
    w1 = ref.gaussian_window_1d(k, s)
    w2 = ref.gaussian_window_2d(k, s)
    assert abs(w1.sum() - 1.0) < 1e-15 and abs(w2.sum() - 1.0) < 1e-15
    assert np.abs(np.outer(w1, w1) - w2).max() < 1e-15
    assert np.allclose(w1, w1[::-1], rtol=0, atol=0)  # symmetric
    # closed form of the centre tap ratio: w(0)/w(1) = exp(1/(2 s^2))
    c = (k - 1) // 2
    assert abs(w1[c] / w1[c + 1] - math.exp(1.0 / (2 * s * s))) < 1e-12


def test_separable_equals_direct_and_scipy():
    scipy_signal = pytest.importorskip("scipy.signal")
    rng = np.random.default_rng(0)
    img = rng.random((2, 23, 31)) * 255
    w = ref.gaussian_window_1d(11, 1.5)
    k2 = np.outer(w, w)
    sep = ref.separable_valid(img, w)
    direct = ref.valid_correlate2d(img, k2)
    assert np.abs(sep - direct).max() < 1e-11
    for i in range(2):
        sp = scipy_signal.correlate2d(img[i], k2, mode="valid")
        assert np.abs(direct[i] - sp).max() < 1e-11


def _ssim_brute(x, y, L, k=11, s=1.5, K=(0.01, 0.03)):
    """Per-pixel SSIM from its definition with explicit loops (tiny inputs)."""
    w = ref.gaussian_window_2d(k, s)
    C1, C2 = (K[0] * L) ** 2, (K[1] * L) ** 2
    oh, ow = x.shape[0] - k + 1, x.shape[1] - k + 1
    out = np.zeros((oh, ow))
    for i in range(oh):
        for j in range(ow):
            px, py = x[i:i + k, j:j + k], y[i:i + k, j:j + k]
            mx, my = (w * px).sum(), (w * py).sum()
            vx = (w * (px - mx) ** 2).sum()
            vy = (w * (py - my) ** 2).sum()
            cxy = (w * (px - mx) * (py - my)).sum()
            out[i, j] = ((2 * mx * my + C1) * (2 * cxy + C2)
                         / ((mx * mx + my * my + C1) * (vx + vy + C2)))
    return out


def test_ssim_map_equals_brute_force_definition():
    a, b = natural_pair(19, 24, 12.0, seed=5)
    got, _ = ref.ssim_maps(a, b, 255.0)
    want = _ssim_brute(a, b, 255.0)
    assert np.abs(got - want).max() < 1e-12


def test_ssim_identity_and_symmetry():
    a, b = natural_pair(40, 50, 8.0, seed=2)
    s, cs = ref.ssim_maps(a, a, 255.0)
    assert np.abs(s - 1).max() < 1e-14 and np.abs(cs - 1).max() < 1e-14
    s1, _ = ref.ssim_maps(a, b, 255.0)
    s2, _ = ref.ssim_maps(b, a, 255.0)
    assert np.abs(s1 - s2).max() < 1e-14


def test_ssim_batch_conventions():
    a, b = u8_pair((3, 2, 30, 40), 10.0, seed=1)
    per = ref.ssim(a, b, 255.0, reduction="none")
    for i in range(3):
        planes = [ref.ssim_maps(a[i, c], b[i, c], 255.0)[0].mean() for c in range(2)]
        assert abs(per[i] - np.mean(planes)) < 1e-14
    assert abs(ref.ssim(a, b, 255.0) - per.mean()) < 1e-15


# --------------------------------------------------------------------------- #
# pixel losses
# --------------------------------------------------------------------------- #


def test_sse_sad_exact_against_python_ints():
    a, b = u8_pair((2, 1, 17, 23), 30.0, seed=4)
    for i in range(2):
        da = [int(p) - int(q) for p, q in zip(a[i].ravel(), b[i].ravel())]
        assert ref.sse_u8(a, b, per_image=True)[i] == sum(d * d for d in da)
        assert ref.sad_u8(a, b, per_image=True)[i] == sum(abs(d) for d in da)
    # chunking does not change an exact sum
    assert ref.sse_u8(a, b, chunk=7) == ref.sse_u8(a, b)


def test_mse_psnr_closed_forms():
    a, b = u8_pair((2, 3, 20, 20), 9.0, seed=8)
    m = ref.mse(a, b)
    assert m == ref.sse_u8(a, b) / a.size
    assert abs(ref.mse(a, b) - ((a.astype(float) - b) ** 2).mean()) < 1e-12
    assert abs(ref.psnr(a, b, 255.0) - 10 * math.log10(255.0 ** 2 / m)) < 1e-12
    assert ref.psnr(a, a, 255.0) == float("inf")
    per = ref.mse(a, b, "none")
    assert abs(per.mean() - m) < 1e-12


def test_pixel_losses_against_torch():
    rng = np.random.default_rng(3)
    a = rng.random((2, 3, 9, 11)) * 4
    b = rng.random((2, 3, 9, 11)) * 4
    ta, tb = torch.from_numpy(a), torch.from_numpy(b)
    for delta in (0.5, 1.0, 2.5):
        assert abs(ref.huber(a, b, delta) - float(F.huber_loss(ta, tb, delta=delta))) < 1e-14
    assert abs(ref.l1(a, b) - float(F.l1_loss(ta, tb))) < 1e-14
    assert abs(ref.mse(a, b) - float(F.mse_loss(ta, tb))) < 1e-14
    assert abs(ref.charbonnier(a, a, eps=0.25) - 0.25) < 1e-15
    big = ref.charbonnier(a, b, eps=1e-9)
    assert abs(big - ref.l1(a, b)) < 1e-8  # eps -> 0 reduces to L1


def test_luma_closed_form():
    px = np.array([[[[10.0]], [[200.0]], [[30.0]]]])  # (1, 3, 1, 1)
    assert ref.rgb_to_luma(px, "bt601")[0, 0, 0, 0] == pytest.approx(0.299 * 10 + 0.587 * 200 + 0.114 * 30)
    assert ref.rgb_to_luma(px, "matlab", 255.0)[0, 0, 0, 0] == pytest.approx(
        (65.481 * 10 + 128.553 * 200 + 24.966 * 30) / 255.0 + 16.0)


# --------------------------------------------------------------------------- #
# MS-SSIM / GMSD
# --------------------------------------------------------------------------- #


def test_avg_pool_equals_torch():
    rng = np.random.default_rng(1)
    for shape in [(1, 2, 9, 12), (2, 1, 10, 7)]:
        x = rng.random(shape)
        want = F.avg_pool2d(torch.from_numpy(x), 2).numpy()
        assert np.abs(ref.avg_pool2(x) - want).max() < 1e-15


def test_ms_ssim_special_cases():
    a, b = u8_pair((2, 2, 44, 52), 12.0, seed=6)
    s0 = ref.ssim(a, b, 255.0, reduction="none")
    # one scale with weight 1 is plain SSIM per plane, channels averaged after
    per = ref.ms_ssim(a, b, 255.0, weights=(1.0,), reduction="none")
    assert np.abs(per - s0).max() < 1e-14
    # (1, 0): the first scale's cs alone
    _, cs0 = ref.ssim_maps(a.astype(float), b.astype(float), 255.0)
    want = np.maximum(cs0.mean(axis=(-2, -1)), 0).mean(axis=1)
    assert np.abs(ref.ms_ssim(a, b, 255.0, weights=(1.0, 0.0), reduction="none") - want).max() < 1e-14
    # identity
    assert abs(ref.ms_ssim(a, a, 255.0, weights=(0.5, 0.5)) - 1.0) < 1e-14


def _photo_pair(h, w, seed, noise):
    """Smooth texture plus noise, the style of the reference's MS-SSIM tests
    (test_training_metrics.py:30-36)."""
    rng = np.random.default_rng(seed)
    yy, xx = np.mgrid[0:h, 0:w].astype(np.float64)
    a = np.clip(120 + 50 * np.sin(xx / 11.0) * np.cos(yy / 13.0)
                + 12 * rng.standard_normal((h, w)), 0, 255).round()
    b = np.clip(a + noise * rng.standard_normal((h, w)), 0, 255).round()
    return a, b


def test_ms_ssim_channels_averaged_after_the_product():
    """The reference's own case (test_training_metrics.py:97-110): a 2-channel
    MS-SSIM equals the mean of the two 1-channel values.  Averaging the
    per-scale terms over channels before the product gives a different
    number, so the check can tell the two conventions apart."""
    a1, b1 = _photo_pair(184, 200, seed=21, noise=8.0)
    a2, b2 = _photo_pair(184, 200, seed=22, noise=30.0)
    r1 = ref.ms_ssim(a1[None, None], b1[None, None], 255.0)
    r2 = ref.ms_ssim(a2[None, None], b2[None, None], 255.0)
    x = np.stack([a1, a2])[None]
    y = np.stack([b1, b2])[None]
    got = ref.ms_ssim(x, y, 255.0)
    assert abs(got - 0.5 * (r1 + r2)) < 1e-15
    # negative control: the channel mean taken first, per scale
    terms = ref.ms_ssim_terms(x, y, 255.0)
    w = ref.MS_SSIM_WEIGHTS
    first = 1.0
    for i, wi in enumerate(w):
        v = terms[i][0] if i == len(w) - 1 else terms[i][1]
        first *= max(float(v.mean()), 0.0) ** wi
    assert abs(first - got) > 1e-4, (first, got)


def test_ms_ssim_coarsest_scale_alone_is_ssim_of_the_fourth_pool():
    """weights (0, 0, 0, 0, 1) leave only the full SSIM at scale 4: the SSIM of
    the pair pooled four times by torch's avg_pool2d (which drops an odd
    trailing row / column).  A pyramid one level too shallow or too deep, or
    cs in place of SSIM at the last scale, fails this."""
    a, b = u8_pair((2, 2, 181, 199), 10.0, seed=31)
    b = np.clip(b.astype(np.int32) + 40, 0, 255).astype(np.uint8)  # a luminance gap
    tx = torch.from_numpy(a.astype(np.float64))
    ty = torch.from_numpy(b.astype(np.float64))
    pooled = []
    for _ in range(4):
        tx, ty = F.avg_pool2d(tx, 2), F.avg_pool2d(ty, 2)
        pooled.append((tx.numpy(), ty.numpy()))
    assert tuple(tx.shape[-2:]) == (11, 12)
    want = ref.ssim(tx.numpy(), ty.numpy(), 255.0, reduction="none")
    got = ref.ms_ssim(a, b, 255.0, weights=(0, 0, 0, 0, 1), reduction="none")
    assert np.abs(got - want).max() < 1e-14
    # negative controls: cs in place of SSIM at the coarsest scale, and a
    # pyramid one level shallower, are measurably different
    _, cs4 = ref.ssim_maps(tx.numpy(), ty.numpy(), 255.0)
    assert np.abs(cs4.mean(axis=(-2, -1)).mean(axis=1) - got).max() > 1e-3
    s3 = ref.ssim(*pooled[2], 255.0, reduction="none")
    assert np.abs(s3 - got).max() > 1e-3


def test_ms_ssim_clamps_anti_correlated_content_to_zero():
    """y = 255 - x makes cs at scale 0 negative (sigma_xy = -sigma_x^2); the
    clamp at zero (reference functional.py:893-896) makes the product exactly
    0, where the unclamped fractional power is not real."""
    a, _ = u8_pair((1, 1, 176, 180), 8.0, seed=41)
    b = 255 - a
    terms = ref.ms_ssim_terms(a, b, 255.0)
    assert float(terms[0][1].min()) < -0.5
    assert ref.ms_ssim(a, b, 255.0) == 0.0
    with np.errstate(invalid="ignore"):
        assert np.isnan(np.power(terms[0][1][0, 0], ref.MS_SSIM_WEIGHTS[0]))


def _ms_fd(x, y, i, j, n=0, c=0, h=1e-4, **kw):
    xp, xm = x.copy(), x.copy()
    xp[n, c, i, j] += h
    xm[n, c, i, j] -= h
    return (ref.ms_ssim(xp, y, **kw) - ref.ms_ssim(xm, y, **kw)) / (2 * h)


@pytest.mark.parametrize("shape,kw", [
    ((2, 2, 180, 192), {}),
    ((1, 3, 64, 70), {"win_size": 7, "weights": (0.3, 0.7)}),
])
def test_ms_ssim_grad_central_differences(shape, kw):
    """The closed-form MS-SSIM adjoint (clamp, product, channel and batch
    means, pyramid) against central differences of the float64 forward, at
    pixels in different images and channels, inside the valid grid of every
    scale and in a dropped odd trailing row / column."""
    rng = np.random.default_rng(7)
    x = rng.random(shape)
    y = np.clip(x + 0.05 * rng.standard_normal(shape), 0, 1)
    opts = dict(data_range=1.0, **kw)
    gx, gy = ref.ms_ssim_grad(x, y, **opts)
    H, W = shape[-2:]
    pts = [(0, 0, 40, 60), (shape[0] - 1, shape[1] - 1, H // 2, W // 3),
           (0, shape[1] - 1, 3, W - 5), (shape[0] - 1, 0, H - 1, 7)]
    scale = np.abs(gx).max()
    for n, c, i, j in pts:
        fd = _ms_fd(x, y, i, j, n, c, **opts)
        assert abs(fd - gx[n, c, i, j]) <= 2e-7 * scale, (n, c, i, j, fd, gx[n, c, i, j])
    # d/dy by symmetry of the formula in (x, y): the swapped call's dx
    gy2, _ = ref.ms_ssim_grad(y, x, **opts)
    assert np.abs(gy - gy2).max() <= 1e-12 * scale
    n, c, i, j = pts[1]
    yp, ym = y.copy(), y.copy()
    yp[n, c, i, j] += 1e-4
    ym[n, c, i, j] -= 1e-4
    fd = (ref.ms_ssim(x, yp, **opts) - ref.ms_ssim(x, ym, **opts)) / 2e-4
    assert abs(fd - gy[n, c, i, j]) <= 2e-7 * scale


def test_ms_ssim_grad_upstream_and_clamped_planes():
    """A per-image upstream vector scales each image's gradient, and a plane
    whose scale-0 cs is clamped contributes no gradient at all."""
    rng = np.random.default_rng(8)
    x = rng.random((2, 1, 176, 176))
    y = np.clip(x + 0.05 * rng.standard_normal(x.shape), 0, 1)
    y[1] = 1.0 - x[1]  # anti-correlated: clamped to 0
    gx, _ = ref.ms_ssim_grad(x, y, data_range=1.0, upstream=np.array([3.0, 5.0]))
    g0, _ = ref.ms_ssim_grad(x[:1], y[:1], data_range=1.0, upstream=np.array([1.0]))
    assert np.abs(gx[0] - 3.0 * g0[0]).max() <= 1e-12 * np.abs(g0).max()
    assert np.abs(gx[1]).max() == 0.0


def test_gmsd_against_torch_conv_and_identity():
    a, b = natural_pair(40, 46, 9.0, seed=9)
    x4, y4 = a[None, None], b[None, None]
    m, s = ref.gmsd_stats(x4, y4, 255.0, downsample=True)
    kx = torch.tensor([[1.0, 0.0, -1.0]] * 3, dtype=torch.float64) / 3.0
    k = torch.stack([kx, kx.t()]).unsqueeze(1)
    tx = F.avg_pool2d(torch.from_numpy(x4), 2)
    ty = F.avg_pool2d(torch.from_numpy(y4), 2)
    eps = (1e-6 * 255.0) ** 2
    g1 = torch.sqrt((F.conv2d(tx, k) ** 2).sum(1) + eps)
    g2 = torch.sqrt((F.conv2d(ty, k) ** 2).sum(1) + eps)
    q = (2 * g1 * g2 + 170.0) / (g1 * g1 + g2 * g2 + 170.0)
    assert abs(float(q.mean()) - m[0]) < 1e-14
    assert abs(float(q.std(unbiased=False)) - s[0]) < 1e-13
    mi, si = ref.gmsd_stats(x4, x4, 255.0)
    assert mi[0] == 1.0 and si[0] == 0.0


def _gmsd_decimal(x, y, L, down, digits=40):
    """Per-pixel GMS statistics of one plane in 40-digit decimal arithmetic."""
    import decimal

    ctx = decimal.Context(prec=digits)
    D = lambda v: decimal.Decimal(float(v))  # noqa: E731  exact binary value
    X = [[D(v) for v in row] for row in x]
    Y = [[D(v) for v in row] for row in y]
    if down:
        q4 = decimal.Decimal(4)
        pool = lambda A: [[ctx.divide(A[2 * i][2 * j] + A[2 * i][2 * j + 1] + A[2 * i + 1][2 * j]  # noqa: E731
                                      + A[2 * i + 1][2 * j + 1], q4)
                           for j in range(len(A[0]) // 2)] for i in range(len(A) // 2)]
        X, Y = pool(X), pool(Y)
    T = D(170.0 * (L / 255.0) ** 2)
    eps = D((1e-6 * L) ** 2)
    three = decimal.Decimal(3)

    def grad(A, i, j):
        gx = sum(A[i + r][j] - A[i + r][j + 2] for r in range(3))
        gy = sum(A[i][j + c] - A[i + 2][j + c] for c in range(3))
        gx, gy = ctx.divide(gx, three), ctx.divide(gy, three)
        return ctx.sqrt(gx * gx + gy * gy + eps)

    qs = []
    for i in range(len(X) - 2):
        for j in range(len(X[0]) - 2):
            g1, g2 = grad(X, i, j), grad(Y, i, j)
            qs.append(ctx.divide(2 * g1 * g2 + T, g1 * g1 + g2 * g2 + T))
    n = decimal.Decimal(len(qs))
    m = ctx.divide(sum(qs), n)
    var = ctx.divide(sum((q - m) * (q - m) for q in qs), n)
    return m, ctx.sqrt(var)


def test_gmsd_stats_hp_pinned():
    """gmsd_stats_hp equals gmsd_stats where both are accurate, and matches a
    40-digit brute force on nearly identical images, where gmsd_stats' float64
    q (rounded near 1) is not."""
    for kind in ("natural", "uniform"):
        a, b = natural_pair(29, 34, 9.0, seed=4, kind=kind)
        for down in (True, False):
            m0, s0 = ref.gmsd_stats(a[None, None], b[None, None], 255.0, downsample=down)
            m1, s1 = ref.gmsd_stats_hp(a[None, None], b[None, None], 255.0, downsample=down)
            assert abs(m0[0] - m1[0]) < 1e-14 and abs(s0[0] / s1[0] - 1) < 1e-12
    rng = np.random.default_rng(11)
    for down, shape in ((False, (8, 9)), (True, (12, 14))):
        x = rng.random(shape)
        y = x + 1e-7 * rng.standard_normal(shape)
        dm, ds = _gmsd_decimal(x, y, 1.0, down)
        m, sd = ref.gmsd_stats_hp(x[None, None], y[None, None], 1.0, downsample=down)
        assert abs(m[0] - float(dm)) < 1e-15
        assert abs(sd[0] / float(ds) - 1) < 1e-9
    mi, si = ref.gmsd_stats_hp(x[None, None], x[None, None], 1.0)
    assert mi[0] == 1.0 and si[0] == 0.0


# --------------------------------------------------------------------------- #
# SSIM gradient
# --------------------------------------------------------------------------- #


def _torch_ssim_mean(x, y, L, k=11, s=1.5):
    """Independent float64 torch SSIM (2-D window, five convolutions)."""
    w2 = torch.from_numpy(ref.gaussian_window_2d(k, s))[None, None]
    n, c, h, wd = x.shape
    X, Y = x.reshape(n * c, 1, h, wd), y.reshape(n * c, 1, h, wd)
    mx, my = F.conv2d(X, w2), F.conv2d(Y, w2)
    vx = F.conv2d(X * X, w2) - mx * mx
    vy = F.conv2d(Y * Y, w2) - my * my
    cxy = F.conv2d(X * Y, w2) - mx * my
    C1, C2 = (0.01 * L) ** 2, (0.03 * L) ** 2
    smap = (2 * mx * my + C1) * (2 * cxy + C2) / ((mx * mx + my * my + C1) * (vx + vy + C2))
    return smap.mean()


def test_ssim_grad_against_autograd64():
    rng = np.random.default_rng(4)
    x = rng.random((2, 2, 30, 34))
    y = np.clip(x + 0.05 * rng.standard_normal(x.shape), 0, 1)
    tx = torch.from_numpy(x).requires_grad_(True)
    ty = torch.from_numpy(y).requires_grad_(True)
    _torch_ssim_mean(tx, ty, 1.0).backward()
    gx, gy = ref.ssim_mean_grad(x, y, 1.0)
    assert float((torch.from_numpy(gx) - tx.grad).abs().max() / tx.grad.abs().max()) < 1e-10
    assert float((torch.from_numpy(gy) - ty.grad).abs().max() / ty.grad.abs().max()) < 1e-10


def test_ssim_grad_against_central_differences():
    rng = np.random.default_rng(1)
    x = rng.random((1, 1, 26, 29))
    y = np.clip(x + 0.05 * rng.standard_normal(x.shape), 0, 1)
    gx, _ = ref.ssim_mean_grad(x, y, 1.0)
    # h = 1e-4 balances the O(h^2) truncation against float64 cancellation
    # (the mean SSIM moves by ~1e-9 per 1e-6 step at a corner pixel); the
    # bound is max-normwise, like every gradient comparison in this suite
    h = 1e-4
    scale = np.abs(gx).max()
    for (i, j) in [(0, 0), (5, 7), (13, 14), (25, 28), (10, 3)]:
        xp, xm = x.copy(), x.copy()
        xp[0, 0, i, j] += h
        xm[0, 0, i, j] -= h
        fd = (ref.ssim(xp, y, 1.0) - ref.ssim(xm, y, 1.0)) / (2 * h)
        assert abs(fd - gx[0, 0, i, j]) <= 1e-6 * scale, (i, j, fd, gx[0, 0, i, j])


def test_ssim_grad_map_upstream():
    rng = np.random.default_rng(2)
    x = rng.random((1, 1, 20, 21))
    y = np.clip(x + 0.05 * rng.standard_normal(x.shape), 0, 1)
    up = rng.random((1, 1, 10, 11))
    tx = torch.from_numpy(x).requires_grad_(True)
    w2 = torch.from_numpy(ref.gaussian_window_2d())[None, None]
    ty = torch.from_numpy(y)
    mx, my = F.conv2d(tx, w2), F.conv2d(ty, w2)
    vx = F.conv2d(tx * tx, w2) - mx * mx
    vy = F.conv2d(ty * ty, w2) - my * my
    cxy = F.conv2d(tx * ty, w2) - mx * my
    C1, C2 = 1e-4, 9e-4
    smap = (2 * mx * my + C1) * (2 * cxy + C2) / ((mx * mx + my * my + C1) * (vx + vy + C2))
    (smap * torch.from_numpy(up)).sum().backward()
    gx, _ = ref.ssim_mean_grad(x, y, 1.0, upstream=up)
    assert float((torch.from_numpy(gx) - tx.grad).abs().max() / tx.grad.abs().max()) < 1e-10


# --------------------------------------------------------------------------- #
# against the reference's own CPU C++ (live if built, golden values otherwise)
# --------------------------------------------------------------------------- #


def _golden():
    return json.loads(GOLDEN.read_text())


def _golden_inputs(case):
    if case["gen"] == "natural":
        a, b = natural_pair(case["h"], case["w"], case["noise"], seed=case["seed"], kind=case["kind"])
        return a.astype(np.uint8)[None, None], b.astype(np.uint8)[None, None]
    a, b = u8_pair(tuple(case["shape"]), case["sigma"], seed=case["seed"])
    return a, b


def test_oracle_against_reference_cpu_golden():
    """Golden values from the reference CPU kernels (tests/golden/make_golden.py):
    SSIM / MS-SSIM scale terms / GMSD within the reference's 5e-6 gate (its
    kernels are float32), MSE exactly (integer sums both sides)."""
    g = _golden()
    for case in g["cases"]:
        a, b = _golden_inputs(case)
        exp = case["expect"]
        assert ref.mse(a, b) == exp["mse"]
        assert abs(ref.l1(a, b) - exp["l1"]) == 0.0
        per = ref.ssim(a, b, 255.0, reduction="none")
        assert np.abs(per - np.array(exp["ssim_per_image"])).max() < 5e-6
        if "ssim_cs" in exp:
            s, cs = ref.ms_ssim_terms(a, b, 255.0, scales=1)[0]
            assert np.abs(s - np.array(exp["ssim_cs"][0])).max() < 5e-6
            assert np.abs(cs - np.array(exp["ssim_cs"][1])).max() < 5e-6
        if "gmsd" in exp:
            m, sd = ref.gmsd_stats(a, b, 255.0)
            assert np.abs(m - np.array(exp["gmsd"][0])).max() < 5e-6
            assert np.abs(sd - np.array(exp["gmsd"][1])).max() < 5e-6


@pytest.mark.skipif(not ref_cpu.available(), reason="oracle/_ref not built")
def test_oracle_against_reference_cpu_live():
    for h, w, kind, noise in [(64, 64, "uniform", 20.0), (127, 233, "natural", 8.0),
                              (33, 41, "flat", 5.0), (200, 232, "natural", 8.0)]:
        a, b = natural_pair(h, w, noise, seed=h * w, kind=kind)
        a8, b8 = a.astype(np.uint8)[None, None], b.astype(np.uint8)[None, None]
        assert ref_cpu.pixel_reduce(a8, b8, "mse") == ref.mse(a8, b8)
        assert ref_cpu.pixel_reduce(a8, b8, "l1") == ref.l1(a8, b8)
        got = ref_cpu.ssim_per_image(a8, b8)
        assert abs(got[0] - ref.ssim(a8, b8, 255.0)) < 5e-6
        s, cs = ref_cpu.ssim_cs(a8, b8)
        os_, ocs = ref.ms_ssim_terms(a8, b8, 255.0, scales=1)[0]
        assert abs(s[0, 0] - os_[0, 0]) < 5e-6 and abs(cs[0, 0] - ocs[0, 0]) < 5e-6
        for down in (True, False):
            m, sd = ref_cpu.gmsd(a8, b8, downsample=down)
            om, osd = ref.gmsd_stats(a8, b8, 255.0, downsample=down)
            assert abs(m[0] - om[0]) < 5e-6 and abs(sd[0] - osd[0]) < 5e-6
        for eps in (1e-3, 3.0):
            assert abs(ref_cpu.pixel_reduce(a8, b8, "charbonnier", eps * eps)
                       - ref.charbonnier(a8, b8, eps)) < 1e-6 * ref.charbonnier(a8, b8, eps)
        for delta in (1.0, 4.0):
            assert abs(ref_cpu.pixel_reduce(a8, b8, "huber", delta)
                       - ref.huber(a8, b8, delta)) < 1e-6 * max(ref.huber(a8, b8, delta), 1e-12)


@pytest.mark.parametrize("down", [True, False])
def test_gms_stats_grad_central_differences(down):
    """The analytic GMS / GMSD gradient against central differences of the
    float64 forward, for a mixed upstream on both statistics (odd sizes, so
    the dropped row / column is exercised)."""
    rng = np.random.default_rng(3)
    x = rng.uniform(0, 255, (2, 2, 13, 15))
    y = np.clip(x + rng.normal(0, 20, x.shape), 0, 255)
    gm, gs = np.array([0.7, -1.3]), np.array([2.1, 0.4])

    def loss(a, b):
        m, s = ref.gmsd_stats(a, b, 255.0, downsample=down)
        return float((gm * m + gs * s).sum())

    dx, dy = ref.gms_stats_grad(x, y, 255.0, downsample=down, g_mean=gm, g_std=gs)
    h = 1e-3
    for arr, grad, other_first in ((x, dx, True), (y, dy, False)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            p, mm = arr.copy(), arr.copy()
            p[idx] += h
            mm[idx] -= h
            fp = loss(p, y) if other_first else loss(x, p)
            fm = loss(mm, y) if other_first else loss(x, mm)
            num[idx] = (fp - fm) / (2 * h)
        err = np.abs(num - grad).max() / np.abs(num).max()
        assert err < 1e-6, err
    if down:  # the dropped odd row / column gets no gradient
        assert np.all(dx[..., 12, :] == 0) and np.all(dx[..., :, 14] == 0)

