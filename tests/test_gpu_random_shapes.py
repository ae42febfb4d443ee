"""Parity of the headline kernels over seeded random shapes.

Each case draws a batch, channel count, height and width (some widths a
multiple of 8, which the matrix-core SSIM kernel takes, some not) and checks,
against the float64 oracle: SSIM per image within 1e-6 relative, uint8 MSE and
SSE-based PSNR bit-exact / to 1e-12, GMSD and GMS per image within 1e-6.  The
heights cover every remainder modulo 16, so the SSIM kernel's last row block
reads rows past the image (the range check of its loads turns them into
zeros) at every offset, and the chunk boundaries fall differently per case.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import frame_analytics_amd as fa
from oracle import reference as ref

pytestmark = pytest.mark.gpu

REL = 1e-6


def _case(seed):
    rng = np.random.default_rng(1000 + seed)
    n = int(rng.integers(1, 4))
    c = int(rng.choice([1, 3]))
    h = int(11 + seed % 16 + 16 * rng.integers(0, 12))
    w = int(rng.integers(2, 50)) * 8 + (0 if seed % 3 else int(rng.integers(1, 8)))
    a = rng.integers(0, 256, (n, c, h, w)).astype(np.float64)
    b = np.clip(a + rng.normal(0.0, 4.0 + seed, a.shape), 0, 255).round()
    # a smooth region too: flat patches keep the variance terms small
    a[..., : h // 3, : w // 3] = 100.0 + seed
    b[..., : h // 3, : w // 3] = 101.0 + seed
    return a.astype(np.uint8), b.astype(np.uint8)


@pytest.mark.parametrize("seed", range(16))
def test_random_shapes(gpu, seed):
    a, b = _case(seed)
    x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    shape = a.shape

    got = fa.ssim(x, y, data_range=255.0, reduction="none").cpu().numpy()
    want = ref.ssim(a, b, 255.0, reduction="none")
    assert np.all(np.abs(got - want) <= REL * np.abs(want)), (shape, got, want)

    assert np.array_equal(fa.mse(x, y, reduction="none").cpu().numpy(),
                          ref.mse(a, b, reduction="none")), shape
    pw = ref.psnr(a, b, 255.0, reduction="none")
    pg = fa.psnr(x, y, data_range=255.0, reduction="none").cpu().numpy()
    assert np.all(np.abs(pg - pw) <= 1e-12 * np.abs(pw)), (shape, pg, pw)

    if shape[-2] >= 6 and shape[-1] >= 6:
        m, s = ref.gmsd_stats(a, b, 255.0)
        gs = fa.gmsd(x, y, data_range=255.0, reduction="none").cpu().numpy()
        gm = fa.gms(x, y, data_range=255.0, reduction="none").cpu().numpy()
        assert np.all(np.abs(gs - s) <= REL * np.abs(s)), (shape, gs, s)
        assert np.all(np.abs(gm - m) <= REL * np.abs(m)), (shape, gm, m)


_FLOATS = [torch.float16, torch.bfloat16, torch.float32, torch.float64]


@pytest.mark.parametrize("seed", range(12))
def test_random_shapes_floating(gpu, seed):
    """Floating input over seeded random shapes, through the public calls,
    which hand the stream's accumulator to the one-launch finishes (the SSIM
    strip kernel's, GMSD's): a random dtype, sometimes a cropped view, and for
    three channels sometimes BT.601 luma formed in the kernel; SSIM and GMSD
    per image within 1e-6 of the oracle on the same (rounded) samples, and the
    accumulators zero afterwards."""
    from frame_analytics_amd import backend

    rng = np.random.default_rng(5000 + seed)
    a, b = _case(seed + 40)
    dt = _FLOATS[int(rng.integers(0, len(_FLOATS)))]
    x = torch.from_numpy(a).to(gpu).to(dt)
    y = torch.from_numpy(b).to(gpu).to(dt)
    if seed % 3 == 1 and x.shape[-2] > 20 and x.shape[-1] > 20:
        x, y = x[..., 2:-3, 1:-2], y[..., 2:-3, 1:-2]  # views, read in place
    luma = "bt601" if (x.shape[1] == 3 and seed % 2 == 0) else None
    xo, yo = x.double().cpu().numpy(), y.double().cpu().numpy()
    if luma:
        xo, yo = ref.rgb_to_luma(xo, "bt601"), ref.rgb_to_luma(yo, "bt601")
    got = fa.ssim(x, y, data_range=255.0, reduction="none", luma=luma).cpu().numpy()
    want = ref.ssim(xo, yo, 255.0, reduction="none")
    assert np.all(np.abs(got - want) <= REL * np.abs(want)), (dt, x.shape, luma, got, want)
    if x.shape[-2] >= 6 and x.shape[-1] >= 6:
        m, s = ref.gmsd_stats(xo, yo, 255.0)
        gs = fa.gmsd(x, y, data_range=255.0, reduction="none", luma=luma).cpu().numpy()
        gm = fa.gms(x, y, data_range=255.0, reduction="none", luma=luma).cpu().numpy()
        assert np.all(np.abs(gs - s) <= REL * np.abs(s)), (dt, x.shape, luma, gs, s)
        assert np.all(np.abs(gm - m) <= REL * np.abs(m)), (dt, x.shape, luma, gm, m)
    torch.cuda.synchronize()
    st = torch.cuda.current_stream().cuda_stream
    for kind in ("ssim", "gmsd"):
        acc = backend._stream_acc.get((kind, 0, st))
        assert acc is None or not bool(acc.any()), kind


@pytest.mark.parametrize("seed", range(10))
def test_random_uint8_views(gpu, seed):
    """uint8 views cut from larger frames at random offsets, read in place: a
    base aligned to 1, 2, 4 or 8 bytes, a width that is a multiple of 8 or
    not.  SSIM per image within 1e-6 of the oracle, PSNR to 1e-12; where the
    base is 4-byte aligned and the width a multiple of 8 the view takes the
    matrix-core kernel, as its contiguous copy does, and the two agree bit
    for bit."""
    rng = np.random.default_rng(7000 + seed)
    n = int(rng.integers(1, 3))
    c = int(rng.choice([1, 3]))
    H0 = int(rng.integers(30, 140))
    W0 = 8 * int(rng.integers(6, 40))
    a = rng.integers(0, 256, (n, c, H0, W0)).astype(np.float64)
    b = np.clip(a + rng.normal(0.0, 6.0, a.shape), 0, 255).round()
    a, b = a.astype(np.uint8), b.astype(np.uint8)
    top = int(rng.integers(0, 8))
    left = [0, 4, 2, 1, 4, 3, 0, 4, 6, 4][seed]
    w = W0 - left - int(rng.integers(0, 16))
    if seed % 2 == 0:
        w -= w % 8  # a multiple of 8
    h = H0 - top - int(rng.integers(0, 8))
    xv = torch.from_numpy(a).to(gpu)[..., top:top + h, left:left + w]
    yv = torch.from_numpy(b).to(gpu)[..., top:top + h, left:left + w]
    av, bv = a[..., top:top + h, left:left + w], b[..., top:top + h, left:left + w]
    got = fa.ssim(xv, yv, data_range=255.0, reduction="none").cpu().numpy()
    want = ref.ssim(av, bv, 255.0, reduction="none")
    assert np.all(np.abs(got - want) <= REL * np.abs(want)), (left, w, got, want)
    if left % 4 == 0 and w % 8 == 0:
        copy = fa.ssim(xv.contiguous(), yv.contiguous(), data_range=255.0,
                       reduction="none").cpu().numpy()
        assert np.array_equal(got, copy), (left, w, got, copy)
    pw = ref.psnr(av, bv, 255.0, reduction="none")
    pg = fa.psnr(xv, yv, data_range=255.0, reduction="none").cpu().numpy()
    assert np.all(np.abs(pg - pw) <= 1e-12 * np.abs(pw)), (left, w, pg, pw)
