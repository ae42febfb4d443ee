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
