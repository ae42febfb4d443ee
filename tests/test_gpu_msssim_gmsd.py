"""GPU parity of MS-SSIM (value and gradient) and GMSD / GMS.

Bar: values within 1e-6 relative of float64; gradients 1e-6 max-normwise
relative (the MS-SSIM pyramid is exact, see fa_pool.hip).  Where the true value
is zero (GMSD of identical frames) the bar is the reference's absolute one.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import frame_analytics_amd as fa
from oracle import reference as ref
from tests.conftest import float_pair, natural_pair, u8_pair

pytestmark = pytest.mark.gpu

REL = 1e-6


def _rel(got, want):
    return abs(got - want) / max(abs(want), 1e-12)


def _plane_pair(h=200, w=232, seed=11, noise=7.0):
    """Smooth texture plus noise (reference test_training_metrics.py:30-36 style)."""
    rng = np.random.default_rng(seed)
    yy, xx = np.mgrid[0:h, 0:w].astype(np.float64)
    a = np.clip(120 + 50 * np.sin(xx / 11.0) * np.cos(yy / 13.0)
                + 12 * rng.standard_normal((h, w)), 0, 255).round()
    b = np.clip(a + noise * rng.standard_normal((h, w)), 0, 255).round()
    return a, b


# --------------------------------------------------------------------------- #
# MS-SSIM
# --------------------------------------------------------------------------- #


@pytest.mark.parametrize("dt", [torch.uint8, torch.float32, torch.float64])
@pytest.mark.parametrize("hw", [(200, 232), (257, 193), (176, 176)])
def test_ms_ssim_matches_oracle(gpu, dt, hw):
    a, b = _plane_pair(*hw, seed=hw[0] + hw[1])
    want = ref.ms_ssim(a[None, None], b[None, None], 255.0)
    x = torch.as_tensor(a, dtype=dt, device=gpu)[None, None]
    y = torch.as_tensor(b, dtype=dt, device=gpu)[None, None]
    got = float(fa.ms_ssim(x, y, data_range=255.0))
    assert _rel(got, want) <= REL, (dt, got, want)


def test_ms_ssim_batch_channels_identity(gpu):
    a, b = u8_pair((3, 3, 192, 208), 10.0, seed=4)
    x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    per = fa.ms_ssim(x, y, data_range=255.0, reduction="none").cpu().numpy()
    want = ref.ms_ssim(a, b, 255.0, reduction="none")
    assert per.shape == (3,)
    assert np.all(np.abs(per - want) <= REL * np.abs(want))
    assert abs(float(fa.ms_ssim(x, x, data_range=255.0)) - 1.0) < 1e-7
    w = (0.4, 0.6)
    assert _rel(float(fa.ms_ssim(x, y, data_range=255.0, weights=w)),
                ref.ms_ssim(a, b, 255.0, weights=w)) <= REL


def test_ms_ssim_configs4_full_size(gpu):
    """configs[4] MS-SSIM: 8x3x1080x1920 uint8; image 0 against the oracle,
    the batch by per-image consistency."""
    a, b = u8_pair((8, 3, 1080, 1920), 8.0, seed=1)
    x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    per = fa.ms_ssim(x, y, data_range=255.0, reduction="none").cpu().numpy()
    want0 = ref.ms_ssim(a[:1], b[:1], 255.0)
    assert _rel(float(per[0]), want0) <= REL, (per[0], want0)
    assert abs(float(fa.ms_ssim(x[3:4], y[3:4], data_range=255.0)) - float(per[3])) < 1e-12
    assert abs(float(fa.ms_ssim(x, y, data_range=255.0)) - float(per.mean())) < 1e-12


def test_ms_ssim_too_small(gpu):
    x = torch.zeros(1, 1, 175, 300, device=gpu)
    with pytest.raises(ValueError, match="too small"):
        fa.ms_ssim(x, x, data_range=1.0)
    z = torch.zeros(1, 1, 176, 300, device=gpu)
    assert float(fa.ms_ssim(z, z, data_range=1.0)) == pytest.approx(1.0)


@pytest.mark.parametrize("shape", [(1, 1, 192, 192), (2, 3, 180, 200)])
@pytest.mark.parametrize("wrt", [("x",), ("x", "y")])
def test_ms_ssim_backward_matches_autograd64(gpu, shape, wrt):
    """dL/dx of 1 - ms_ssim against float64 autograd over the portable path."""
    xa, ya = float_pair(shape, 0.05, seed=shape[-1])

    def grads(device, dtype, hint):
        x = torch.from_numpy(xa).to(device, dtype).requires_grad_("x" in wrt)
        y = torch.from_numpy(ya).to(device, dtype).requires_grad_("y" in wrt)
        (1.0 - fa.ms_ssim(x, y, data_range=1.0, backend_hint=hint)).backward()
        return x.grad, y.grad

    nat = grads(gpu, torch.float32, "auto")
    want = grads("cpu", torch.float64, "torch")
    for n, r in zip(nat, want):
        assert (n is None) == (r is None)
        if r is None:
            continue
        err = float((n.double().cpu() - r).abs().max() / r.abs().max())
        assert err <= REL, err


# --------------------------------------------------------------------------- #
# GMSD / GMS
# --------------------------------------------------------------------------- #


@pytest.mark.parametrize("down", [True, False])
@pytest.mark.parametrize("dt", [torch.uint8, torch.float32])
def test_gmsd_matches_oracle(gpu, down, dt):
    a, b = _plane_pair()
    m, s = ref.gmsd_stats(a[None, None], b[None, None], 255.0, downsample=down)
    x = torch.as_tensor(a, dtype=dt, device=gpu)[None, None]
    y = torch.as_tensor(b, dtype=dt, device=gpu)[None, None]
    assert _rel(float(fa.gmsd(x, y, data_range=255.0, downsample=down)), float(s[0])) <= REL
    assert _rel(float(fa.gms(x, y, data_range=255.0, downsample=down)), float(m[0])) <= REL


@pytest.mark.parametrize("hw", [(157, 203), (64, 65), (7, 9), (1080, 1920)])
def test_gmsd_sizes(gpu, hw):
    a, b = natural_pair(*hw, noise=9.0, seed=hw[0])
    m, s = ref.gmsd_stats(a[None, None], b[None, None], 255.0)
    x = torch.as_tensor(a, dtype=torch.uint8, device=gpu)[None, None]
    y = torch.as_tensor(b, dtype=torch.uint8, device=gpu)[None, None]
    assert _rel(float(fa.gmsd(x, y, data_range=255.0)), float(s[0])) <= REL
    assert _rel(float(fa.gms(x, y, data_range=255.0)), float(m[0])) <= REL


def test_gmsd_batch_channels(gpu):
    a, b = u8_pair((3, 3, 130, 150), 15.0, seed=8)
    x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    m, s = ref.gmsd_stats(a, b, 255.0)
    got = fa.gmsd(x, y, data_range=255.0, reduction="none").cpu().numpy()
    assert np.all(np.abs(got - s) <= REL * np.abs(s))
    gm = fa.gms(x, y, data_range=255.0, reduction="none").cpu().numpy()
    assert np.all(np.abs(gm - m) <= REL * np.abs(m))
    # configs[4] grayscale variant through luma
    ya = ref.rgb_to_luma(a.astype(np.float64), "bt601")
    yb = ref.rgb_to_luma(b.astype(np.float64), "bt601")
    _, s1 = ref.gmsd_stats(ya, yb, 255.0)
    got1 = fa.gmsd(x, y, data_range=255.0, luma="bt601", reduction="none").cpu().numpy()
    assert np.all(np.abs(got1 - s1) <= REL * np.abs(s1))


def test_gmsd_identity(gpu):
    a, _ = _plane_pair()
    x = torch.as_tensor(a, dtype=torch.uint8, device=gpu)[None, None]
    assert float(fa.gmsd(x, x, data_range=255.0)) < 1e-6
    assert abs(float(fa.gms(x, x, data_range=255.0)) - 1.0) < 1e-7


def test_gmsd_map_and_native_hint(gpu):
    a, b = _plane_pair()
    x = torch.as_tensor(a, dtype=torch.uint8, device=gpu)[None, None]
    y = torch.as_tensor(b, dtype=torch.uint8, device=gpu)[None, None]
    m = fa.gmsd(x, y, data_range=255.0, return_map=True)
    assert m.shape == (1, 1, a.shape[0] // 2 - 2, a.shape[1] // 2 - 2)
    assert abs(float(m.double().std(unbiased=False)) - float(fa.gmsd(x, y, data_range=255.0))) < 1e-6
    for fn in (fa.gms, fa.gmsd):
        with pytest.raises(RuntimeError, match="native GMSD"):
            fn(x, y, data_range=255.0, return_map=True, backend_hint="native")


def test_gms_loss_gradient_finite(gpu):
    x = torch.rand(1, 1, 64, 64, device=gpu, requires_grad=True)
    y = x.detach().clone()
    fa.GMSD(data_range=1.0).loss(x, y).backward()
    assert torch.isfinite(x.grad).all()


# --------------------------------------------------------------------------- #
# the pyramid step
# --------------------------------------------------------------------------- #


@pytest.mark.parametrize("dt", [torch.uint8, torch.float16, torch.bfloat16, torch.float32,
                                torch.float64])
@pytest.mark.parametrize("hw", [(2, 2), (9, 12), (10, 7), (33, 1), (1080, 1920)])
def test_pool2_exact(gpu, dt, hw):
    """fa_gpu_pool2 equals float64 avg_pool2d bit for bit, in the exact type."""
    from frame_analytics_amd import backend

    h, w = hw
    if w < 2:
        pytest.skip("needs two columns")
    g = torch.Generator(device=gpu)
    g.manual_seed(h * 31 + w)
    if dt == torch.uint8:
        x = torch.randint(0, 256, (2, 3, h, w), dtype=dt, device=gpu, generator=g)
        y = torch.randint(0, 256, (2, 3, h, w), dtype=dt, device=gpu, generator=g)
    else:
        x = torch.rand((2, 3, h, w), device=gpu, generator=g).to(dt)
        y = torch.rand((2, 3, h, w), device=gpu, generator=g).to(dt)
    ox, oy = backend.pool2_gpu(x, y)
    assert ox.dtype == backend.pyramid_dtype(dt)
    wx = torch.nn.functional.avg_pool2d(x.double(), 2)
    wy = torch.nn.functional.avg_pool2d(y.double(), 2)
    assert torch.equal(ox.double(), wx) and torch.equal(oy.double(), wy)
