"""GPU parity of MS-SSIM (value and gradient) and GMSD / GMS.

Bar: values within 1e-6 relative of float64; gradients 1e-6 max-normwise
relative (the MS-SSIM pyramid levels are exact: float32 below uint8 input,
float64 below floating input).  Where the true value
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


@pytest.mark.parametrize("weights", [None, (0.2, 0.3, 0.5)])
@pytest.mark.parametrize("luma", [None, "bt601"])
def test_ms_ssim_one_reduction_matches_per_scale_means(gpu, weights, luma):
    """The inference path leaves each scale's partial sums unreduced and
    finishes every scale in one reduction (fa_gpu_ms_ssim_reduce).  Its result
    equals the per-scale plane means (one finalize per scale, as the training
    path uses them) combined on the host, for both reductions, with luma and a
    cropped view."""
    from frame_analytics_amd import backend
    from frame_analytics_amd.functional import MS_SSIM_WEIGHTS, _luma_tuple, gaussian_window_1d

    a, b = u8_pair((3, 3, 200, 216), 9.0, seed=21)
    x = torch.from_numpy(a).to(gpu)[..., 2:-2, 3:-1]
    y = torch.from_numpy(b).to(gpu)[..., 2:-2, 3:-1]
    w = MS_SSIM_WEIGHTS if weights is None else weights
    kw = {} if weights is None else {"weights": weights}
    per = fa.ms_ssim(x, y, data_range=255.0, reduction="none", luma=luma, **kw)
    tot = fa.ms_ssim(x, y, data_range=255.0, luma=luma, **kw)
    win = gaussian_window_1d(11, 1.5, device=gpu, dtype=torch.float32)
    lw = None if luma is None else _luma_tuple(luma, 255.0)
    pdt = torch.float64 if lw is not None else torch.float32
    cx, cy, terms = x, y, []
    for i in range(len(w)):
        last = i == len(w) - 1
        out = backend.ssim_cs_pool(cx, cy, win, 127.5, 6.5025, 58.5225, None if last else pdt,
                                   luma=lw if i == 0 else None)
        terms.append((out[0] if last else out[1]).double().cpu().numpy().reshape(3, -1))
        if not last:
            cx, cy = out[2], out[3]
    plane = np.ones_like(terms[0])
    for t, wi in zip(terms, w):
        plane = plane * np.maximum(t, 0.0) ** wi
    want = plane.mean(axis=1)
    assert np.abs(per.cpu().numpy() - want).max() < 1e-14
    assert abs(float(tot) - want.mean()) < 1e-14


@pytest.mark.parametrize("n", [1, 8, 69])
def test_ms_ssim_batch_equals_single_images(gpu, n):
    """The inference reduction (fa_gpu_ms_ssim_reduce) over a batch gives each
    image the value a one-image call gives it, to 1e-14, and the batch mean
    of them; 69 RGB images at 5 scales are 1035 (plane, scale) terms."""
    a, b = u8_pair((n, 3, 176, 184), 9.0, seed=n)
    x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    per = fa.ms_ssim(x, y, data_range=255.0, reduction="none").cpu().numpy()
    for i in sorted({0, n // 2, n - 1}):
        one = float(fa.ms_ssim(x[i:i + 1], y[i:i + 1], data_range=255.0))
        assert abs(one - per[i]) < 1e-14, (i, one, per[i])
    assert abs(float(fa.ms_ssim(x, y, data_range=255.0)) - per.mean()) < 1e-14
    if n == 1:
        want = ref.ms_ssim(a.astype(np.float64), b.astype(np.float64), 255.0)
        assert _rel(float(per[0]), float(want)) <= REL


def test_ms_ssim_nan_propagates_like_torch(gpu):
    """A NaN sample makes MS-SSIM NaN on every path: the fused inference
    reduction (fa_gpu_ms_ssim_reduce) clamps like torch's clamp_min, which
    keeps NaN, as the per-scale path of a gradient call does."""
    a, b = _plane_pair(192, 200, seed=3)
    x = torch.as_tensor(a, dtype=torch.float32, device=gpu)[None, None].clone()
    y = torch.as_tensor(b, dtype=torch.float32, device=gpu)[None, None]
    x[0, 0, 100, 100] = float("nan")
    fused = fa.ms_ssim(x, y, data_range=255.0)
    fused_none = fa.ms_ssim(x, y, data_range=255.0, reduction="none")
    per_scale = fa.ms_ssim(x.clone().requires_grad_(True), y, data_range=255.0)
    assert torch.isnan(fused) and torch.isnan(fused_none).all()
    assert torch.isnan(per_scale.detach())


def test_ms_ssim_too_small(gpu):
    x = torch.zeros(1, 1, 175, 300, device=gpu)
    with pytest.raises(ValueError, match="too small"):
        fa.ms_ssim(x, x, data_range=1.0)
    z = torch.zeros(1, 1, 176, 300, device=gpu)
    assert float(fa.ms_ssim(z, z, data_range=1.0)) == pytest.approx(1.0)


def _ms_call(x, y, weights, k=11, acc=None):
    """fa_gpu_ms_ssim through the C ABI over a workspace filled with 0xFF:
    (per-image values, batch mean, the workspace afterwards)."""
    import ctypes

    from frame_analytics_amd import backend
    from frame_analytics_amd.functional import gaussian_window_1d

    n, c, h, w = (int(v) for v in x.shape)
    m = len(weights)
    win = gaussian_window_1d(k, 1.5, device=x.device, dtype=torch.float32)
    nb = ctypes.c_int64(0)
    assert backend.call_gpu("fa_gpu_ms_ssim_workspace", 0, n, c, h, w, k, m, 0,
                            ctypes.byref(nb)) == 0
    ws = torch.full((nb.value,), 0xFF, dtype=torch.uint8, device=x.device)
    out = torch.full((n + 1,), -7.0, dtype=torch.float64, device=x.device)
    x, xs = backend._view_strides(x)
    y, ys = backend._view_strides(y)
    wts = (ctypes.c_double * m)(*[float(v) for v in weights])
    stream = torch.cuda.current_stream().cuda_stream
    rc = backend.call_gpu("fa_gpu_ms_ssim", x.data_ptr(), y.data_ptr(), 0, n, c, h, w, xs, ys,
                          None, win.data_ptr(), k, 127.5, (0.01 * 255) ** 2, (0.03 * 255) ** 2,
                          wts, m, ws.data_ptr(), nb.value,
                          None if acc is None else acc.data_ptr(), out.data_ptr(),
                          out[n:].data_ptr(), 0, stream)
    assert rc == 0, rc
    o = out.cpu().numpy()
    return o[:n], float(o[n]), ws


def test_ms_ssim_three_launch_path_at_256_planes(gpu):
    """The three-launch path at its plane limit (256 planes: every slot of the
    final workgroup's term array in use), against the per-scale path to 1e-12
    and two of its images against the oracle."""
    from frame_analytics_amd import backend
    from frame_analytics_amd.functional import MS_SSIM_WEIGHTS

    a, b = u8_pair((256, 1, 256, 256), 9.0, seed=256)
    x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    w = tuple(MS_SSIM_WEIGHTS)
    acc = torch.zeros(backend._ACC_WORDS["ms"], dtype=torch.int64, device=gpu)
    per0, tot0, _ = _ms_call(x, y, w)
    per, tot, ws = _ms_call(x, y, w, acc=acc)
    scratch = len(w) * 256 * 8
    start = -((scratch + 255) // 256 * 256)
    assert bool((ws[start:start + scratch] == 0xFF).all())  # the three-launch path ran
    assert int((acc != 0).sum()) == 0
    assert np.all(np.abs(per - per0) <= 1e-12 * np.abs(per0))
    assert abs(tot - tot0) <= 1e-12 * abs(tot0)
    for i in (0, 255):
        want = ref.ms_ssim(a[i:i + 1].astype(np.float64), b[i:i + 1].astype(np.float64), 255.0)
        assert _rel(float(per[i]), float(want)) <= REL, (i, per[i], want)


def test_ms_ssim_three_launch_path_declines_past_its_limits(gpu):
    """With the accumulator, calls the three-launch path does not take run the
    per-scale path and give its result bit for bit, leaving the accumulator
    zero: more than 256 planes (86 RGB images), six scales, and a width whose
    first level is not a multiple of 8 (360 -> 180)."""
    from frame_analytics_amd import backend

    acc = torch.zeros(backend._ACC_WORDS["ms"], dtype=torch.int64, device=gpu)
    cases = [((86, 3, 256, 256), (0.0448, 0.2856, 0.3001, 0.2363, 0.1333)),
             ((1, 3, 704, 704), (0.1, 0.1, 0.2, 0.2, 0.2, 0.2)),
             ((2, 3, 352, 360), (0.0448, 0.2856, 0.3001, 0.2363, 0.1333))]
    for shape, w in cases:
        a, b = u8_pair(shape, 9.0, seed=shape[0])
        x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
        per0, tot0, _ = _ms_call(x, y, w)
        per1, tot1, _ = _ms_call(x, y, w, acc=acc)
        assert np.array_equal(per0, per1) and tot0 == tot1, shape
        assert int((acc != 0).sum()) == 0


@pytest.mark.parametrize("shape,weights,k,crop", [
    ((3, 3, 517, 512), None, 11, False),
    ((2, 1, 256, 640), (0.3, 0.3, 0.4), 11, False),
    ((2, 3, 384, 384), (0.1, 0.2, 0.3, 0.4), 7, True),
])
def test_ms_ssim_three_launch_path(gpu, shape, weights, k, crop):
    """uint8 MS-SSIM with the stream's accumulator: scale 0, scale 1 (which
    also writes the levels of scales 3 and 4), then the coarse scales side by
    side in one launch whose last workgroup finishes the reduction from
    fixed-point sums.  Against the per-scale path (no accumulator) to 1e-12
    relative and against the oracle to the bar, on two calls in a row; each
    call leaves the accumulator zero and never writes the per-scale path's
    reduction scratch (the workspace's last region, which that path fills)."""
    from frame_analytics_amd import backend
    from frame_analytics_amd.functional import MS_SSIM_WEIGHTS

    w = tuple(MS_SSIM_WEIGHTS) if weights is None else weights
    n, c, h, wd = shape
    if crop:
        a, b = u8_pair((n, c, h + 16, wd + 24), 9.0, seed=5)
        x = torch.from_numpy(a).to(gpu)[..., 5:5 + h, 8:8 + wd]
        y = torch.from_numpy(b).to(gpu)[..., 5:5 + h, 8:8 + wd]
    else:
        a, b = u8_pair(shape, 9.0, seed=5)
        x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    m = len(w)
    scratch = m * n * c * 8
    start = -((scratch + 255) // 256 * 256)  # the reduction's scratch, last in the workspace
    per0, tot0, ws0 = _ms_call(x, y, w, k)
    assert not bool((ws0[start:start + scratch] == 0xFF).all())
    acc = torch.zeros(backend._ACC_WORDS["ms"], dtype=torch.int64, device=gpu)
    for _ in range(2):
        per, tot, ws = _ms_call(x, y, w, k, acc=acc)
        assert bool((ws[start:start + scratch] == 0xFF).all())
        assert int((acc != 0).sum()) == 0
        assert np.all(np.abs(per - per0) <= 1e-12 * np.abs(per0)), (per, per0)
        assert abs(tot - tot0) <= 1e-12 * abs(tot0), (tot, tot0)
    want = ref.ms_ssim(x.cpu().numpy().astype(np.float64), y.cpu().numpy().astype(np.float64),
                       255.0, win_size=k, weights=w, reduction="none")
    assert np.all(np.abs(per - want) <= REL * np.abs(want)), (per, want)


@pytest.mark.parametrize("recompute", ["0", "1"])
@pytest.mark.parametrize("shape", [(1, 1, 192, 192), (2, 3, 180, 200)])
@pytest.mark.parametrize("wrt", [("x",), ("x", "y")])
def test_ms_ssim_backward_matches_oracle(gpu, shape, wrt, recompute, monkeypatch):
    """dL/dx and dL/dy of 1 - ms_ssim against the oracle's closed-form float64
    MS-SSIM adjoint (oracle.ms_ssim_grad, itself pinned by central differences
    of the float64 forward), 1e-6 max-normwise: with the coefficient maps
    written by the forward (the default) and recomputed in the backward
    (FA_MS_SSIM_RECOMPUTE=1)."""
    monkeypatch.setenv("FA_MS_SSIM_RECOMPUTE", recompute)
    xa, ya = float_pair(shape, 0.05, seed=shape[-1])
    x = torch.from_numpy(xa).to(gpu).requires_grad_("x" in wrt)
    y = torch.from_numpy(ya).to(gpu).requires_grad_("y" in wrt)
    (1.0 - fa.ms_ssim(x, y, data_range=1.0)).backward()
    gx, gy = ref.ms_ssim_grad(xa, ya, data_range=1.0)
    for got, want in ((x.grad, -gx), (y.grad, -gy if "y" in wrt else None)):
        assert (got is None) == (want is None)
        if want is None:
            continue
        err = float(np.abs(got.double().cpu().numpy() - want).max() / np.abs(want).max())
        assert err <= REL, err


@pytest.mark.parametrize("dt", [torch.float32, torch.float64])
@pytest.mark.parametrize("unit_s", [False, True])
@pytest.mark.parametrize("need_dy", [False, True])
def test_cs_coef_scatter_matches_recomputed_backward(gpu, dt, unit_s, need_dy):
    """The training CS pass that also writes unit-gradient coefficient maps
    (fa_gpu_ssim_cs_coef) and the scatter that scales them per plane
    (fa_gpu_ssim_cs_scatter) against the CS forward and the recomputing
    backward (fa_gpu_ssim_cs_backward_ex) with the same gradient: plane means
    to 1e-6 of the float32 forward (1e-12 of the float64 one), the pyramid
    levels bit for bit, dx / dy to 1e-6 max-normwise (both paths round the
    maps to float32: one the unit maps, the other the scaled ones), with and
    without the level's gradient."""
    from frame_analytics_amd import backend
    from frame_analytics_amd.functional import gaussian_window_1d

    xa, ya = float_pair((2, 3, 100, 124), 0.05, seed=7)
    x = torch.from_numpy(xa).to(device=gpu, dtype=dt)
    y = torch.from_numpy(ya).to(device=gpu, dtype=dt)
    win = gaussian_window_1d(11, 1.5, device=gpu, dtype=torch.float32)
    consts = (0.5, (0.01) ** 2, (0.03) ** 2)
    s0, cs0, px0, py0 = backend.ssim_cs_forward(x, y, win, *consts, torch.float64)
    s1, cs1, px1, py1, aux = backend.ssim_cs_coef_forward(x, y, win, *consts, unit_s,
                                                          torch.float64, need_dy)
    tol = 1e-6 if dt == torch.float32 else 1e-12
    for a, b in ((s1, s0), (cs1, cs0)):
        assert float(((a - b).abs() / b.abs()).max()) <= tol
    assert torch.equal(px1, px0) and torch.equal(py1, py0)
    g = torch.linspace(-1.5, 2.0, 6, device=gpu, dtype=torch.float64)
    zero = torch.zeros_like(g)
    gen = torch.Generator(device="cpu").manual_seed(3)
    for gp in (None, torch.randn(px0.shape, generator=gen, dtype=torch.float64).to(gpu)):
        gpy = gp if need_dy else None
        dx, dy = backend.ssim_cs_scatter(x, y, g, aux, win, consts[0], True, need_dy, gp, gpy)
        wx, wy = backend.ssim_cs_backward(x, y, g if unit_s else zero, zero if unit_s else g,
                                          win, *consts, True, need_dy, gp, gpy)
        for got, want in ((dx, wx), (dy, wy)):
            assert (got is None) == (want is None)
            if want is None:
                continue
            err = float((got - want).abs().max() / want.abs().max())
            assert err <= 1e-6, err


def test_cs_coef_path_falls_back_when_both_means_get_gradients(gpu):
    """A loss that reads both plane means of a scale made with ``use="cs"``
    (not MS-SSIM's) gets the recomputing backward: its gradient equals the one
    of the same loss without ``use``."""
    from frame_analytics_amd.functional import _NativeSSIM, gaussian_window_1d

    xa, ya = float_pair((1, 2, 64, 72), 0.05, seed=9)
    win = gaussian_window_1d(11, 1.5, device=gpu, dtype=torch.float32)
    consts = (0.5, (0.01) ** 2, (0.03) ** 2)
    grads = []
    for use in ("cs", None):
        x = torch.from_numpy(xa).to(gpu).requires_grad_(True)
        y = torch.from_numpy(ya).to(gpu)
        s, cs, px, _ = _NativeSSIM.apply(x, y, win, consts, "cs+pool", torch.float64, use)
        (s.sum() + 2.0 * cs.sum() + px.sum()).backward()
        grads.append(x.grad.double())
    err = float((grads[0] - grads[1]).abs().max() / grads[1].abs().max())
    assert err <= 1e-6, err


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


@pytest.mark.parametrize("down", [True, False])
@pytest.mark.parametrize("dt", [torch.uint8, torch.float16, torch.float32, torch.float64])
@pytest.mark.parametrize("mode", ["bt601", "bt709", "matlab"])
def test_gmsd_luma_fused(gpu, mode, dt, down):
    """Luma formed inside the kernel (float64) against the float64 oracle's
    luma-then-GMSD; 216 columns take the dword path for uint8 + downsampling."""
    a, b = u8_pair((2, 3, 134, 216), 12.0, seed=21)
    la = ref.rgb_to_luma(a.astype(np.float64), mode)
    lb = ref.rgb_to_luma(b.astype(np.float64), mode)
    m, s = ref.gmsd_stats(la, lb, 255.0, downsample=down)
    x, y = torch.from_numpy(a).to(gpu, dt), torch.from_numpy(b).to(gpu, dt)
    kw = dict(data_range=255.0, luma=mode, downsample=down, reduction="none")
    got_s = fa.gmsd(x, y, **kw).cpu().numpy()
    got_m = fa.gms(x, y, **kw).cpu().numpy()
    assert np.all(np.abs(got_s - s) <= REL * np.abs(s)), (got_s, s)
    assert np.all(np.abs(got_m - m) <= REL * np.abs(m)), (got_m, m)


@pytest.mark.parametrize("luma", [None, "bt601"])
@pytest.mark.parametrize("border", [3, 4, 8])
def test_gmsd_crop_read_in_place(gpu, border, luma):
    """Cropped views go to the kernel through their strides: border 4 / 8
    keeps every row 4-byte aligned (dword path), border 3 does not."""
    a, b = u8_pair((2, 3, 140, 216), 10.0, seed=border)
    ca = ref.crop(a.astype(np.float64), border)
    cb = ref.crop(b.astype(np.float64), border)
    if luma:
        ca, cb = ref.rgb_to_luma(ca, luma), ref.rgb_to_luma(cb, luma)
    m, s = ref.gmsd_stats(ca, cb, 255.0)
    x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    kw = dict(data_range=255.0, luma=luma, crop_border=border, reduction="none")
    got_s = fa.gmsd(x, y, **kw).cpu().numpy()
    got_m = fa.gms(x, y, **kw).cpu().numpy()
    assert np.all(np.abs(got_s - s) <= REL * np.abs(s)), (got_s, s)
    assert np.all(np.abs(got_m - m) <= REL * np.abs(m)), (got_m, m)


def test_gmsd_channel_view_strides(gpu):
    """A channel slice (image stride 3 planes, channel stride 1 plane)."""
    a, b = u8_pair((3, 3, 96, 128), 14.0, seed=2)
    m, s = ref.gmsd_stats(a[:, 1:3], b[:, 1:3], 255.0)
    x, y = torch.from_numpy(a).to(gpu)[:, 1:3], torch.from_numpy(b).to(gpu)[:, 1:3]
    assert not x.is_contiguous()
    got = fa.gmsd(x, y, data_range=255.0, reduction="none").cpu().numpy()
    assert np.all(np.abs(got - s) <= REL * np.abs(s))


@pytest.mark.parametrize("hw", [(8, 8), (10, 260), (9, 264), (300, 516), (40, 1016), (13, 520)])
def test_gmsd_dword_path_edges(gpu, hw):
    """The uint8 dword path at its edges: smallest grid, one to four wave
    strips (126 outputs each, e.g. 126 + 2), odd row counts."""
    a, b = natural_pair(*hw, noise=9.0, seed=hw[1])
    m, s = ref.gmsd_stats(a[None, None], b[None, None], 255.0)
    x = torch.as_tensor(a, dtype=torch.uint8, device=gpu)[None, None]
    y = torch.as_tensor(b, dtype=torch.uint8, device=gpu)[None, None]
    assert _rel(float(fa.gmsd(x, y, data_range=255.0)), float(s[0])) <= REL
    assert _rel(float(fa.gms(x, y, data_range=255.0)), float(m[0])) <= REL


def test_gmsd_configs4_full_batch(gpu):
    """configs[4] GMSD at its real batch, 8x3x1080x1920 uint8, per channel and
    grayscale through luma="bt601": image 0 against the oracle, every image by
    per-image consistency with a one-image call."""
    a, b = u8_pair((8, 3, 1080, 1920), 8.0, seed=1)
    x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    for luma in (None, "bt601"):
        kw = dict(data_range=255.0, luma=luma)
        per = fa.gmsd(x, y, reduction="none", **kw).cpu().numpy()
        a0, b0 = a[:1].astype(np.float64), b[:1].astype(np.float64)
        if luma:
            a0, b0 = ref.rgb_to_luma(a0, luma), ref.rgb_to_luma(b0, luma)
        _, s0 = ref.gmsd_stats(a0, b0, 255.0)
        assert _rel(float(per[0]), float(s0[0])) <= REL, (luma, per[0], s0)
        # a one-image call splits the work differently, so its float32 group
        # sums differ in the last bits: 1e-9 relative, well inside the bar
        for i in (3, 7):
            one = float(fa.gmsd(x[i:i + 1], y[i:i + 1], **kw))
            assert abs(one - float(per[i])) <= 1e-9 * abs(one), (luma, i)
        assert abs(float(fa.gmsd(x, y, **kw)) - float(per.mean())) <= 1e-12 * float(per.mean())


def test_gmsd_identity(gpu):
    a, _ = _plane_pair()
    x = torch.as_tensor(a, dtype=torch.uint8, device=gpu)[None, None]
    assert float(fa.gmsd(x, x, data_range=255.0)) < 1e-6
    assert abs(float(fa.gms(x, x, data_range=255.0)) - 1.0) < 1e-7


@pytest.mark.parametrize("down", [True, False])
def test_gmsd_map_native(gpu, down):
    """The kernel writes the float32 q map (return_map=True)."""
    a, b = _plane_pair()
    x = torch.as_tensor(a, dtype=torch.uint8, device=gpu)[None, None]
    y = torch.as_tensor(b, dtype=torch.uint8, device=gpu)[None, None]
    want = ref.gms_map(a[None, None], b[None, None], 255.0, downsample=down)
    for fn in (fa.gms, fa.gmsd):
        m = fn(x, y, data_range=255.0, return_map=True, downsample=down, backend_hint="native")
        assert m.dtype == torch.float32 and tuple(m.shape) == want.shape
        assert np.abs(m.cpu().double().numpy() - want).max() <= 1e-6
    xf, yf = x.float(), y.float()
    m = fa.gmsd(xf, yf, data_range=255.0, return_map=True, downsample=down)
    assert np.abs(m.cpu().double().numpy() - want).max() <= 1e-6


def test_gmsd_map_luma_crop(gpu):
    a, b = u8_pair((2, 3, 90, 120), 12.0, seed=31)
    x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    la = ref.rgb_to_luma(ref.crop(a.astype(np.float64), 4), "bt709")
    lb = ref.rgb_to_luma(ref.crop(b.astype(np.float64), 4), "bt709")
    want = ref.gms_map(la, lb, 255.0)
    m = fa.gms(x, y, data_range=255.0, return_map=True, luma="bt709", crop_border=4)
    assert tuple(m.shape) == want.shape
    assert np.abs(m.cpu().double().numpy() - want).max() <= 1e-6


@pytest.mark.parametrize("down", [True, False])
@pytest.mark.parametrize("dt", [torch.float32, torch.float64])
def test_gms_gmsd_gradient_matches_oracle(gpu, down, dt):
    """The native float64 backward of per-image GMS and GMSD (both at once,
    mixed upstream) against the float64 oracle gradient, 1e-6 normwise."""
    rng = np.random.default_rng(17)
    a = np.stack([_plane_pair(75, 93, seed=s)[0] for s in range(6)]).reshape(2, 3, 75, 93) / 255.0
    b = np.clip(a + 0.05 * rng.standard_normal(a.shape), 0, 1)
    gm = np.array([0.8, -1.1])
    gs = np.array([1.7, 0.6])
    x = torch.tensor(a, dtype=dt, device=gpu, requires_grad=True)
    y = torch.tensor(b, dtype=dt, device=gpu, requires_grad=True)
    # the oracle sees exactly the values the kernel sees (float32-rounded)
    a, b = x.detach().cpu().double().numpy(), y.detach().cpu().double().numpy()
    kw = dict(data_range=1.0, downsample=down, reduction="none")
    m = fa.gms(x, y, **kw)
    s = fa.gmsd(x, y, **kw)
    mw, sw = ref.gmsd_stats(a, b, 1.0, downsample=down)
    assert np.all(np.abs(m.detach().cpu().numpy() - mw) <= REL * np.abs(mw))
    assert np.all(np.abs(s.detach().cpu().numpy() - sw) <= REL * np.abs(sw))
    ((m * torch.tensor(gm, device=gpu)).sum() + (s * torch.tensor(gs, device=gpu)).sum()).backward()
    wx, wy = ref.gms_stats_grad(a, b, 1.0, downsample=down, g_mean=gm, g_std=gs)
    for got, want in ((x.grad, wx), (y.grad, wy)):
        g = got.detach().cpu().double().numpy()
        assert g.shape == want.shape
        err = np.abs(g - want).max() / np.abs(want).max()
        assert err <= 1e-6, err


def test_gms_loss_gradient_finite(gpu):
    x = torch.rand(1, 1, 64, 64, device=gpu, requires_grad=True)
    y = x.detach().clone()
    fa.GMSD(data_range=1.0).loss(x, y).backward()
    assert torch.isfinite(x.grad).all()


# --------------------------------------------------------------------------- #
# the pyramid step
# --------------------------------------------------------------------------- #


def _rand_pair(dt, shape, seed, gpu):
    g = torch.Generator(device=gpu)
    g.manual_seed(seed)
    if dt == torch.uint8:
        x = torch.randint(0, 256, shape, dtype=dt, device=gpu, generator=g)
        y = torch.randint(0, 256, shape, dtype=dt, device=gpu, generator=g)
    else:
        x = (255 * torch.rand(shape, device=gpu, generator=g, dtype=torch.float64)).to(dt)
        y = (255 * torch.rand(shape, device=gpu, generator=g, dtype=torch.float64)).to(dt)
    return x, y


# (H, W, K): one strip / chunk, odd trailing row and column, several strips
# (246 output columns each at K=11) and 64-row chunks, other windows
_LEVEL_CASES = [(11, 11, 11), (12, 13, 11), (75, 300, 11), (141, 501, 11), (257, 511, 7),
                (66, 258, 3), (1080, 1920, 11)]


@pytest.mark.parametrize("dt", [torch.uint8, torch.float16, torch.bfloat16, torch.float32,
                                torch.float64])
@pytest.mark.parametrize("case", _LEVEL_CASES)
def test_fused_pyramid_level_exact(gpu, dt, case):
    """The level written by the CS pass equals float64 avg_pool2d bit for bit
    (float64 input: to rounding), and the (ssim, cs) means equal those of the
    plain CS pass bit for bit."""
    from frame_analytics_amd import backend
    from frame_analytics_amd.functional import gaussian_window_1d

    h, w, k = case
    x, y = _rand_pair(dt, (2, 3, h, w), h * 31 + w + k, gpu)
    win = gaussian_window_1d(k, 1.5, device=gpu, dtype=torch.float32)
    pdt = backend.pyramid_dtype(dt)
    s, cs, px, py = backend.ssim_cs_pool(x, y, win, 127.5, 6.5025, 58.5225, pdt)
    s0, cs0 = backend.ssim_cs_pool(x, y, win, 127.5, 6.5025, 58.5225, None)
    torch.cuda.synchronize()
    assert px.dtype == pdt and px.shape == (2, 3, h // 2, w // 2)
    wx = torch.nn.functional.avg_pool2d(x.double(), 2)
    wy = torch.nn.functional.avg_pool2d(y.double(), 2)
    if dt == torch.float64:
        # four doubles summed in another order: within two units in the last place
        for got, want in ((px, wx), (py, wy)):
            assert ((got - want).abs() <= 2.0 ** -51 * want.abs()).all()
    else:
        assert torch.equal(px.double(), wx) and torch.equal(py.double(), wy)
    assert torch.equal(s, s0) and torch.equal(cs, cs0)


@pytest.mark.parametrize("dt", [torch.float32, torch.float64])
def test_fused_pyramid_level_gradient(gpu, dt):
    """d/dx of a loss on (s, cs, px, py) equals the CS gradient plus a quarter
    of the level gradient spread over each 2x2 block (odd edge excluded)."""
    from frame_analytics_amd import backend
    from frame_analytics_amd.functional import _NativeSSIM, gaussian_window_1d

    n, c, h, w = 1, 2, 75, 263
    x0, y0 = _rand_pair(dt, (n, c, h, w), 5, gpu)
    win = gaussian_window_1d(11, 1.5, device=gpu, dtype=torch.float32)
    pdt = torch.float64
    x = x0.clone().requires_grad_(True)
    y = y0.clone().requires_grad_(True)
    g = torch.Generator(device=gpu)
    g.manual_seed(9)
    rs = torch.rand(n * c, device=gpu, generator=g, dtype=torch.float64)
    rcs = torch.rand(n * c, device=gpu, generator=g, dtype=torch.float64)
    r1 = torch.rand((n, c, h // 2, w // 2), device=gpu, generator=g, dtype=pdt)
    r2 = torch.rand((n, c, h // 2, w // 2), device=gpu, generator=g, dtype=pdt)
    s, cs, px, py = _NativeSSIM.apply(x, y, win, (127.5, 6.5025, 58.5225), "cs+pool", pdt)
    ((s * rs).sum() + (cs * rcs).sum() + (px * r1).sum() + (py * r2).sum()).backward()

    dx, dy = backend.ssim_cs_backward(x0, y0, rs, rcs, win, 127.5, 6.5025, 58.5225,
                                      True, True)

    def spread(r):
        full = torch.zeros((n, c, h, w), dtype=torch.float64, device=gpu)
        full[..., : 2 * (h // 2), : 2 * (w // 2)] = (
            0.25 * r).repeat_interleave(2, -2).repeat_interleave(2, -1)
        return full

    tol = 1e-6 if dt == torch.float32 else 1e-12
    for got, base, r in ((x.grad, dx, r1), (y.grad, dy, r2)):
        want = base.double() + spread(r)
        err = (got.double() - want).abs().max() / want.abs().max()
        assert err <= tol, (dt, float(err))


def _gmsd_call(name, x, y, T, eps, down, acc=None, batch=False, luma=None):
    """fa_gpu_gmsd (or fa_gpu_gmsd_once with ``acc``) through the C ABI:
    (mean, std[, batch means]) as float64 numpy arrays."""
    import ctypes

    from frame_analytics_amd import backend

    n, c, h, w = (int(v) for v in x.shape)
    bpp = backend.workspace_slots("gmsd", h, w, int(down))
    planes = n * (1 if luma else c)
    ps = torch.full((2, planes, bpp), -7.0, dtype=torch.float64, device=x.device)
    out = torch.full((2 * n + 2,), -7.0, dtype=torch.float64, device=x.device)
    stream = torch.cuda.current_stream().cuda_stream
    head = (x.data_ptr(), y.data_ptr(), backend._DTYPE_CODE[x.dtype], n, c, h, w)
    lw = None if luma is None else (ctypes.c_double * 3)(*luma)
    if name == "fa_gpu_gmsd":
        rc = backend.call_gpu(name, *head, float(T), float(eps), int(down), ps[0].data_ptr(),
                              ps[1].data_ptr(), bpp, out.data_ptr(), out[n:].data_ptr(), 0,
                              stream)
    else:
        rc = backend.call_gpu(name, *head, None, None, lw, float(T), float(eps), int(down),
                              ps[0].data_ptr(), ps[1].data_ptr(), bpp,
                              None if acc is None else acc.data_ptr(), out.data_ptr(),
                              out[n:].data_ptr(), out[2 * n:].data_ptr() if batch else None,
                              0, stream)
    assert rc == 0, (name, rc)
    o = out.cpu().numpy()
    return o[:n], o[n:2 * n], o[2 * n:]


@pytest.mark.parametrize("shape,down", [((1, 1, 200, 232), True), ((8, 3, 1080, 1920), True),
                                        ((5, 3, 130, 150), False), ((64, 1, 96, 80), True),
                                        ((65, 1, 40, 48), True)])
def test_gmsd_one_launch_matches_two_launches(gpu, shape, down):
    """fa_gpu_gmsd_once: per-image statistics whose sums went through the
    fixed-point atomics agree with fa_gpu_gmsd's fixed-order float64 sums --
    mean q to 1e-12 relative, std q to 1e-10 (each workgroup's sum of d^2 is
    rounded to 2^-30 at 1080p; over ~200 workgroups that is ~1e-11 of the
    variance, which the E[d^2] - E[d]^2 cancellation carries into the std) --
    and with the oracle to the 1e-6 bar; its batch means
    match the means of the per-image values; the same call twice gives the
    same bits (the adds' order does not matter); the accumulator is zero
    after every call, including a second, smaller call on it.  N = 65 is
    past the one-launch form: the two-launch path with the batch block."""
    from frame_analytics_amd import backend

    a, b = u8_pair(shape, 9.0, seed=shape[0] * 31 + shape[2])
    x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    T, eps = 170.0, (1e-6 * 255.0) ** 2
    acc = torch.zeros(backend._ACC_WORDS["gmsd"], dtype=torch.int64, device=gpu)
    m2, s2, _ = _gmsd_call("fa_gpu_gmsd", x, y, T, eps, down)
    m1, s1, bt = _gmsd_call("fa_gpu_gmsd_once", x, y, T, eps, down, acc=acc, batch=True)
    assert not bool(acc.any())
    assert np.all(np.abs(m1 - m2) <= 1e-12 * np.abs(m2)), (m1, m2)
    assert np.all(np.abs(s1 - s2) <= 1e-10 * np.abs(s2)), (s1, s2)
    assert abs(bt[0] - m1.mean()) <= 1e-12 * abs(m1.mean())
    assert abs(bt[1] - s1.mean()) <= 1e-12 * abs(s1.mean())
    again = _gmsd_call("fa_gpu_gmsd_once", x, y, T, eps, down, acc=acc, batch=True)
    for u, v in zip((m1, s1, bt), again):
        assert np.array_equal(u, v)
    k = max(1, shape[0] // 2)
    mk, sk, _ = _gmsd_call("fa_gpu_gmsd_once", x[:k], y[:k], T, eps, down, acc=acc)
    assert not bool(acc.any())
    assert np.all(np.abs(sk - s2[:k]) <= 1e-9 * np.abs(s2[:k]))
    i = shape[0] - 1
    m0, s0 = ref.gmsd_stats(a[i:i + 1], b[i:i + 1], 255.0, downsample=down)
    assert _rel(float(s1[i]), float(s0[0])) <= REL and _rel(float(m1[i]), float(m0[0])) <= REL
    # luma, through the same one-launch finish
    lw = (0.299, 0.587, 0.114)
    if shape[1] == 3:
        ml, sl, _ = _gmsd_call("fa_gpu_gmsd_once", x, y, T, eps, down, acc=acc, luma=lw)
        al = ref.rgb_to_luma(a[:1].astype(np.float64), "bt601")
        bl = ref.rgb_to_luma(b[:1].astype(np.float64), "bt601")
        _, sr = ref.gmsd_stats(al, bl, 255.0, downsample=down)
        assert _rel(float(sl[0]), float(sr[0])) <= REL
        assert not bool(acc.any())


@pytest.mark.parametrize("dt", [torch.uint8, torch.float16, torch.float32, torch.float64])
def test_gmsd_flat_patch_without_T_and_eps_is_nan(gpu, dt):
    """T = eps = 0: a flat patch is 0 / 0 in q, so its image's statistics are
    NaN, as the oracle (and the reference's portable statistics) give; an
    image without a flat patch stays finite and matches the oracle; T = 0
    with eps > 0 stays finite too."""
    a, b = _plane_pair(120, 136, seed=5)
    a2, b2 = a.copy(), b.copy()
    a2[20:60, 30:80] = 100.0  # the same flat patch in both
    b2[20:60, 30:80] = 100.0
    xa = np.stack([a2, a])[:, None]
    xb = np.stack([b2, b])[:, None]
    x = torch.as_tensor(xa, dtype=dt, device=gpu)
    y = torch.as_tensor(xb, dtype=dt, device=gpu)
    with np.errstate(invalid="ignore", divide="ignore"):
        m0, s0 = ref.gmsd_stats(xa, xb, 255.0, T=0.0, eps=0.0)
    assert np.isnan(m0[0]) and np.isnan(s0[0]) and np.isfinite(s0[1])
    got_s = fa.gmsd(x, y, data_range=255.0, T=0.0, eps=0.0, reduction="none").cpu().numpy()
    got_m = fa.gms(x, y, data_range=255.0, T=0.0, eps=0.0, reduction="none").cpu().numpy()
    assert np.isnan(got_s[0]) and np.isnan(got_m[0]), (got_s, got_m)
    assert _rel(float(got_s[1]), float(s0[1])) <= REL and _rel(float(got_m[1]), float(m0[1])) <= REL
    assert np.isnan(float(fa.gmsd(x, y, data_range=255.0, T=0.0, eps=0.0)))
    if dt != torch.float64:  # (a float64 map is the portable path's, not a kernel's)
        qmap = fa.gms(x, y, data_range=255.0, T=0.0, eps=0.0, return_map=True).cpu().numpy()
        assert np.isnan(qmap[0]).any() and not np.isnan(qmap[1]).any()
    m1, s1 = ref.gmsd_stats(xa, xb, 255.0, T=0.0, eps=1e-30)
    got = fa.gmsd(x, y, data_range=255.0, T=0.0, eps=1e-30, reduction="none").cpu().numpy()
    assert np.all(np.isfinite(got)) and np.all(np.abs(got - s1) <= REL * np.abs(s1)), (got, s1)


def test_gmsd_one_launch_without_workspace(gpu):
    """fa_gpu_gmsd_once with null psum / psumsq: the launch that finishes the
    call does not read them (same statistics); with T = eps = 0 (no one-launch
    form) the call returns FA_E_ARG and writes nothing."""
    from frame_analytics_amd import backend

    a, b = u8_pair((2, 3, 240, 320), 9.0, seed=5)
    x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    acc = torch.zeros(backend._ACC_WORDS["gmsd"], dtype=torch.int64, device=gpu)
    m2, s2, _ = _gmsd_call("fa_gpu_gmsd", x, y, 170.0, 6.5e-8, True)
    bpp = backend.workspace_slots("gmsd", 240, 320, 1)
    st = torch.cuda.current_stream().cuda_stream
    for T, eps, ok in ((170.0, 6.5e-8, True), (0.0, 0.0, False)):
        out = torch.full((4,), -7.0, dtype=torch.float64, device=gpu)
        rc = backend.call_gpu("fa_gpu_gmsd_once", x.data_ptr(), y.data_ptr(), 0, 2, 3, 240, 320,
                              None, None, None, T, eps, 1, None, None, bpp, acc.data_ptr(),
                              out.data_ptr(), out[2:].data_ptr(), None, 0, st)
        torch.cuda.synchronize()
        if ok:
            assert rc == 0
            o = out.cpu().numpy()
            assert np.all(np.abs(o[:2] - m2) <= 1e-12 * np.abs(m2))
            assert np.all(np.abs(o[2:] - s2) <= 1e-10 * np.abs(s2))
        else:
            assert rc == 5 and bool((out == -7.0).all()), rc
        assert not bool(acc.any())


def test_one_launch_finishes_on_two_streams(gpu):
    """fa.ssim, fa.gmsd and fa.ms_ssim (uint8: the one-launch SSIM and GMSD
    forms, MS-SSIM's three launches) interleaved on two streams: each stream
    has its own accumulator, so every value matches the same call made alone
    on the default stream bit for bit (the fixed-point sums do not depend on
    the order), and both streams' accumulators are zero afterwards."""
    from frame_analytics_amd import backend

    a, b = u8_pair((2, 3, 256, 384), 6.0, seed=41)
    c, d = u8_pair((1, 3, 320, 512), 9.0, seed=42)
    ta, tb, tc, td = (torch.from_numpy(v).to(gpu) for v in (a, b, c, d))
    calls = {
        "ssim": lambda x, y: fa.ssim(x, y, data_range=255.0, reduction="none"),
        "gmsd": lambda x, y: fa.gmsd(x, y, data_range=255.0, reduction="none"),
        "ms_ssim": lambda x, y: fa.ms_ssim(x, y, data_range=255.0, reduction="none"),
    }
    alone = {(k, p): f(*xy).cpu() for k, f in calls.items()
             for p, xy in (("ab", (ta, tb)), ("cd", (tc, td)))}
    # the values are the oracle's too (MS-SSIM's three-launch sums: 1e-12)
    assert np.allclose(alone["ms_ssim", "ab"].numpy(), ref.ms_ssim(a, b, 255.0, reduction="none"),
                       rtol=REL, atol=0)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    outs = []
    for _ in range(3):
        for k, f in calls.items():
            with torch.cuda.stream(s1):
                outs.append((k, "ab", f(ta, tb)))
            with torch.cuda.stream(s2):
                outs.append((k, "cd", f(tc, td)))
    torch.cuda.synchronize()
    for k, p, o in outs:
        assert torch.equal(o.cpu(), alone[k, p]), (k, p)
    kinds = {"ssim", "gmsd", "ms"}
    keys = [key for key in backend._stream_acc
            if key[0] in kinds and key[2] in (s1.cuda_stream, s2.cuda_stream)]
    assert len(keys) == 6, keys
    for key in keys:
        assert not bool(backend._stream_acc[key].any()), key


@pytest.mark.parametrize("nc", [(3, 4), (300, 3), (2, 420)])
@pytest.mark.parametrize("per_image", [False, True])
@pytest.mark.parametrize("weights", [(0.0448, 0.2856, 0.3001, 0.2363, 0.1333), (0.5, 0.0, 1.0)])
def test_ms_head_matches_the_torch_expression(gpu, per_image, weights, nc):
    """fa_gpu_ms_ssim_head and its backward (the training path's scale
    product, channel mean and batch mean in one launch each way) against
    torch's autograd of the same expression on the same float64 plane means:
    values and gradients to 1e-14 relative, with zero, negative and NaN means,
    a zero weight, and one scale that needs no gradient; NaN and inf land
    where torch puts them.  Shapes: one LDS chunk of images, several (300
    images), and images whose C * M factors exceed the LDS (420 channels: one
    thread per image)."""
    from frame_analytics_amd.functional import _MsHead

    m, (n, c) = len(weights), nc
    gen = torch.Generator().manual_seed(17 + m)
    base = (torch.rand((m, n, c), generator=gen, dtype=torch.float64) * 1.1 - 0.05)
    base[0, 0, 0] = 0.0                      # zero factor under a fractional weight: inf
    base[1, 1 % n, 2 % c] = -0.2             # clamped: no gradient through it
    base[m - 1, 2 % n, 3 % c] = float("nan")
    base = base.to(gpu)
    expo = torch.tensor(weights, dtype=torch.float64, device=gpu).view(-1, 1, 1)
    ref_terms = [base[i].clone().requires_grad_(True) for i in range(m)]
    got_terms = [base[i].clone().requires_grad_(i != 1) for i in range(m)]
    prod = torch.stack(ref_terms).clamp_min(0.0).pow(expo).prod(dim=0).mean(dim=1)
    want = prod if per_image else prod.mean()
    got = _MsHead.apply(tuple(weights), per_image, *got_terms)
    assert got.shape == want.shape and got.dtype == torch.float64
    w_, g_ = want.detach().cpu(), got.detach().cpu()
    assert torch.equal(torch.isnan(g_), torch.isnan(w_))
    fin = torch.isfinite(w_)
    assert torch.allclose(g_[fin], w_[fin], rtol=1e-13, atol=0)
    up = torch.rand(want.shape, generator=gen, dtype=torch.float64).to(gpu) + 0.5
    want_g = torch.autograd.grad(want, ref_terms, up)
    got_g = torch.autograd.grad(got, [t for t in got_terms if t.requires_grad], up)
    want_g = [v for i, v in enumerate(want_g) if i != 1]
    for i, (a, b) in enumerate(zip(got_g, want_g)):
        a, b = a.cpu(), b.cpu()
        assert torch.equal(torch.isnan(a), torch.isnan(b)), i
        assert torch.equal(torch.isinf(a), torch.isinf(b)), i
        f = torch.isfinite(b)
        assert torch.allclose(a[f], b[f], rtol=1e-14, atol=1e-300), i


def test_ms_ssim_training_path_uses_the_head(gpu):
    """fa.ms_ssim with a gradient combines the scales in the head's two
    launches (no torch product in the graph) and its value and gradient
    match the same loss combined by the torch expression."""
    from frame_analytics_amd import backend, functional

    a, b = u8_pair((2, 3, 192, 224), 8.0, seed=23)
    x0 = torch.from_numpy(a).to(gpu).float() / 255.0
    y = torch.from_numpy(b).to(gpu).float() / 255.0
    x = x0.clone().requires_grad_(True)
    before = backend.native_calls["fa_gpu_ms_ssim_head_backward"]
    loss = 1.0 - fa.ms_ssim(x, y, data_range=1.0)
    loss.backward()
    assert backend.native_calls["fa_gpu_ms_ssim_head_backward"] == before + 1
    xr = x0.clone().requires_grad_(True)
    orig = backend.ms_head_available
    try:
        backend.ms_head_available = lambda terms: False  # the torch expression instead
        loss_r = 1.0 - fa.ms_ssim(xr, y, data_range=1.0)
        loss_r.backward()
    finally:
        backend.ms_head_available = orig
    assert abs(float(loss.detach()) - float(loss_r.detach())) <= 1e-14
    err = float((x.grad - xr.grad).abs().max() / xr.grad.abs().max())
    assert err <= 1e-12, err
    del functional


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32, torch.float64])
def test_gmsd_one_launch_floating_input(gpu, dt):
    """fa_gpu_gmsd_once over floating input finishes in its launch as over
    uint8: statistics within 1e-12 (mean) / 1e-10 (std) of the two-launch
    form, the same bits twice, the batch means, the oracle to 1e-6, the
    accumulator zero; and a NaN or an inf sample makes its image's
    statistics and the batch means NaN (the two-launch form and the oracle
    agree) while the other image stays finite."""
    from frame_analytics_amd import backend

    a, b = u8_pair((3, 3, 200, 264), 9.0, seed=61)
    x = torch.from_numpy(a).to(gpu).to(dt)
    y = torch.from_numpy(b).to(gpu).to(dt)
    T, eps = 170.0, (1e-6 * 255.0) ** 2
    acc = torch.zeros(backend._ACC_WORDS["gmsd"], dtype=torch.int64, device=gpu)
    m2, s2, _ = _gmsd_call("fa_gpu_gmsd", x, y, T, eps, True)
    m1, s1, bt = _gmsd_call("fa_gpu_gmsd_once", x, y, T, eps, True, acc=acc, batch=True)
    assert not bool(acc.any())
    assert np.all(np.abs(m1 - m2) <= 1e-12 * np.abs(m2)), (m1, m2)
    assert np.all(np.abs(s1 - s2) <= 1e-10 * np.abs(s2)), (s1, s2)
    assert abs(bt[0] - m1.mean()) <= 1e-12 * abs(m1.mean())
    again = _gmsd_call("fa_gpu_gmsd_once", x, y, T, eps, True, acc=acc, batch=True)
    for u, v in zip((m1, s1, bt), again):
        assert np.array_equal(u, v)
    xo, yo = x.double().cpu().numpy(), y.double().cpu().numpy()
    m0, s0 = ref.gmsd_stats(xo, yo, 255.0)
    assert np.all(np.abs(s1 - s0) <= REL * np.abs(s0)) and np.all(np.abs(m1 - m0) <= REL * np.abs(m0))
    xb = x.clone()
    xb[0, 1, 50, 60] = float("nan")
    xb[2, 0, 10, 200] = float("inf")
    mb, sb, bb = _gmsd_call("fa_gpu_gmsd_once", xb, y, T, eps, True, acc=acc, batch=True)
    mr, sr, _ = _gmsd_call("fa_gpu_gmsd", xb, y, T, eps, True)
    assert not bool(acc.any())
    for got in (mb, sb, mr, sr):
        assert np.isnan(got[0]) and np.isnan(got[2]) and np.isfinite(got[1])
    assert np.isnan(bb[0]) and np.isnan(bb[1])
    assert abs(mb[1] - mr[1]) <= 1e-12 * abs(mr[1]) and abs(sb[1] - sr[1]) <= 1e-10 * abs(sr[1])
    with np.errstate(invalid="ignore"):
        mo, so = ref.gmsd_stats(xb.double().cpu().numpy(), yo, 255.0)
    assert np.isnan(mo[0]) and np.isnan(so[2])
    # a clean call after them on the same accumulator
    mc, sc, _ = _gmsd_call("fa_gpu_gmsd_once", x, y, T, eps, True, acc=acc)
    assert np.array_equal(mc, m1) and np.array_equal(sc, s1)
