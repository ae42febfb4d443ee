"""GPU parity of the fused SSIM forward against the float64 oracle.

Bar (north star): SSIM values within 1e-6 relative of float64.  The SSIM map
is stored as float32; its elements are held to 2e-5 absolute (the reference's
own gate is 5e-5, validate.py:25).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import frame_analytics_amd as fa
from oracle import reference as ref
from tests.conftest import natural_pair, u8_pair

pytestmark = pytest.mark.gpu

REL = 1e-6
MAP_ABS = 2e-5

# the reference's accuracy-gate corpus (validate.py:80-87)
CASES = [(64, 64, "uniform", 20.0), (127, 233, "natural", 8.0), (256, 256, "natural", 3.0),
         (512, 384, "natural", 25.0), (720, 1280, "natural", 12.0), (33, 41, "flat", 5.0)]


def _rel(got, want):
    return abs(got - want) / max(abs(want), 1e-12)


@pytest.mark.parametrize("h,w,kind,noise", CASES)
def test_ssim_matches_oracle(gpu, h, w, kind, noise):
    a, b = natural_pair(h, w, noise, seed=h * w, kind=kind)
    want = ref.ssim(a[None, None], b[None, None], 255.0)
    want_map = ref.ssim(a[None, None], b[None, None], 255.0, return_map=True)
    for dt in (torch.uint8, torch.float32):
        x = torch.as_tensor(a, dtype=dt, device=gpu)
        y = torch.as_tensor(b, dtype=dt, device=gpu)
        got = float(fa.ssim(x, y, data_range=255.0))
        assert _rel(got, want) <= REL, (dt, got, want)
        m = fa.ssim(x, y, data_range=255.0, return_map=True)
        assert m.shape == (1, 1, h - 10, w - 10) and m.dtype == torch.float32
        err = float((m.double().cpu() - torch.from_numpy(want_map)).abs().max())
        assert err <= MAP_ABS, (dt, err)


@pytest.mark.parametrize("win", [3, 5, 7, 9, 11])
def test_window_sizes(gpu, win):
    a, b = natural_pair(97, 131, 7.0, seed=3)
    want = ref.ssim(a[None, None], b[None, None], 255.0, win_size=win)
    x = torch.as_tensor(a, dtype=torch.uint8, device=gpu)
    y = torch.as_tensor(b, dtype=torch.uint8, device=gpu)
    got = float(fa.ssim(x, y, data_range=255.0, win_size=win))
    assert _rel(got, want) <= REL, (win, got, want)
    got_map = fa.ssim(x, y, data_range=255.0, win_size=win, return_map=True).double().cpu()
    want_map = ref.ssim(a[None, None], b[None, None], 255.0, win_size=win, return_map=True)
    assert float((got_map - torch.from_numpy(want_map)).abs().max()) <= MAP_ABS


def test_sigma_and_K(gpu):
    a, b = natural_pair(90, 120, 10.0, seed=5)
    want = ref.ssim(a[None, None], b[None, None], 255.0, win_size=7, sigma=2.0, K=(0.02, 0.05))
    x = torch.as_tensor(a, dtype=torch.uint8, device=gpu)
    y = torch.as_tensor(b, dtype=torch.uint8, device=gpu)
    got = float(fa.ssim(x, y, data_range=255.0, win_size=7, sigma=2.0, K=(0.02, 0.05)))
    assert _rel(got, want) <= REL


@pytest.mark.parametrize("dt", [torch.uint8, torch.float16, torch.bfloat16, torch.float32,
                                torch.float64])
def test_dtypes(gpu, dt):
    a, b = natural_pair(97, 131, 7.0, seed=4)
    x = torch.as_tensor(a, dtype=dt, device=gpu)
    y = torch.as_tensor(b, dtype=dt, device=gpu)
    # the oracle sees the values the kernel sees (integers are exact in all five)
    want = ref.ssim(x.double().cpu().numpy()[None, None], y.double().cpu().numpy()[None, None],
                    255.0)
    got = float(fa.ssim(x, y, data_range=255.0))
    # float64 input runs a float64 kernel; the ABI hands it a float32 window,
    # whose rounding (6e-8 per tap) is what is left between it and the oracle
    tol = 1e-9 if dt == torch.float64 else REL
    assert _rel(got, want) <= tol, (dt, got, want)


def test_batch_channels_reduction_none(gpu):
    a, b = u8_pair((5, 3, 64, 80), 10.0, seed=9)
    x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    per = fa.ssim(x, y, data_range=255.0, reduction="none").cpu().numpy()
    want = ref.ssim(a, b, 255.0, reduction="none")
    assert per.shape == (5,)
    assert np.all(np.abs(per - want) <= REL * np.abs(want))
    assert abs(float(per.mean()) - float(fa.ssim(x, y, data_range=255.0))) < 1e-12
    m = fa.ssim(x, y, data_range=255.0, return_map=True)
    assert abs(float(m.double().mean()) - float(fa.ssim(x, y, data_range=255.0))) < 1e-7


def test_ranks_agree_bitwise(gpu):
    a, b = natural_pair(97, 131, 7.0, seed=3)
    x = torch.as_tensor(a, dtype=torch.uint8, device=gpu)
    y = torch.as_tensor(b, dtype=torch.uint8, device=gpu)
    v2 = float(fa.ssim(x, y, data_range=255.0))
    v3 = float(fa.ssim(x[None], y[None], data_range=255.0))
    v4 = float(fa.ssim(x[None, None], y[None, None], data_range=255.0))
    assert v2 == v3 == v4


def test_identity(gpu):
    x = torch.randint(0, 256, (2, 3, 64, 64), dtype=torch.uint8, device=gpu)
    assert abs(float(fa.ssim(x, x, data_range=255.0)) - 1.0) < 1e-6
    xf = torch.rand(2, 3, 64, 64, device=gpu)
    assert abs(float(fa.ssim(xf, xf, data_range=1.0)) - 1.0) < 1e-6


def test_luma_and_crop(gpu):
    rng = np.random.default_rng(12)
    a = rng.integers(0, 256, (3, 140, 176)).astype(np.float64)
    b = np.clip(a + 9.0 * rng.standard_normal(a.shape), 0, 255).round()
    ta = torch.from_numpy(a.astype(np.uint8))[None].to(gpu)
    tb = torch.from_numpy(b.astype(np.uint8))[None].to(gpu)
    for mode in ("bt601", "bt709", "matlab"):
        for cb in (0, 4):
            ya = ref.crop(ref.rgb_to_luma(a[None], mode), cb)
            yb = ref.crop(ref.rgb_to_luma(b[None], mode), cb)
            want = ref.ssim(ya, yb, 255.0)
            got = float(fa.ssim(ta, tb, data_range=255.0, luma=mode, crop_border=cb))
            assert _rel(got, want) <= REL, (mode, cb)
    for cb in (1, 3, 8):
        manual = float(fa.ssim(ta[..., cb:-cb, cb:-cb].contiguous(),
                               tb[..., cb:-cb, cb:-cb].contiguous(), data_range=255.0))
        assert abs(float(fa.ssim(ta, tb, data_range=255.0, crop_border=cb)) - manual) < 1e-12


@pytest.mark.parametrize("dt", [torch.uint8, torch.float16, torch.float32, torch.float64])
@pytest.mark.parametrize("mode", ["bt601", "bt709", "matlab"])
def test_luma_formed_in_kernel(gpu, mode, dt):
    """The kernel forms kr R + kg G + kb B + offset itself (fa_gpu_ssim_ex):
    per-image values and the map against the float64 oracle on luma planes."""
    rng = np.random.default_rng(5)
    a = rng.integers(0, 256, (2, 3, 97, 131)).astype(np.float64)
    b = np.clip(a + 11.0 * rng.standard_normal(a.shape), 0, 255).round()
    la, lb = ref.rgb_to_luma(a, mode), ref.rgb_to_luma(b, mode)
    x, y = torch.from_numpy(a).to(gpu, dt), torch.from_numpy(b).to(gpu, dt)
    want = ref.ssim(la, lb, 255.0, reduction="none")
    got = fa.ssim(x, y, data_range=255.0, luma=mode, reduction="none").cpu().numpy()
    assert np.all(np.abs(got - want) <= REL * np.abs(want)), (got, want)
    if dt != torch.float64:  # a float64 map takes the portable path
        wmap = ref.ssim(la, lb, 255.0, return_map=True)
        gmap = fa.ssim(x, y, data_range=255.0, luma=mode, return_map=True).cpu().double().numpy()
        assert gmap.shape == wmap.shape and np.abs(gmap - wmap).max() <= MAP_ABS


@pytest.mark.parametrize("cb", [3, 4, 7])
def test_ms_ssim_luma_and_crop_in_place(gpu, cb):
    """MS-SSIM's first scale reads the crop in place and forms luma itself;
    the pyramid below it is float64."""
    rng = np.random.default_rng(cb)
    a = rng.integers(0, 256, (2, 3, 200, 240)).astype(np.float64)
    b = np.clip(a + 9.0 * rng.standard_normal(a.shape), 0, 255).round()
    x = torch.from_numpy(a.astype(np.uint8)).to(gpu)
    y = torch.from_numpy(b.astype(np.uint8)).to(gpu)
    for mode in (None, "bt601", "matlab"):
        ca, cbb = ref.crop(a, cb), ref.crop(b, cb)
        if mode:
            ca, cbb = ref.rgb_to_luma(ca, mode), ref.rgb_to_luma(cbb, mode)
        want = ref.ms_ssim(ca, cbb, 255.0, reduction="none")
        got = fa.ms_ssim(x, y, data_range=255.0, luma=mode, crop_border=cb,
                         reduction="none").cpu().numpy()
        assert np.all(np.abs(got - want) <= REL * np.abs(want)), (mode, got, want)


def test_configs1_full_size(gpu):
    """8x3x1080x1920 uint8 (sigma 8).  Image 0 against the oracle;
    the batch through size-independent properties (per-image consistency,
    map mean = per-image value, map shape)."""
    a, b = u8_pair((8, 3, 1080, 1920), 8.0, seed=1)
    x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    per = fa.ssim(x, y, data_range=255.0, reduction="none").cpu().numpy()
    total = float(fa.ssim(x, y, data_range=255.0))
    want0 = ref.ssim(a[:1], b[:1], 255.0)
    assert _rel(float(per[0]), want0) <= REL, (per[0], want0)
    single = float(fa.ssim(x[5:6], y[5:6], data_range=255.0))
    assert abs(single - float(per[5])) < 1e-12
    assert abs(total - float(per.mean())) < 1e-12
    m = fa.ssim(x, y, data_range=255.0, return_map=True)
    assert m.shape == (8, 3, 1070, 1910)
    pm = m.double().mean(dim=(1, 2, 3)).cpu().numpy()
    assert np.all(np.abs(pm - per) < 1e-7)


@pytest.mark.portable_ok  # a 13-wide window has no kernel on purpose
def test_native_hint_and_errors(gpu):
    x = torch.zeros(1, 1, 32, 32, device=gpu)
    with pytest.raises(ValueError):
        fa.ssim(x, torch.zeros(1, 1, 32, 33, device=gpu))
    with pytest.raises(ValueError):
        fa.ssim(torch.zeros(1, 1, 8, 8, device=gpu), torch.zeros(1, 1, 8, 8, device=gpu))
    # a 13-wide window has no kernel: "native" must say so, "auto" must still answer
    a, b = natural_pair(64, 64, 5.0, seed=1)
    ta = torch.as_tensor(a, dtype=torch.float32, device=gpu)
    tb = torch.as_tensor(b, dtype=torch.float32, device=gpu)
    with pytest.raises(RuntimeError):
        fa.ssim(ta, tb, data_range=255.0, win_size=13, backend_hint="native")
    want = ref.ssim(a[None, None], b[None, None], 255.0, win_size=13)
    assert _rel(float(fa.ssim(ta, tb, data_range=255.0, win_size=13)), want) < 1e-5


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("fn", ["ssim", "ms_ssim", "gmsd", "gms"])
def test_autocast_does_not_move_the_metric(gpu, dt, fn):
    """A measurement does not change with the surrounding autocast context,
    with or without a gradient (reference test_training_metrics.py:506-518)."""
    torch.manual_seed(0)
    x = torch.rand(1, 3, 192, 192, device=gpu, requires_grad=True)
    y = (x.detach() + 0.05 * torch.randn_like(x)).clamp(0, 1)
    call = getattr(fa, fn)
    plain = float(call(x, y, data_range=1.0).detach())
    with torch.autocast("cuda", dtype=dt):
        cast = call(x, y, data_range=1.0)
    assert abs(float(cast.detach()) - plain) <= 1e-6 * max(abs(plain), 1e-3)
    cast.backward()  # the differentiable kernels run under autocast too
    assert x.grad is not None and torch.isfinite(x.grad).all()
    with torch.no_grad(), torch.autocast("cuda", dtype=dt):
        assert abs(float(call(x, y, data_range=1.0)) - plain) <= 1e-6 * max(abs(plain), 1e-3)


_DT = {torch.uint8: 0, torch.float16: 1, torch.bfloat16: 2, torch.float32: 3, torch.float64: 4}


def _ssim_call(name, x, y, acc=None, luma=None, K=11, L=255.0, partial=True):
    """fa_gpu_ssim_ex, or fa_gpu_ssim_once with ``acc``, on views of x / y
    (element strides passed through) with optional luma: (status,
    per-image means, batch mean) as numpy float64."""
    from frame_analytics_amd import backend

    n, c, h, w = (int(v) for v in x.shape)
    cout = 1 if luma is not None else c
    bpp = backend.workspace_slots("ssim", h, w, K)
    part = (torch.full((n * cout, bpp), -3.0, dtype=torch.float64, device=x.device)
            if partial else None)
    out = torch.full((n + 1,), -3.0, dtype=torch.float64, device=x.device)
    st = torch.cuda.current_stream().cuda_stream
    win = fa.gaussian_window_1d(K, 1.5, device=x.device, dtype=torch.float32)
    xs = (ctypes.c_int64 * 3)(x.stride(0), x.stride(1), x.stride(2))
    ys = (ctypes.c_int64 * 3)(y.stride(0), y.stride(1), y.stride(2))
    lw = (ctypes.c_double * 4)(*luma) if luma is not None else None
    args = [x.data_ptr(), y.data_ptr(), _DT[x.dtype], n, c, h, w, xs, ys, lw, win.data_ptr(), K,
            L / 2, (0.01 * L) ** 2, (0.03 * L) ** 2, None,
            None if part is None else part.data_ptr(), bpp]
    if name == "fa_gpu_ssim_once":
        args.append(None if acc is None else acc.data_ptr())
    rc = backend.call_gpu(name, *args, out.data_ptr(), out[n:].data_ptr(), 0, st)
    o = out.cpu().numpy()
    return rc, o[:n], o[n]


@pytest.mark.parametrize("dt", [torch.float32, torch.float64, torch.float16, torch.bfloat16])
def test_strip_one_launch_finish(gpu, dt):
    """The strip kernel's one-launch finish (fa_gpu_ssim_once over float
    input): per-image and batch means within 1e-12 of fa_gpu_ssim_ex's float64
    finalize, the same bits on a repeat, the accumulator zero after every
    call (a second, smaller call included), with a null workspace (the launch
    does not read it), over cropped views and with luma formed in the kernel;
    the oracle agrees.  A call whose counts do not fit the words (C * tiles
    per image >= 4096) takes the workspace and the two-launch form."""
    from frame_analytics_amd import backend

    g = torch.Generator(device="cpu").manual_seed(31)
    base = torch.rand((3, 3, 150, 212), generator=g, dtype=torch.float64) * 255.0
    noisy = (base + 9.0 * torch.randn(base.shape, generator=g, dtype=torch.float64)).clamp(0, 255)
    x, y = base.to(gpu, dt), noisy.to(gpu, dt)
    acc = torch.zeros(backend._ACC_WORDS["ssim"], dtype=torch.int64, device=gpu)
    bt601 = (0.299, 0.587, 0.114, 0.0)
    for xx, yy, luma in ((x, y, None), (x[:, :, 3:-2, 5:-4], y[:, :, 3:-2, 5:-4], None),
                         (x, y, bt601)):
        rc2, p2, t2 = _ssim_call("fa_gpu_ssim_ex", xx, yy, luma=luma)
        rc1, p1, t1 = _ssim_call("fa_gpu_ssim_once", xx, yy, acc, luma=luma, partial=False)
        assert rc1 == 0 and rc2 == 0
        assert not bool(acc.any())
        assert np.all(np.abs(p1 - p2) <= 1e-12 * np.abs(p2)), (p1, p2)
        assert abs(t1 - t2) <= 1e-12 * abs(t2)
        _, q1, u1 = _ssim_call("fa_gpu_ssim_once", xx, yy, acc, luma=luma, partial=False)
        assert np.array_equal(p1, q1) and t1 == u1
        _, pk, tk = _ssim_call("fa_gpu_ssim_once", xx[:1], yy[:1], acc, luma=luma, partial=False)
        assert not bool(acc.any())
        assert abs(pk[0] - p2[0]) <= 1e-12 * abs(p2[0])
    xo = x.double().cpu().numpy()
    yo = y.double().cpu().numpy()
    _, p1, _ = _ssim_call("fa_gpu_ssim_once", x, y, acc, partial=False)
    want = ref.ssim(xo, yo, 255.0, reduction="none")
    assert np.all(np.abs(p1 - want) <= 1e-6 * np.abs(want))
    if dt == torch.float32:
        # 4096 channels of one image (one tile per 24 x 24 plane): 4096
        # contributions per word is past 4095, so the call needs the
        # workspace (refused without it)
        wide_x = torch.rand((1, 4096, 24, 24), generator=g, dtype=torch.float64).to(gpu, dt) * 255
        wide_y = (wide_x + 5.0).clamp(0, 255)
        rc0, _, _ = _ssim_call("fa_gpu_ssim_once", wide_x, wide_y, acc, partial=False)
        rcw, pw, tw = _ssim_call("fa_gpu_ssim_once", wide_x, wide_y, acc)
        _, pr, tr = _ssim_call("fa_gpu_ssim_ex", wide_x, wide_y)
        assert (rc0, rcw) == (5, 0) and np.array_equal(pw, pr) and tw == tr
        assert not bool(acc.any())


def test_strip_one_launch_finish_carries_nan(gpu):
    """Floating input can hold NaN and inf, which make SSIM values NaN; the
    one-launch finish flags such a workgroup sum instead of packing it, so an
    image with a NaN or an inf sample comes out NaN, as do the batch mean and
    the two-launch form and the oracle, while the other image stays finite;
    the accumulator and its flags are zero afterwards, and a clean call right
    after gives finite means again."""
    from frame_analytics_amd import backend

    g = torch.Generator(device="cpu").manual_seed(8)
    base = torch.rand((3, 1, 96, 128), generator=g, dtype=torch.float64) * 255.0
    noisy = (base + 6.0 * torch.randn(base.shape, generator=g, dtype=torch.float64)).clamp(0, 255)
    x, y = base.to(gpu, torch.float32), noisy.to(gpu, torch.float32)
    xb = x.clone()
    xb[0, 0, 40, 50] = float("nan")
    xb[2, 0, 10, 100] = float("inf")
    acc = torch.zeros(backend._ACC_WORDS["ssim"], dtype=torch.int64, device=gpu)
    rc1, p1, t1 = _ssim_call("fa_gpu_ssim_once", xb, y, acc, partial=False)
    rc2, p2, t2 = _ssim_call("fa_gpu_ssim_ex", xb, y)
    assert rc1 == 0 and rc2 == 0
    want = ref.ssim(xb.double().cpu().numpy(), y.double().cpu().numpy(), 255.0, reduction="none")
    for got in (p1, p2, want):
        assert np.isnan(got[0]) and np.isnan(got[2]) and np.isfinite(got[1])
    assert np.isnan(t1) and np.isnan(t2)
    assert abs(p1[1] - p2[1]) <= 1e-12 * abs(p2[1])
    assert not bool(acc.any())
    _, pc, tc = _ssim_call("fa_gpu_ssim_once", x, y, acc, partial=False)
    assert np.all(np.isfinite(pc)) and np.isfinite(tc)
    assert not bool(acc.any())
    # through the public call: fa.ssim hands the stream's accumulator
    per = fa.ssim(xb, y, data_range=255.0, reduction="none").cpu().numpy()
    assert np.isnan(per[0]) and np.isnan(per[2]) and abs(per[1] - p2[1]) <= 1e-12 * abs(p2[1])
    assert np.isnan(float(fa.ssim(xb, y, data_range=255.0)))
