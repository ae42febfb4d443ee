"""GPU parity of the matrix-core SSIM forward (fa_ssim_mfma.hip).

uint8 inputs whose rows and planes are 8-byte aligned (W % 8 == 0) take the
MFMA kernel, and so do the float32 levels of a uint8 MS-SSIM pyramid when the
caller flags them (FA_DTYPE_U8_PYRAMID); everything else takes the vector-ALU
strip kernel.  Both are held
to the float64 oracle at the north star's bar (SSIM values within 1e-6
relative; float32 map elements within 2e-5 absolute, their mean error within
2e-7 and 99% of them within 2e-6), and to each other:
``FA_SSIM_MFMA=0`` in the environment selects the strip kernel for a call.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import frame_analytics_amd as fa
from oracle import reference as ref
from tests.conftest import natural_pair, u8_pair

pytestmark = pytest.mark.gpu

REL = 1e-6
MAP_ABS = 2e-5    # every element (the reference's own gate is 5e-5)
# The error distribution over the map: both kernels share the float32
# epilogue's floor (mean 5e-8 to 1.2e-7, 99th percentile up to 1.2e-6,
# isolated low-variance pixels up to ~6e-6, measured on MI355X).  A low fp16
# piece of the window or of H lost on any operand class would put every
# element near 1e-4, far past these.
MAP_MEAN = 2e-7
MAP_P99 = 2e-6


def _rel(got, want):
    return abs(got - want) / max(abs(want), 1e-12)


class _VectorAlu:
    """Runs the body with the matrix-core kernel switched off."""

    def __enter__(self):
        os.environ["FA_SSIM_MFMA"] = "0"

    def __exit__(self, *exc):
        os.environ.pop("FA_SSIM_MFMA", None)


def _u8(a):
    """The planes as uint8 (natural_pair returns integer-valued float64)."""
    a = np.asarray(a)
    return a if a.dtype == np.uint8 else np.clip(np.rint(a), 0, 255).astype(np.uint8)


def _check(a, b, gpu, win=11, sigma=1.5, L=255.0, K=(0.01, 0.03)):
    a, b = _u8(a), _u8(b)
    assert a.dtype == np.uint8 and a.shape[-1] % 8 == 0  # the matrix-core kernel's inputs
    x = torch.as_tensor(a, device=gpu)
    y = torch.as_tensor(b, device=gpu)
    kw = dict(data_range=L, win_size=win, sigma=sigma, K=K)
    want = ref.ssim(a, b, L, win_size=win, sigma=sigma, K=K, reduction="none")
    want_map = ref.ssim(a, b, L, win_size=win, sigma=sigma, K=K, return_map=True)
    got = fa.ssim(x, y, reduction="none", **kw).cpu().numpy()
    for g, w in zip(got, want):
        assert _rel(float(g), float(w)) <= REL, (a.shape, win, sigma, g, w)
    m = fa.ssim(x, y, return_map=True, **kw).double().cpu().numpy()
    assert m.shape == want_map.shape
    err = np.abs(m - want_map)
    assert float(err.max()) <= MAP_ABS
    if err.size >= 1000:  # a distribution: a few pixels would be one pixel's error
        assert float(err.mean()) <= MAP_MEAN, (a.shape, win, sigma, float(err.mean()))
        assert float(np.quantile(err, 0.99)) <= MAP_P99, (a.shape, win, sigma)
    with _VectorAlu():
        alu = fa.ssim(x, y, reduction="none", **kw).cpu().numpy()
    for g, w in zip(got, alu):
        assert _rel(float(g), float(w)) <= REL, ("vs strip kernel", g, w)
    return got


# heights around the 16-row blocks, widths around the 64-column workgroup strips
@pytest.mark.parametrize("h,w", [(16, 16), (26, 24), (27, 32), (42, 72), (43, 80), (58, 136),
                                 (75, 200), (121, 264), (160, 320), (301, 1024)])
def test_shapes(gpu, h, w):
    a, b = natural_pair(h, w, 9.0, seed=h * 1000 + w)
    _check(a[None, None], b[None, None], gpu)


# the narrowest rows the kernel takes (W = 8: one 8-byte chunk, clamped for
# every lane past it) and the shortest maps (Hout = 1)
@pytest.mark.parametrize("h,w,win", [(8, 8, 3), (9, 16, 5), (20, 8, 7), (11, 24, 11), (3, 40, 3)])
def test_narrow_and_short(gpu, h, w, win):
    a, b = natural_pair(h, w, 11.0, seed=h * 100 + w + win)
    _check(a[None, None], b[None, None], gpu, win=win)


@pytest.mark.parametrize("win", [3, 5, 7, 9, 11])
@pytest.mark.parametrize("sigma", [0.5, 1.5, 4.0])
def test_windows(gpu, win, sigma):
    a, b = natural_pair(67, 96, 6.0, seed=win * 10 + int(sigma * 2))
    _check(a[None, None], b[None, None], gpu, win=win, sigma=sigma)


def test_batch_and_channels(gpu):
    a, b = u8_pair((3, 3, 90, 136), 10.0, seed=7)
    _check(a, b, gpu)


def test_baseline_generator_1080p(gpu):
    a, b = u8_pair((1, 3, 1080, 1920), 8.0, seed=11)
    _check(a, b, gpu)


@pytest.mark.parametrize("kind", ["flat", "uniform"])
def test_extremes(gpu, kind):
    h, w = 48, 64
    if kind == "flat":  # far apart means, no variance: the tiny-SSIM corner
        a = np.full((1, 1, h, w), 255, np.uint8)
        b = np.zeros((1, 1, h, w), np.uint8)
    else:
        rng = np.random.default_rng(5)
        a = rng.integers(0, 256, (1, 1, h, w), dtype=np.uint8)
        b = rng.integers(0, 256, (1, 1, h, w), dtype=np.uint8)
    x = torch.as_tensor(a, device=gpu)
    y = torch.as_tensor(b, device=gpu)
    want_map = ref.ssim(a, b, 255.0, return_map=True)
    m = fa.ssim(x, y, data_range=255.0, return_map=True).double().cpu().numpy()
    assert float(np.abs(m - want_map).max()) <= MAP_ABS
    # SSIM ~ 1e-4 for the flat pair: float32 moments cancel to ~1e-7 absolute
    # there (sigma^2 = E (x'-y')^2 - (ux - uy)^2 with both terms near 65025),
    # in this kernel and in the strip kernel alike
    want = ref.ssim(a, b, 255.0)
    bar = REL * abs(want) if abs(want) > 0.1 else 1e-7
    got = float(fa.ssim(x, y, data_range=255.0))
    assert abs(got - want) <= bar, (got, want)
    with _VectorAlu():
        alu = float(fa.ssim(x, y, data_range=255.0))
    assert abs(alu - want) <= bar, (alu, want)


def test_identity_is_one(gpu):
    a, _ = natural_pair(80, 128, 5.0, seed=2)
    x = torch.as_tensor(_u8(a)[None, None], device=gpu)
    got = fa.ssim(x, x.clone(), data_range=255.0, return_map=True)
    assert float((got.double() - 1.0).abs().max()) <= 1e-6


@pytest.mark.parametrize("L", [1.0, 100.0, 255.0])
def test_data_range(gpu, L):
    a, b = natural_pair(50, 88, 12.0, seed=int(L))
    _check(a[None, None], b[None, None], gpu, L=L)


def test_views_aligned_and_not(gpu):
    # crops read in place: crops of 8 and 4 pixels (bases 8- and 4-byte
    # aligned, widths multiples of 8) stay on the matrix cores, so each gives
    # the bits of the same crop copied out contiguously; a 2-pixel crop (width
    # 156) moves to the strip kernel; all match the oracle
    a, b = u8_pair((2, 3, 96, 160), 9.0, seed=13)
    x = torch.as_tensor(a, device=gpu)
    y = torch.as_tensor(b, device=gpu)
    for c in (8, 4, 2):
        want = ref.ssim(a[..., c:-c, c:-c], b[..., c:-c, c:-c], 255.0, reduction="none")
        got = fa.ssim(x, y, data_range=255.0, crop_border=c, reduction="none").cpu().numpy()
        for g, w in zip(got, want):
            assert _rel(float(g), float(w)) <= REL, (c, g, w)
        if c % 4 == 0:
            xc = x[..., c:-c, c:-c].contiguous()
            yc = y[..., c:-c, c:-c].contiguous()
            copy = fa.ssim(xc, yc, data_range=255.0, reduction="none").cpu().numpy()
            assert np.array_equal(got, copy), (c, got, copy)
            with _VectorAlu():
                alu = fa.ssim(x, y, data_range=255.0, crop_border=c,
                              reduction="none").cpu().numpy()
            assert not np.array_equal(got, alu), c  # the strip kernel's bits differ


def test_ms_ssim_four_pixel_crop_in_place(gpu):
    # a 4-pixel crop of 264-wide frames: a 4-byte aligned base, and every
    # scale's width (256 .. 16) a multiple of 8, so the crop read in place
    # takes the three-launch matrix-core path and gives the bits of the
    # contiguous copy
    a, b = u8_pair((2, 3, 200, 264), 9.0, seed=21)
    x = torch.as_tensor(a, device=gpu)
    y = torch.as_tensor(b, device=gpu)
    got = fa.ms_ssim(x, y, data_range=255.0, crop_border=4, reduction="none").cpu().numpy()
    copy = fa.ms_ssim(x[..., 4:-4, 4:-4].contiguous(), y[..., 4:-4, 4:-4].contiguous(),
                      data_range=255.0, reduction="none").cpu().numpy()
    assert np.array_equal(got, copy), (got, copy)
    want = ref.ms_ssim(a[..., 4:-4, 4:-4], b[..., 4:-4, 4:-4], 255.0, reduction="none")
    for g, w in zip(got, want):
        assert _rel(float(g), float(w)) <= REL, (g, w)


# MS-SSIM over uint8: scale 0 (SSIM and cs sums plus the first pyramid level,
# 2 x 2 means written by the same kernel) runs on the matrix cores
@pytest.mark.parametrize("shape", [(1, 1, 176, 176), (2, 3, 200, 264), (1, 3, 361, 648),
                                   (3, 1, 190, 184), (22, 3, 176, 176)])  # 66 planes: two-launch reduction
def test_ms_ssim(gpu, shape):
    a, b = u8_pair(shape, 9.0, seed=sum(shape))
    x = torch.as_tensor(a, device=gpu)
    y = torch.as_tensor(b, device=gpu)
    want = ref.ms_ssim(a, b, 255.0, reduction="none")
    got = fa.ms_ssim(x, y, data_range=255.0, reduction="none").cpu().numpy()
    for g, w in zip(got, want):
        assert _rel(float(g), float(w)) <= REL, (shape, g, w)
    with _VectorAlu():
        alu = fa.ms_ssim(x, y, data_range=255.0, reduction="none").cpu().numpy()
    for g, w in zip(got, alu):
        assert _rel(float(g), float(w)) <= REL, ("vs strip kernel", g, w)


@pytest.mark.parametrize("w", [136, 134])  # 134: rows of 134 bytes take the strip kernel
@pytest.mark.parametrize("pool", ["float32", "float16"])
@pytest.mark.parametrize("kernel", ["auto", "strip"])
def test_ms_ssim_pyramid_level_exact(gpu, w, pool, kernel):
    # the level the CS pass writes is the exact 2 x 2 mean of the uint8 input,
    # in float32 or in float16 (a multiple of 1/4 in [0, 255] is exact there)
    import contextlib
    import ctypes

    from frame_analytics_amd import backend

    a, b = u8_pair((2, 3, 90, w), 7.0, seed=4)
    x = torch.as_tensor(a, device=gpu)
    y = torch.as_tensor(b, device=gpu)
    n, c, h, w = a.shape
    win = fa.gaussian_window_1d(11, 1.5, device=gpu, dtype=torch.float32)
    bpp = backend.workspace_slots("ssim", h, w, 11)
    part = torch.empty((n * c, bpp), dtype=torch.float64, device=gpu)
    part_cs = torch.empty_like(part)
    out_s = torch.empty(n * c, dtype=torch.float64, device=gpu)
    out_cs = torch.empty_like(out_s)
    pdt = getattr(torch, pool)
    px = torch.full((n, c, h // 2, w // 2), -1.0, device=gpu, dtype=pdt)
    py = torch.full_like(px, -1.0)
    slots = ctypes.c_int(0)
    stream = torch.cuda.current_stream().cuda_stream
    with _VectorAlu() if kernel == "strip" else contextlib.nullcontext():
        rc = backend.call_gpu("fa_gpu_ssim_cs_ex", x.data_ptr(), y.data_ptr(), 0, n, c, h, w,
                              None, None, None, win.data_ptr(), 11, 127.5, (0.01 * 255) ** 2,
                              (0.03 * 255) ** 2, part.data_ptr(), part_cs.data_ptr(), bpp,
                              out_s.data_ptr(), out_cs.data_ptr(), ctypes.addressof(slots),
                              px.data_ptr(), py.data_ptr(), 3 if pool == "float32" else 1, 0,
                              stream)
    assert rc == 0
    want_x = ref.avg_pool2(a.astype(np.float64))
    want_y = ref.avg_pool2(b.astype(np.float64))
    assert np.array_equal(px.cpu().numpy().astype(np.float64), want_x)
    assert np.array_equal(py.cpu().numpy().astype(np.float64), want_y)
    s_ref, cs_ref = ref.ssim_maps(a.astype(float), b.astype(float))
    got_s = out_s.cpu().numpy().reshape(n, c)
    got_cs = out_cs.cpu().numpy().reshape(n, c)
    assert np.allclose(got_s, s_ref.mean(axis=(-2, -1)), rtol=1e-6, atol=0)
    assert np.allclose(got_cs, cs_ref.mean(axis=(-2, -1)), rtol=1e-6, atol=0)


@pytest.mark.parametrize("kernel", ["auto", "strip"])
@pytest.mark.parametrize("w", [136, 134])
def test_cs_sums_alone_uint8(gpu, kernel, w):
    # uint8 input, the cs sums alone (partial null, as MS-SSIM asks below its
    # coarsest scale) with the float16 level: cs matches the oracle, the
    # level is exact
    import contextlib

    from frame_analytics_amd import backend

    a, b = u8_pair((2, 3, 90, w), 7.0, seed=5)
    x = torch.as_tensor(a, device=gpu)
    y = torch.as_tensor(b, device=gpu)
    n, c = a.shape[:2]
    win = fa.gaussian_window_1d(11, 1.5, device=gpu, dtype=torch.float32)
    with _VectorAlu() if kernel == "strip" else contextlib.nullcontext():
        ps, pcs, sl, npix, px, py = backend.ssim_cs_partials(
            x, y, win, 127.5, (0.01 * 255) ** 2, (0.03 * 255) ** 2, torch.float16,
            ssim_sums=False)
    assert ps is None and px.dtype == torch.float16
    _, cs_ref = ref.ssim_maps(a.astype(float), b.astype(float))
    cs_mean = pcs.reshape(-1)[: n * c * sl].reshape(n * c, sl).sum(1).cpu().numpy() / npix
    assert np.allclose(cs_mean, cs_ref.mean(axis=(-2, -1)).reshape(-1), rtol=REL, atol=0)
    assert np.array_equal(px.cpu().numpy().astype(np.float64), ref.avg_pool2(a.astype(float)))
    assert np.array_equal(py.cpu().numpy().astype(np.float64), ref.avg_pool2(b.astype(float)))


def test_float16_level_only_below_uint8(gpu):
    # a float16 level is exact only for the 2 x 2 means of bytes: any other
    # input, or luma, is refused
    import ctypes

    from frame_analytics_amd import backend

    n, c, h, w = 1, 3, 32, 32
    win = fa.gaussian_window_1d(11, 1.5, device=gpu, dtype=torch.float32)
    bpp = backend.workspace_slots("ssim", h, w, 11)
    part = torch.empty((3, bpp), dtype=torch.float64, device=gpu)
    px = torch.empty((n, c, h // 2, w // 2), dtype=torch.float16, device=gpu)
    slots = ctypes.c_int(0)
    stream = torch.cuda.current_stream().cuda_stream
    lw = (ctypes.c_double * 4)(0.299, 0.587, 0.114, 0.0)
    for dt, luma in ((torch.float32, None), (torch.float16, None), (torch.uint8, lw)):
        x = torch.zeros((n, c, h, w), dtype=dt, device=gpu)
        code = backend._DTYPE_CODE[dt]
        rc = backend.call_gpu("fa_gpu_ssim_cs_ex", x.data_ptr(), x.data_ptr(), code, n, c, h, w,
                              None, None, luma, win.data_ptr(), 11, 127.5, 1.0, 1.0,
                              part.data_ptr(), part.data_ptr(), bpp, None, None,
                              ctypes.addressof(slots), px.data_ptr(), px.data_ptr(), 1, 0,
                              stream)
        assert rc == 1, (dt, luma is not None)  # FA_E_DTYPE


@pytest.mark.parametrize("kernel", ["auto", "strip"])
@pytest.mark.parametrize("w", [120, 124])  # 124: the strip kernel reads the float16 level
def test_pyramid_level_flag_float16(gpu, kernel, w):
    # the first level of a uint8 pyramid in float16 (multiples of 1/4 in
    # [0, 255]) with FA_DTYPE_U8_PYRAMID: the statistics match the oracle and
    # the next level (float32) is exact
    import contextlib

    from frame_analytics_amd import backend

    rng = np.random.default_rng(w)
    n, c, h = 2, 3, 70
    ka = rng.integers(0, 1021, (n, c, h, w))
    kb = np.clip(ka + rng.integers(-36, 37, ka.shape), 0, 1020)
    a, b = ka / 4.0, kb / 4.0
    x = torch.as_tensor(a.astype(np.float16), device=gpu)
    y = torch.as_tensor(b.astype(np.float16), device=gpu)
    assert np.array_equal(x.cpu().numpy().astype(np.float64), a)
    win = fa.gaussian_window_1d(11, 1.5, device=gpu, dtype=torch.float32)
    C1, C2 = (0.01 * 255) ** 2, (0.03 * 255) ** 2
    s_ref, cs_ref = ref.ssim_maps(a, b)
    for sums in (True, False):  # with the SSIM sums, or the cs sums alone
        with _VectorAlu() if kernel == "strip" else contextlib.nullcontext():
            ps, pcs, sl, npix, px, py = backend.ssim_cs_partials(
                x, y, win, 127.5, C1, C2, torch.float32, u8_pyramid=True, ssim_sums=sums)
        cs_mean = pcs.reshape(-1)[: n * c * sl].reshape(n * c, sl).sum(1).cpu().numpy() / npix
        assert np.allclose(cs_mean, cs_ref.mean(axis=(-2, -1)).reshape(-1), rtol=REL, atol=0)
        if sums:
            s_mean = ps.reshape(-1)[: n * c * sl].reshape(n * c, sl).sum(1).cpu().numpy() / npix
            assert np.allclose(s_mean, s_ref.mean(axis=(-2, -1)).reshape(-1), rtol=REL, atol=0)
        assert px.dtype == torch.float32
        assert np.array_equal(px.cpu().numpy().astype(np.float64), ref.avg_pool2(a))
        assert np.array_equal(py.cpu().numpy().astype(np.float64), ref.avg_pool2(b))


@pytest.mark.parametrize("s", [1, 2, 4])
def test_pyramid_level_flag(gpu, s):
    # float32 samples that are multiples of 4^-s in [0, 255] (a uint8 pyramid
    # level) run on the matrix cores with FA_DTYPE_U8_PYRAMID; the statistics
    # and the next level match the strip kernel and the oracle
    from frame_analytics_amd import backend

    rng = np.random.default_rng(s)
    q = 4 ** s
    n, c, h, w = 2, 3, 70, 120
    ka = rng.integers(0, 255 * q + 1, (n, c, h, w))
    kb = np.clip(ka + rng.integers(-9 * q, 9 * q + 1, ka.shape), 0, 255 * q)
    a, b = (ka / q).astype(np.float32), (kb / q).astype(np.float32)
    x = torch.as_tensor(a, device=gpu)
    y = torch.as_tensor(b, device=gpu)
    win = fa.gaussian_window_1d(11, 1.5, device=gpu, dtype=torch.float32)
    C1, C2 = (0.01 * 255) ** 2, (0.03 * 255) ** 2
    s_ref, cs_ref = ref.ssim_maps(a.astype(np.float64), b.astype(np.float64))
    want_s = s_ref.mean(axis=(-2, -1)).reshape(-1)
    want_cs = cs_ref.mean(axis=(-2, -1)).reshape(-1)
    for flag in (True, False):
        for sums in (True, False):  # with the SSIM sums, or the cs sums alone
            ps, pcs, sl, npix, px, py = backend.ssim_cs_partials(
                x, y, win, 127.5, C1, C2, torch.float32, u8_pyramid=flag, ssim_sums=sums)
            assert (ps is None) == (not sums)
            # each plane's partials are packed at the used stride `sl`
            cs_mean = pcs.reshape(-1)[: n * c * sl].reshape(n * c, sl).sum(1).cpu().numpy() / npix
            assert np.allclose(cs_mean, want_cs, rtol=REL, atol=0), (flag, sums, cs_mean, want_cs)
            if sums:
                s_mean = ps.reshape(-1)[: n * c * sl].reshape(n * c, sl).sum(1).cpu().numpy() / npix
                assert np.allclose(s_mean, want_s, rtol=REL, atol=0), (flag, s_mean, want_s)
            assert np.array_equal(px.cpu().numpy().astype(np.float64),
                                  ref.avg_pool2(a.astype(np.float64)))
            assert np.array_equal(py.cpu().numpy().astype(np.float64),
                                  ref.avg_pool2(b.astype(np.float64)))


def test_pyramid_flag_is_an_ex_hint_only(gpu):
    from frame_analytics_amd import backend

    x = torch.zeros((1, 1, 32, 32), device=gpu)
    win = fa.gaussian_window_1d(11, 1.5, device=gpu, dtype=torch.float32)
    bpp = backend.workspace_slots("ssim", 32, 32, 11)
    part = torch.empty((1, bpp), dtype=torch.float64, device=gpu)
    o = torch.empty(1, dtype=torch.float64, device=gpu)
    stream = torch.cuda.current_stream().cuda_stream
    # the reference-shaped entry point refuses the flag
    rc = backend.call_gpu("fa_gpu_ssim_cs", x.data_ptr(), x.data_ptr(),
                          3 | backend.FA_DTYPE_U8_PYRAMID, 1, 1, 32, 32, win.data_ptr(), 11,
                          0.5, 1e-4, 9e-4, part.data_ptr(), part.data_ptr(), bpp, o.data_ptr(),
                          o.data_ptr(), 0, stream)
    assert rc == 1  # FA_E_DTYPE
    with pytest.raises(ValueError):
        backend.ssim_cs_partials(x.double(), x.double(), win, 0.5, 1e-4, 9e-4, None,
                                 u8_pyramid=True)


def _ssim_abi(name, x, y, win, acc=None, K=11, L=255.0, per_image=True, total=True):
    """fa_gpu_ssim (or fa_gpu_ssim_once with ``acc``) with both mean sinks:
    (per-image means, batch mean) as numpy float64."""
    from frame_analytics_amd import backend

    n, c, h, w = (int(v) for v in x.shape)
    bpp = backend.workspace_slots("ssim", h, w, K)
    part = torch.full((n * c, bpp), -3.0, dtype=torch.float64, device=x.device)
    out = torch.full((n + 1,), -3.0, dtype=torch.float64, device=x.device)
    stream = torch.cuda.current_stream().cuda_stream
    head = (x.data_ptr(), y.data_ptr(), 0, n, c, h, w)
    consts = (win.data_ptr(), K, L / 2, (0.01 * L) ** 2, (0.03 * L) ** 2, None,
              part.data_ptr(), bpp)
    sinks = (out.data_ptr() if per_image else None, out[n:].data_ptr() if total else None)
    if name == "fa_gpu_ssim":
        rc = backend.call_gpu(name, *head, *consts, *sinks, 0, stream)
    else:
        rc = backend.call_gpu(name, *head, None, None, None, *consts,
                              None if acc is None else acc.data_ptr(), *sinks, 0, stream)
    assert rc == 0, (name, rc)
    o = out.cpu().numpy()
    return o[:n], o[n]


@pytest.mark.parametrize("shape", [(8, 3, 1080, 1920), (1, 1, 96, 128), (3, 2, 200, 256),
                                   (256, 1, 24, 32), (257, 1, 24, 32)])
def test_one_launch_finish_matches_finalize(gpu, shape):
    """fa_gpu_ssim_once on the matrix-core forward: the per-image and batch
    means its workgroups finish through fixed-point atomics agree with
    fa_gpu_ssim's fixed-order float64 finalize to 1e-12 relative (the
    rounding is 2^-24 per workgroup sum at configs[1]), repeat bit for bit,
    and leave the accumulator zero, also over a second, smaller call and with
    only one of the two sinks.  257 images is past the one-launch form."""
    from frame_analytics_amd import backend

    a, b = u8_pair(shape, 8.0, seed=shape[0] + shape[2])
    x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    win = fa.gaussian_window_1d(11, 1.5, device=gpu, dtype=torch.float32)
    acc = torch.zeros(backend._ACC_WORDS["ssim"], dtype=torch.int64, device=gpu)
    p2, t2 = _ssim_abi("fa_gpu_ssim", x, y, win)
    p1, t1 = _ssim_abi("fa_gpu_ssim_once", x, y, win, acc)
    assert not bool(acc.any())
    assert np.all(np.abs(p1 - p2) <= 1e-12 * np.abs(p2)), (p1, p2)
    assert abs(t1 - t2) <= 1e-12 * abs(t2), (t1, t2)
    q1, u1 = _ssim_abi("fa_gpu_ssim_once", x, y, win, acc)
    assert np.array_equal(p1, q1) and t1 == u1
    k = max(1, shape[0] // 2)
    pk, tk = _ssim_abi("fa_gpu_ssim_once", x[:k], y[:k], win, acc)
    assert not bool(acc.any())
    assert np.all(np.abs(pk - p2[:k]) <= 1e-12 * np.abs(p2[:k]))
    for pi, to in ((True, False), (False, True)):
        pj, tj = _ssim_abi("fa_gpu_ssim_once", x, y, win, acc, per_image=pi, total=to)
        assert not bool(acc.any()), (pi, to)
        if pi:
            assert np.array_equal(pj, p1)
        else:
            assert tj == t1
    want = ref.ssim(a[:1].astype(np.float64), b[:1].astype(np.float64), 255.0)
    assert _rel(float(p1[0]), float(want)) <= REL


def test_one_launch_finish_without_workspace(gpu):
    """fa_gpu_ssim_once with a null `partial`: the launch that finishes the
    call does not read it (same means), the matrix-core kernel's for uint8 and
    the strip kernel's for float32; a map call returns FA_E_ARG and writes
    nothing."""
    from frame_analytics_amd import backend

    a, b = u8_pair((2, 3, 200, 256), 8.0, seed=77)
    x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    win = fa.gaussian_window_1d(11, 1.5, device=gpu, dtype=torch.float32)
    acc = torch.zeros(backend._ACC_WORDS["ssim"], dtype=torch.int64, device=gpu)
    st = torch.cuda.current_stream().cuda_stream
    bpp = backend.workspace_slots("ssim", 200, 256, 11)

    def two_launch(xx, yy, code):
        part = torch.empty((6, bpp), dtype=torch.float64, device=gpu)
        out = torch.empty((3,), dtype=torch.float64, device=gpu)
        assert backend.call_gpu("fa_gpu_ssim", xx.data_ptr(), yy.data_ptr(), code, 2, 3, 200, 256,
                                win.data_ptr(), 11, 127.5, (0.01 * 255) ** 2, (0.03 * 255) ** 2,
                                None, part.data_ptr(), bpp, out.data_ptr(), out[2:].data_ptr(),
                                0, st) == 0
        o = out.cpu().numpy()
        return o[:2], o[2]

    for xx, yy, code, with_map, ok in ((x, y, 0, False, True), (x.float(), y.float(), 3, False, True),
                                       (x, y, 0, True, False)):
        want_p, want_t = two_launch(xx, yy, code)
        out = torch.full((3,), -3.0, dtype=torch.float64, device=gpu)
        smap = (torch.empty((2, 3, 190, 246), dtype=torch.float32, device=gpu)
                if with_map else None)
        rc = backend.call_gpu("fa_gpu_ssim_once", xx.data_ptr(), yy.data_ptr(), code, 2, 3, 200,
                              256, None, None, None, win.data_ptr(), 11, 127.5,
                              (0.01 * 255) ** 2, (0.03 * 255) ** 2,
                              None if smap is None else smap.data_ptr(), None, bpp,
                              acc.data_ptr(), out.data_ptr(), out[2:].data_ptr(), 0, st)
        torch.cuda.synchronize()
        if ok:
            assert rc == 0
            o = out.cpu().numpy()
            assert np.all(np.abs(o[:2] - want_p) <= 1e-12 * np.abs(want_p))
            assert abs(o[2] - want_t) <= 1e-12 * abs(want_t)
        else:
            assert rc == 5 and bool((out == -3.0).all()), (code, with_map, rc)
        assert not bool(acc.any())


def test_zero_constants_keep_nan_like_the_reference(gpu):
    """uint8 SSIM with K = (0, 0): a patch flat in both frames is 0 / 0, NaN,
    and the reference's mean carries it (functional.py's float sums).  fa.ssim
    on uint8 hands the call its stream's accumulator, whose fixed-point words
    cannot hold NaN, so the one-launch finish declines such calls and the
    two-launch form returns NaN for that image and the batch; an image
    without a flat patch stays finite and matches the oracle, and the
    accumulator stays zero."""
    from frame_analytics_amd import backend

    a, b = u8_pair((2, 1, 96, 128), 8.0, seed=5)
    a[0, 0, 20:60, 30:80] = 100
    b[0, 0, 20:60, 30:80] = 100
    x, y = torch.from_numpy(a).to(gpu), torch.from_numpy(b).to(gpu)
    want = ref.ssim(a.astype(np.float64), b.astype(np.float64), 255.0, K=(0.0, 0.0),
                    reduction="none")
    assert np.isnan(want[0]) and np.isfinite(want[1])
    per = fa.ssim(x, y, data_range=255.0, K=(0.0, 0.0), reduction="none").cpu().numpy()
    tot = float(fa.ssim(x, y, data_range=255.0, K=(0.0, 0.0)))
    assert np.isnan(per[0]) and np.isnan(tot)
    assert _rel(float(per[1]), float(want[1])) <= REL
    st = torch.cuda.current_stream().cuda_stream
    acc = backend._stream_acc.get(("ssim", 0, st))
    assert acc is not None and not bool(acc.any())
