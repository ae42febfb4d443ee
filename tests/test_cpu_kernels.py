"""The host kernel library (libfa_cpu.so, include/fa_cpu_abi.h) against the
float64 oracle, the reference CPU kernels' golden values, and the reference
CPU build itself where it is present (oracle/_ref).

Bars: uint8 MSE / L1 bit-exact (integer sums both sides); every other value
within 1e-6 relative of the float64 oracle (SSIM within 1e-6 absolute, its
float32 arithmetic); float64 input within 1e-12.  These run on the CPU only.
"""

from __future__ import annotations

import ctypes
import math
import threading

import numpy as np
import pytest
import torch

from frame_analytics_amd import backend
from oracle import ref_cpu
from oracle import reference as ref
from tests.conftest import natural_pair, u8_pair

PSNR_NONE = -1.0e300
OPS = {"mse": 0, "l1": 1, "charbonnier": 2, "huber": 3}
CODES = {torch.uint8: 0, torch.float16: 1, torch.bfloat16: 2, torch.float32: 3,
         torch.float64: 4}


@pytest.fixture(scope="module")
def lib():
    lib = backend.load_cpu()
    if lib is None:
        pytest.skip(f"host kernel library unavailable ({backend._cpu_state})")
    return lib


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


def _pixel(lib, x, y, op, param=0.0, bias=PSNR_NONE, per_image=False):
    x, y = x.contiguous(), y.contiguous()
    n = x.shape[0]
    out = torch.zeros(n if per_image else 1, dtype=torch.float64)
    rc = lib.fa_cpu_pixel_reduce(x.data_ptr(), y.data_ptr(), CODES[x.dtype], n,
                                 x.numel() // n, OPS[op], float(param), float(bias),
                                 int(per_image), out.data_ptr())
    assert rc == 0
    return out.numpy() if per_image else float(out[0])


def _win(k, s=1.5):
    return torch.from_numpy(ref.gaussian_window_1d(k, s).astype(np.float32))


def _consts(L):
    return 0.5 * L, (0.01 * L) ** 2, (0.03 * L) ** 2


def _ssim(lib, x, y, L, k=11, want_map=False):
    n, c, h, w = x.shape
    win = _win(k)
    shift, C1, C2 = _consts(L)
    sums = torch.zeros(n * c, dtype=torch.float64)
    smap = torch.zeros((n, c, h - k + 1, w - k + 1), dtype=torch.float32) if want_map else None
    rc = lib.fa_cpu_ssim(x.data_ptr(), y.data_ptr(), CODES[x.dtype], n, c, h, w,
                         win.data_ptr(), k, shift, C1, C2,
                         None if smap is None else smap.data_ptr(), sums.data_ptr())
    assert rc == 0
    return sums.numpy(), (None if smap is None else smap.numpy())


def _ssim_cs(lib, x, y, L, k=11):
    n, c, h, w = x.shape
    win = _win(k)
    shift, C1, C2 = _consts(L)
    s = torch.zeros(n * c, dtype=torch.float64)
    cs = torch.zeros(n * c, dtype=torch.float64)
    rc = lib.fa_cpu_ssim_cs(x.data_ptr(), y.data_ptr(), CODES[x.dtype], n, c, h, w,
                            win.data_ptr(), k, shift, C1, C2, s.data_ptr(), cs.data_ptr())
    assert rc == 0
    return s.numpy().reshape(n, c), cs.numpy().reshape(n, c)


def _gmsd(lib, x, y, L, down=True):
    n, c, h, w = x.shape
    m = torch.zeros(n, dtype=torch.float64)
    sd = torch.zeros(n, dtype=torch.float64)
    T, eps = 170.0 * (L / 255.0) ** 2, (1e-6 * L) ** 2
    rc = lib.fa_cpu_gmsd(x.data_ptr(), y.data_ptr(), CODES[x.dtype], n, c, h, w, T, eps,
                         int(down), m.data_ptr(), sd.data_ptr())
    assert rc == 0
    return m.numpy(), sd.numpy()


def _float_pair(shape, dt, sigma=0.03, seed=0):
    rng = np.random.default_rng(seed)
    a = rng.random(shape)
    b = np.clip(a + rng.normal(0, sigma, shape), 0, 1)
    x, y = _t(a).to(dt), _t(b).to(dt)
    return x, y, x.double().numpy(), y.double().numpy()


# --------------------------------------------------------------------------- #
# pixel reductions
# --------------------------------------------------------------------------- #


@pytest.mark.parametrize("shape", [(1, 1, 1, 1), (2, 3, 17, 29), (3, 1, 64, 1000),
                                   (1, 3, 513, 257)])
def test_u8_mse_l1_exact(lib, shape):
    a, b = u8_pair(shape, 12.0, seed=sum(shape))
    x, y = _t(a), _t(b)
    assert _pixel(lib, x, y, "mse") == ref.mse(a, b)
    assert _pixel(lib, x, y, "l1") == ref.l1(a, b)
    per = _pixel(lib, x, y, "mse", per_image=True)
    assert np.array_equal(per, ref.mse(a, b, reduction="none"))
    assert np.array_equal(_pixel(lib, x, y, "l1", per_image=True), ref.l1(a, b, reduction="none"))


def test_u8_extremes_exact(lib):
    """All-255 against all-0 over more than 2^24 elements per image: the
    integer sums cannot round (65025 * n and 255 * n exactly)."""
    a = torch.full((2, 3, 2048, 2731), 255, dtype=torch.uint8)
    b = torch.zeros_like(a)
    assert _pixel(lib, a, b, "mse") == 65025.0
    assert _pixel(lib, b, a, "l1") == 255.0
    assert np.array_equal(_pixel(lib, a, b, "mse", per_image=True), [65025.0, 65025.0])


def test_psnr_bias_and_identical_inputs(lib):
    a, b = u8_pair((3, 3, 40, 50), 6.0, seed=4)
    x, y = _t(a), _t(b)
    bias = 10 * math.log10(255.0 ** 2)
    got = _pixel(lib, x, y, "mse", bias=bias, per_image=True)
    want = ref.psnr(a, b, 255.0, reduction="none")
    assert np.abs(got - want).max() < 1e-12
    assert _pixel(lib, x, x, "mse", bias=bias) == math.inf
    per = _pixel(lib, x, x, "mse", bias=bias, per_image=True)
    assert np.all(np.isinf(per)) and np.all(per > 0)


@pytest.mark.parametrize("dt", [torch.uint8, torch.float16, torch.bfloat16, torch.float32,
                                torch.float64])
@pytest.mark.parametrize("op,param", [("mse", 0.0), ("l1", 0.0), ("charbonnier", 1e-6),
                                      ("charbonnier", 9.0), ("huber", 0.05), ("huber", 4.0)])
def test_pixel_ops_all_dtypes(lib, dt, op, param):
    if dt == torch.uint8:
        a, b = u8_pair((2, 3, 31, 77), 10.0, seed=1)
        x, y, xa, ya = _t(a), _t(b), a.astype(np.float64), b.astype(np.float64)
    else:
        x, y, xa, ya = _float_pair((2, 3, 31, 77), dt)
    eps = math.sqrt(param) if op == "charbonnier" else None
    fn = {"mse": lambda: ref.mse(xa, ya, reduction="none"),
          "l1": lambda: ref.l1(xa, ya, reduction="none"),
          "charbonnier": lambda: ref.charbonnier(xa, ya, eps, reduction="none"),
          "huber": lambda: ref.huber(xa, ya, param, reduction="none")}[op]
    want = fn()
    got = _pixel(lib, x, y, op, param, per_image=True)
    # Charbonnier's root is float32 below float64 input (reference fa_cuda.cu:262-277)
    tol = 1e-6 if (op == "charbonnier" and dt != torch.float64) else 1e-12
    assert np.abs(got / want - 1).max() < tol
    tot = _pixel(lib, x, y, op, param)
    assert abs(tot / want.mean() - 1) < tol


# --------------------------------------------------------------------------- #
# SSIM
# --------------------------------------------------------------------------- #


@pytest.mark.parametrize("k", [3, 5, 7, 9, 11])
def test_ssim_windows_and_map(lib, k):
    a, b = u8_pair((2, 3, 45, 70), 15.0, seed=k)
    x, y = _t(a), _t(b)
    sums, smap = _ssim(lib, x, y, 255.0, k, want_map=True)
    s_map, _ = ref.ssim_maps(a, b, 255.0, win_size=k)
    assert np.abs(smap - s_map).max() < 2e-6
    npix = (45 - k + 1) * (70 - k + 1)
    plane_means = s_map.reshape(6, -1).mean(axis=1)
    assert np.abs(sums / npix - plane_means).max() < 1e-6


@pytest.mark.parametrize("h,w", [(11, 11), (11, 300), (300, 11), (12, 13), (97, 131)])
def test_ssim_edge_shapes(lib, h, w):
    """One output row / column, and band boundaries that are not multiples
    of the band height."""
    a, b = natural_pair(h, w, 9.0, seed=h * w)
    a8, b8 = a.astype(np.uint8)[None, None], b.astype(np.uint8)[None, None]
    sums, _ = _ssim(lib, _t(a8), _t(b8), 255.0)
    npix = (h - 10) * (w - 10)
    assert abs(sums[0] / npix - ref.ssim(a8, b8, 255.0)) < 1e-6


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32, torch.float64])
def test_ssim_float_dtypes(lib, dt):
    x, y, xa, ya = _float_pair((2, 2, 40, 53), dt, sigma=0.05, seed=3)
    sums, _ = _ssim(lib, x, y, 1.0)
    s_map, _ = ref.ssim_maps(xa, ya, 1.0)
    want = s_map.reshape(4, -1).mean(axis=1)
    # float64 arithmetic, but the C ABI's window weights are float32
    tol = 1e-9 if dt == torch.float64 else 1e-6
    assert np.abs(sums / s_map[0, 0].size - want).max() < tol


def test_ssim_cs_against_oracle_terms(lib):
    a, b = u8_pair((2, 3, 64, 80), 20.0, seed=9)
    s, cs = _ssim_cs(lib, _t(a), _t(b), 255.0)
    os_, ocs = ref.ms_ssim_terms(a, b, 255.0, scales=1)[0]
    assert np.abs(s - os_).max() < 1e-6 and np.abs(cs - ocs).max() < 1e-6


def test_ssim_rejects_bad_arguments(lib):
    x = torch.zeros((1, 1, 16, 16), dtype=torch.uint8)
    p = x.data_ptr()
    w = _win(11)
    out = torch.zeros(1, dtype=torch.float64)
    call = lib.fa_cpu_ssim
    assert call(p, p, 0, 1, 1, 16, 16, w.data_ptr(), 4, 0.0, 1.0, 1.0, None, out.data_ptr()) == 3
    assert call(p, p, 0, 1, 1, 16, 16, w.data_ptr(), 13, 0.0, 1.0, 1.0, None, out.data_ptr()) == 3
    assert call(p, p, 0, 1, 1, 8, 16, w.data_ptr(), 11, 0.0, 1.0, 1.0, None, out.data_ptr()) == 2
    assert call(p, p, 9, 1, 1, 16, 16, w.data_ptr(), 11, 0.0, 1.0, 1.0, None, out.data_ptr()) == 1
    assert call(p, p, 0, 1, 1, 16, 16, None, 11, 0.0, 1.0, 1.0, None, out.data_ptr()) == 5
    assert call(None, p, 0, 1, 1, 16, 16, w.data_ptr(), 11, 0.0, 1.0, 1.0, None,
                out.data_ptr()) == 5
    assert lib.fa_cpu_pixel_reduce(p, p, 0, 1, 256, 7, 0.0, PSNR_NONE, 0, out.data_ptr()) == 4
    assert lib.fa_cpu_pixel_reduce(p, p, 0, 0, 256, 0, 0.0, PSNR_NONE, 0, out.data_ptr()) == 2
    assert lib.fa_cpu_gmsd(p, p, 0, 1, 1, 5, 5, 170.0, 0.0, 1, out.data_ptr(),
                           out.data_ptr()) == 2


# --------------------------------------------------------------------------- #
# GMSD
# --------------------------------------------------------------------------- #


@pytest.mark.parametrize("down", [True, False])
@pytest.mark.parametrize("h,w", [(6, 6), (3, 3), (67, 91), (129, 64), (200, 301)])
def test_gmsd_u8_shapes(lib, down, h, w):
    if down and (h < 6 or w < 6):
        pytest.skip("downsampled plane smaller than the 3x3 filter")
    a, b = u8_pair((2, 3, h, w), 10.0, seed=h + w)
    m, sd = _gmsd(lib, _t(a), _t(b), 255.0, down)
    om, osd = ref.gmsd_stats(a, b, 255.0, downsample=down)
    # d = 1 - q is float32-accurate: within 1e-6 of d, far inside 1e-6 of q
    assert np.abs(m - om).max() <= 1e-6 * np.abs(1 - om).max() + 1e-15
    assert np.abs(sd - osd).max() <= 1e-6 * osd.max() + 1e-15


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32, torch.float64])
@pytest.mark.parametrize("sigma", [0.2, 0.01, 1e-5])
def test_gmsd_float_dtypes(lib, dt, sigma):
    """float32 arithmetic below float64 input, formed on x + y and x - y so
    that nearly identical images keep their accuracy (sigma 1e-5)."""
    x, y, xa, ya = _float_pair((2, 2, 66, 70), dt, sigma=sigma, seed=8)
    for down in (True, False):
        m, sd = _gmsd(lib, x, y, 1.0, down)
        # the cancellation-free float64 statistics: at sigma 1e-5 the spread
        # of q is ~1e-9, below what gmsd_stats' rounded q resolves
        om, osd = ref.gmsd_stats_hp(xa, ya, 1.0, downsample=down)
        tol = 1e-12 if dt == torch.float64 else 1e-6
        assert np.abs(m - om).max() <= tol * np.abs(1 - om).max() + 1e-16
        assert np.abs(sd / osd - 1).max() < tol


def test_gmsd_identical_inputs_are_exact(lib):
    a, _ = u8_pair((2, 3, 40, 40), 1.0, seed=2)
    m, sd = _gmsd(lib, _t(a), _t(a), 255.0)
    assert np.array_equal(m, [1.0, 1.0]) and np.array_equal(sd, [0.0, 0.0])


# --------------------------------------------------------------------------- #
# against the reference CPU kernels
# --------------------------------------------------------------------------- #


def test_against_reference_cpu_golden_vectors(lib):
    """The committed golden values of the reference's CPU kernels
    (tests/golden/ref_cpu_vectors.json): MSE / L1 exactly, SSIM / CS / GMSD
    within the reference's 5e-6 gate (its kernels compute in float32)."""
    from tests.test_oracle import _golden, _golden_inputs

    for case in _golden()["cases"]:
        a, b = _golden_inputs(case)
        exp = case["expect"]
        x, y = _t(a), _t(b)
        assert _pixel(lib, x, y, "mse") == exp["mse"]
        assert _pixel(lib, x, y, "l1") == exp["l1"]
        n, c, h, w = a.shape
        sums, _ = _ssim(lib, x, y, 255.0)
        per_image = sums.reshape(n, c).sum(axis=1) / ((h - 10) * (w - 10) * c)
        assert np.abs(per_image - np.array(exp["ssim_per_image"])).max() < 5e-6
        if "ssim_cs" in exp:
            s, cs = _ssim_cs(lib, x, y, 255.0)
            assert np.abs(s - np.array(exp["ssim_cs"][0])).max() < 5e-6
            assert np.abs(cs - np.array(exp["ssim_cs"][1])).max() < 5e-6
        if "gmsd" in exp:
            m, sd = _gmsd(lib, x, y, 255.0)
            assert np.abs(m - np.array(exp["gmsd"][0])).max() < 5e-6
            assert np.abs(sd - np.array(exp["gmsd"][1])).max() < 5e-6


@pytest.mark.skipif(not ref_cpu.available(), reason="oracle/_ref not built")
def test_against_reference_cpu_live(lib):
    for h, w, kind in [(64, 64, "uniform"), (127, 233, "natural"), (200, 232, "natural")]:
        a, b = natural_pair(h, w, 8.0, seed=h * w, kind=kind)
        a8, b8 = a.astype(np.uint8)[None, None], b.astype(np.uint8)[None, None]
        x, y = _t(a8), _t(b8)
        assert _pixel(lib, x, y, "mse") == ref_cpu.pixel_reduce(a8, b8, "mse")
        assert _pixel(lib, x, y, "l1") == ref_cpu.pixel_reduce(a8, b8, "l1")
        sums, _ = _ssim(lib, x, y, 255.0)
        assert abs(sums[0] / ((h - 10) * (w - 10)) - ref_cpu.ssim_per_image(a8, b8)[0]) < 5e-6
        for down in (True, False):
            m, sd = _gmsd(lib, x, y, 255.0, down)
            rm, rsd = ref_cpu.gmsd(a8, b8, downsample=down)
            assert abs(m[0] - rm[0]) < 5e-6 and abs(sd[0] - rsd[0]) < 5e-6


# --------------------------------------------------------------------------- #
# pool and routing
# --------------------------------------------------------------------------- #


def test_concurrent_calls_are_serialised_and_deterministic(lib):
    """ctypes drops the GIL: calls from several threads share one pool, which
    runs one job at a time; every result equals the single-threaded one."""
    a, b = u8_pair((2, 3, 120, 160), 12.0, seed=5)
    x, y = _t(a), _t(b)
    want_s, _ = _ssim(lib, x, y, 255.0)
    want_g = _gmsd(lib, x, y, 255.0)
    errors = []

    def work():
        try:
            for _ in range(5):
                s, _ = _ssim(lib, x, y, 255.0)
                g = _gmsd(lib, x, y, 255.0)
                assert np.array_equal(s, want_s)
                assert np.array_equal(g[0], want_g[0]) and np.array_equal(g[1], want_g[1])
                assert _pixel(lib, x, y, "mse") == ref.mse(a, b)
        except Exception as exc:  # surfaced below
            errors.append(exc)

    threads = [threading.Thread(target=work) for _ in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    assert lib.fa_cpu_num_threads() >= 1


def test_many_small_jobs_from_several_threads(lib):
    """Tiny jobs finish without waiting for sleeping workers, and a worker that
    wakes late cannot take a task of the next job: 4 threads x 150 mixed calls
    on small planes, every result equal to the single-threaded one."""
    a, b = u8_pair((2, 3, 24, 40), 12.0, seed=8)
    x, y = _t(a), _t(b)
    want = (_ssim(lib, x, y, 255.0)[0], _pixel(lib, x, y, "l1"), _gmsd(lib, x, y, 255.0, False))
    errors = []

    def work(k):
        try:
            for i in range(150):
                j = (i + k) % 3
                if j == 0:
                    assert np.array_equal(_ssim(lib, x, y, 255.0)[0], want[0])
                elif j == 1:
                    assert _pixel(lib, x, y, "l1") == want[1]
                else:
                    m, sd = _gmsd(lib, x, y, 255.0, False)
                    assert np.array_equal(m, want[2][0]) and np.array_equal(sd, want[2][1])
        except Exception as exc:  # surfaced below
            errors.append(exc)

    threads = [threading.Thread(target=work, args=(k,)) for k in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors


def test_python_api_routes_cpu_tensors_to_the_library(lib, monkeypatch):
    """Inference calls on CPU tensors go through fa_cpu_*; a gradient request
    and luma (formed first, then the kernel) still give the oracle's values."""
    import frame_analytics_amd as fa

    calls = []
    real = backend.load_cpu

    def spy():
        got = real()
        calls.append(got is not None)
        return got

    monkeypatch.setattr(backend, "load_cpu", spy)
    a, b = u8_pair((2, 3, 48, 64), 9.0, seed=6)
    x, y = _t(a), _t(b)
    assert float(fa.mse(x, y)) == ref.mse(a, b)
    assert abs(float(fa.ssim(x, y, data_range=255.0)) - ref.ssim(a, b, 255.0)) < 1e-6
    m, sd = ref.gmsd_stats(a, b, 255.0)
    assert abs(float(fa.gmsd(x, y, data_range=255.0)) - sd.mean()) < 1e-6 * sd.mean()
    assert abs(float(fa.psnr(x, y)) - ref.psnr(a, b)) < 1e-12
    assert calls and all(calls)
    # luma on CPU: the plane is formed in torch, the kernel reduces it
    yl = float(fa.mse(x, y, luma="bt601"))
    la, lb = ref.rgb_to_luma(a, "bt601"), ref.rgb_to_luma(b, "bt601")
    assert abs(yl / ref.mse(la, lb) - 1) < 1e-6


def test_pool_size_is_fixed_after_first_use(lib):
    n = lib.fa_cpu_num_threads()
    assert lib.fa_cpu_set_num_threads(n + 3) == n
    assert n >= 1
