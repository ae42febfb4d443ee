"""API contract on CPU tensors (the portable eager path) -- runs without a GPU.

These mirror the reference's contract tests (test_metrics.py,
test_training_metrics.py): argument handling, reductions, luma / crop, error
behaviour and the module wrappers.  The portable path computes in float32 like
the reference's, so values are held to the reference's gates (5e-6 SSIM-family,
exact integer MSE).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import frame_analytics_amd as fa
from oracle import reference as ref
from tests.conftest import natural_pair, u8_pair

TOL = 5e-6


def test_ssim_mse_psnr_cpu():
    a, b = natural_pair(97, 131, 7.0, seed=3)
    x = torch.as_tensor(a, dtype=torch.uint8)
    y = torch.as_tensor(b, dtype=torch.uint8)
    assert abs(float(fa.ssim(x, y, data_range=255.0)) - ref.ssim(a[None, None], b[None, None])) < TOL
    a8, b8 = a.astype(np.uint8)[None, None], b.astype(np.uint8)[None, None]
    assert float(fa.mse(x, y)) == ref.mse(a8, b8)
    assert abs(float(fa.psnr(x, y)) - float(ref.psnr(a8, b8))) < 1e-9
    v2 = float(fa.ssim(x, y, data_range=255.0))
    assert v2 == float(fa.ssim(x[None], y[None], data_range=255.0)) == float(
        fa.ssim(x[None, None], y[None, None], data_range=255.0))


def test_training_metrics_cpu():
    a, b = natural_pair(200, 232, 8.0, seed=432)
    x = torch.as_tensor(a, dtype=torch.uint8)[None, None]
    y = torch.as_tensor(b, dtype=torch.uint8)[None, None]
    assert abs(float(fa.ms_ssim(x, y, data_range=255.0)) - ref.ms_ssim(a[None, None], b[None, None])) < TOL
    m, s = ref.gmsd_stats(a[None, None], b[None, None], 255.0)
    assert abs(float(fa.gmsd(x, y, data_range=255.0)) - s[0]) < TOL
    assert abs(float(fa.gms(x, y, data_range=255.0)) - m[0]) < TOL
    assert abs(float(fa.l1(x, y)) - ref.l1(a, b)) < 1e-9
    assert abs(float(fa.charbonnier(x, y)) - ref.charbonnier(a, b)) < 1e-6
    assert abs(float(fa.huber(x, y, delta=4.0)) - ref.huber(a, b, 4.0)) < 1e-9


def test_reductions_and_shapes():
    a, b = u8_pair((5, 1, 64, 64), 20.0, seed=1)
    x, y = torch.from_numpy(a), torch.from_numpy(b)
    for fn in (fa.ssim, fa.mse, fa.l1, fa.huber, fa.charbonnier):
        per = fn(x, y, reduction="none")
        assert per.shape == (5,)
    assert fa.psnr(x, y, reduction="none").shape == (5,)
    assert fa.ssim(x, y, return_map=True).shape == (5, 1, 54, 54)
    assert abs(float(fa.ssim(x, y, reduction="none").mean()) - float(fa.ssim(x, y))) < 1e-9


def test_errors():
    x = torch.zeros(1, 1, 32, 32)
    with pytest.raises(ValueError):
        fa.ssim(x, torch.zeros(1, 1, 32, 33))
    with pytest.raises(ValueError):
        fa.ssim(torch.zeros(1, 1, 8, 8), torch.zeros(1, 1, 8, 8))
    with pytest.raises(ValueError):
        fa.mse(x, x, reduction="sum")
    with pytest.raises(ValueError):
        fa.huber(x, x, delta=0.0)
    with pytest.raises(ValueError):
        fa.mse(x, x, crop_border=16)
    with pytest.raises(ValueError):
        fa.mse(x, x, crop_border=-1)
    with pytest.raises(ValueError):
        fa.psnr(torch.zeros(1, 3, 32, 32), torch.zeros(1, 3, 32, 32), luma="rec2020")
    with pytest.raises(TypeError):
        fa.psnr(torch.zeros(1, 3, 32, 32), torch.zeros(1, 3, 32, 32), luma=3)
    with pytest.raises(ValueError):
        fa.psnr(torch.zeros(1, 2, 32, 32), torch.zeros(1, 2, 32, 32), luma=True)
    with pytest.raises(ValueError, match="too small"):
        fa.ms_ssim(torch.zeros(1, 1, 175, 300), torch.zeros(1, 1, 175, 300), data_range=1.0)
    with pytest.raises(ValueError):
        fa.ssim(torch.zeros(2, 2, 2, 16, 16), torch.zeros(2, 2, 2, 16, 16))


def test_luma_crop_cpu():
    rng = np.random.default_rng(12)
    a = rng.integers(0, 256, (3, 60, 70)).astype(np.float64)
    b = np.clip(a + 9.0 * rng.standard_normal(a.shape), 0, 255).round()
    x = torch.from_numpy(a.astype(np.uint8))[None]
    y = torch.from_numpy(b.astype(np.uint8))[None]
    for mode in ("bt601", "bt709", "matlab"):
        ya, yb = ref.crop(ref.rgb_to_luma(a[None], mode), 2), ref.crop(ref.rgb_to_luma(b[None], mode), 2)
        assert abs(float(fa.ssim(x, y, luma=mode, crop_border=2)) - ref.ssim(ya, yb)) < TOL
        assert abs(float(fa.psnr(x, y, luma=mode, crop_border=2)) - float(ref.psnr(ya, yb))) < 1e-5
    assert float(fa.psnr(x, y, luma=True)) == float(fa.psnr(x, y, luma="bt601"))


def test_modules_agree_with_functions():
    a, b = natural_pair(200, 232, 8.0, seed=7)
    x = torch.as_tensor(a, dtype=torch.uint8)[None, None]
    y = torch.as_tensor(b, dtype=torch.uint8)[None, None]
    pairs = [
        (fa.SSIM(data_range=255.0)(x, y), fa.ssim(x, y, data_range=255.0)),
        (fa.MSSSIM(data_range=255.0)(x, y), fa.ms_ssim(x, y, data_range=255.0)),
        (fa.GMSD(data_range=255.0)(x, y), fa.gmsd(x, y, data_range=255.0)),
        (fa.MSE()(x, y), fa.mse(x, y)),
        (fa.PSNR()(x, y), fa.psnr(x, y)),
        (fa.L1()(x, y), fa.l1(x, y)),
        (fa.Charbonnier(eps=2.0)(x, y), fa.charbonnier(x, y, eps=2.0)),
        (fa.Huber(delta=3.0)(x, y), fa.huber(x, y, delta=3.0)),
    ]
    for got, want in pairs:
        assert float(got) == float(want)
    assert abs(float(fa.GMSD(data_range=255.0).loss(x, y))
               - (1.0 - float(fa.gms(x, y, data_range=255.0)))) < 1e-12


def test_gradients_cpu_portable():
    x = torch.rand(1, 1, 64, 64, requires_grad=True)
    y = torch.rand(1, 1, 64, 64)
    fa.SSIM(data_range=1.0).loss(x, y).backward()
    assert torch.isfinite(x.grad).all() and float(x.grad.abs().sum()) > 0
    for fn in (fa.l1, fa.charbonnier, fa.huber):
        z = torch.rand(1, 3, 32, 32, requires_grad=True)
        fn(z, torch.rand(1, 3, 32, 32)).backward()
        assert torch.isfinite(z.grad).all()


def test_status_without_gpu():
    st = fa.backend_status()
    if not torch.cuda.is_available():
        assert st["available"] is False and st["error"]


def test_no_grad_still_reaches_the_native_kernel():
    """requires_grad on a tensor nobody differentiates does not decline the
    inference kernels (reference test_training_metrics.py:466-478)."""
    from frame_analytics_amd import backend

    x = torch.rand(1, 1, 64, 64, requires_grad=True)
    y = torch.rand(1, 1, 64, 64)
    assert not backend._usable(x, y)
    with torch.no_grad():
        assert backend._usable(x, y)
    with torch.inference_mode():
        assert backend._usable(x, y)


def test_declined_kernel_warns_once_and_falls_back(monkeypatch):
    """A kernel that returns a non-zero status makes the call warn once and
    take the portable path, as the reference's backend does (backend.py:213-224)."""
    import warnings

    from frame_analytics_amd import backend

    lib = backend.load_cpu()
    if lib is None:
        pytest.skip("host kernel library unavailable")
    monkeypatch.setattr(lib, "fa_cpu_pixel_reduce", lambda *args: 5)
    monkeypatch.setattr(backend, "_declined_seen", set())
    g = torch.Generator().manual_seed(3)
    x = torch.randint(0, 256, (2, 3, 20, 24), generator=g, dtype=torch.uint8)
    y = torch.randint(0, 256, (2, 3, 20, 24), generator=g, dtype=torch.uint8)
    want = ((x.double() - y.double()) ** 2).mean()
    with pytest.warns(RuntimeWarning, match="declined"):
        got = fa.mse(x, y)
    assert abs(float(got) - float(want)) < 1e-9
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        assert abs(float(fa.mse(x, y)) - float(want)) < 1e-9  # warned once only


def test_failed_one_launch_call_drops_the_stream_accumulator(monkeypatch):
    """A one-launch call keeps its stream's accumulator zero between calls;
    one that fails may have stopped between launches (MS-SSIM makes three),
    so the backend drops that accumulator and the next call starts on a new
    one.  FA_E_ARG (refused before any launch) retries with the workspace and
    keeps it.  No kernel runs: the library calls are replaced."""
    from frame_analytics_amd import backend

    acc = torch.zeros(8, dtype=torch.int64)
    key = ("ms", 0, 12345)
    monkeypatch.setattr(backend, "_stream_acc", {key: acc})
    codes = []
    monkeypatch.setattr(backend, "call_gpu", lambda name, *args: codes.pop(0))

    codes[:] = [5, 0]  # refused without the workspace, done with it
    backend._run_or_needs_workspace("fa_gpu_ssim_once", (), lambda: (), acc)
    assert backend._stream_acc.get(key) is acc and not codes

    codes[:] = [5, 6]  # refused, then failed with the workspace
    with pytest.raises(backend.KernelError):
        backend._run_or_needs_workspace("fa_gpu_ssim_once", (), lambda: (), acc)
    assert key not in backend._stream_acc and not codes

    backend._stream_acc[key] = acc
    codes[:] = [6]  # failed outright: no retry
    with pytest.raises(backend.KernelError):
        backend._run_or_needs_workspace("fa_gpu_ssim_once", (), lambda: (), acc)
    assert key not in backend._stream_acc and not codes

    backend._stream_acc[key] = acc
    codes[:] = [6]
    with pytest.raises(backend.KernelError):
        backend._run_acc("fa_gpu_ms_ssim", acc)
    assert key not in backend._stream_acc
    codes[:] = [0]
    backend._stream_acc[key] = acc
    backend._run_acc("fa_gpu_ms_ssim", acc)
    assert backend._stream_acc.get(key) is acc


def test_scale_product_gradient_matches_torch_autograd():
    """MS-SSIM's scale product (clamp at zero, power, product over the scales)
    differentiated without the host read torch's prod backward makes: the
    same gradient as torch's autograd of the plain expression, including
    negative, zero and NaN terms, zero exponents and a zero factor under a
    fractional exponent (inf), and again under create_graph."""
    from frame_analytics_amd.functional import _CombineScales

    g = torch.Generator().manual_seed(5)
    base = torch.rand((5, 3, 4), generator=g, dtype=torch.float64) * 1.2 - 0.1
    base[0, 0, 0] = 0.0          # a zero factor, fractional exponent: inf
    base[1, 1, 1] = -0.3         # clamped: no gradient through it
    base[2, 2, 2] = float("nan")
    base[3, 0, 3] = 0.0
    for expo_v in ((0.0448, 0.2856, 0.3001, 0.2363, 0.1333), (0.5, 0.0, 1.0, 2.0, 0.25)):
        expo = torch.tensor(expo_v, dtype=torch.float64).view(-1, 1, 1)
        upstream = torch.rand((3, 4), generator=g, dtype=torch.float64)
        a = base.clone().requires_grad_(True)
        b = base.clone().requires_grad_(True)
        want_v = a.clamp_min(0.0).pow(expo).prod(dim=0)
        got_v = _CombineScales.apply(b, expo)
        assert torch.equal(torch.nan_to_num(got_v, nan=-7.0), torch.nan_to_num(want_v, nan=-7.0))
        (want,) = torch.autograd.grad(want_v, a, upstream)
        (got,) = torch.autograd.grad(got_v, b, upstream)
        assert torch.equal(torch.isnan(got), torch.isnan(want))
        assert torch.equal(torch.isinf(got), torch.isinf(want))
        fin = torch.isfinite(want)
        assert torch.allclose(got[fin], want[fin], rtol=1e-14, atol=0)
    # float32 terms: the gradient comes back float32, like the input
    a32 = base.abs().float().clamp_min(0.01).requires_grad_(True)
    expo = torch.tensor(MS_W, dtype=torch.float64).view(-1, 1, 1)
    (g32,) = torch.autograd.grad(_CombineScales.apply(a32, expo).sum(), a32)
    assert g32.dtype == torch.float32
    # second derivative, on strictly positive terms (finite everywhere)
    pos = (base.abs() + 0.05).nan_to_num(0.5)
    a = pos.clone().requires_grad_(True)
    b = pos.clone().requires_grad_(True)
    (ga,) = torch.autograd.grad(a.clamp_min(0.0).pow(expo).prod(dim=0).sum(), a, create_graph=True)
    (gb,) = torch.autograd.grad(_CombineScales.apply(b, expo).sum(), b, create_graph=True)
    (ha,) = torch.autograd.grad((ga * ga).sum(), a)
    (hb,) = torch.autograd.grad((gb * gb).sum(), b)
    assert torch.allclose(hb, ha, rtol=1e-12, atol=0)


MS_W = (0.0448, 0.2856, 0.3001, 0.2363, 0.1333)


def test_private_accumulator_scope_is_per_thread():
    """backend.private_accumulators (a graph's own accumulators) applies to
    the thread that opened it: another thread's calls meanwhile keep their
    streams' shared accumulators, and the scope ends with its block."""
    import threading

    from frame_analytics_amd import backend

    seen = {}
    mine: dict = {}
    with backend.private_accumulators(mine):
        assert getattr(backend._private, "store", None) is mine
        t = threading.Thread(target=lambda: seen.setdefault(
            "other", getattr(backend._private, "store", None)))
        t.start()
        t.join()
    assert seen["other"] is None
    assert getattr(backend._private, "store", None) is None
