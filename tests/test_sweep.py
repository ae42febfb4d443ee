"""Seeded sweep of the public API against the float64 oracle, on the GPU
(the kernels) and on the CPU (the host library and the portable path).

Each case draws a function, element type, shape (odd sizes included), batch,
channels, luma convention, border crop, reduction and the function's own
options from a fixed seed, so a failure names a reproducible configuration.
Bars: uint8 MSE / L1 without luma bit-exact; other pixel losses 1e-9
relative (Charbonnier below float64 input and uint8 Huber 1e-6: float32
terms, as in the reference's kernels, fa_cuda.cu:252-359); PSNR 1e-9 dB;
SSIM / MS-SSIM 1e-6 (float64 input 1e-9); GMSD / GMS 1e-6 relative on
1 - q and on the standard deviation.  Float16 / bfloat16 inputs are compared
with the oracle on their rounded values.  On the CPU a luma plane is formed
in the working type first (float32 below float64 input, as the reference's
portable path does), so pixel losses and PSNR with luma are held to 1e-6
there, and GMSD / GMS to 1e-5.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import frame_analytics_amd as fa
from oracle import reference as ref

FUNCS = ("mse", "psnr", "l1", "charbonnier", "huber", "ssim", "ms_ssim", "gmsd", "gms")
DTYPES = (torch.uint8, torch.float16, torch.bfloat16, torch.float32, torch.float64)
LUMAS = (None, "bt601", "bt709", "matlab")


def _case(i):
    rng = np.random.default_rng(1000 + i)
    fn = FUNCS[i % len(FUNCS)]
    dt = DTYPES[rng.integers(len(DTYPES))]
    n = int(rng.integers(1, 4))
    c = int(rng.choice([1, 3]))
    lo = 182 if fn == "ms_ssim" else 24
    h, w = (int(v) for v in rng.integers(lo, lo + 60, 2))
    luma = LUMAS[rng.integers(len(LUMAS))] if c == 3 else None
    crop = int(rng.choice([0, 0, 1, 3]))
    red = str(rng.choice(["mean", "none"]))
    sigma = float(rng.uniform(2.0, 25.0))
    opts = {}
    if fn in ("ssim",):
        opts["win_size"] = int(rng.choice([3, 5, 7, 9, 11]))
    if fn in ("gmsd", "gms"):
        opts["downsample"] = bool(rng.integers(2))
    if fn == "charbonnier":
        opts["eps"] = float(rng.choice([1e-3, 0.5]))
    if fn == "huber":
        opts["delta"] = float(rng.choice([0.02, 1.0]))
    return dict(fn=fn, dt=dt, shape=(n, c, h, w), luma=luma, crop=crop, red=red,
                sigma=sigma, opts=opts, seed=1000 + i)


def _inputs(cfg):
    rng = np.random.default_rng(cfg["seed"])
    shape = cfg["shape"]
    a = rng.integers(0, 256, shape).astype(np.float64)
    b = np.clip(a + np.round(rng.normal(0, cfg["sigma"], shape)), 0, 255)
    dt = cfg["dt"]
    if dt == torch.uint8:
        return a.astype(np.uint8), b.astype(np.uint8), 255.0
    return a / 255.0, b / 255.0, 1.0


def _oracle(cfg, xa, ya, L):
    fn, red, o = cfg["fn"], cfg["red"], cfg["opts"]
    if cfg["luma"] is not None:
        xa, ya = ref.rgb_to_luma(xa, cfg["luma"], L), ref.rgb_to_luma(ya, cfg["luma"], L)
    xa, ya = ref.crop(xa, cfg["crop"]), ref.crop(ya, cfg["crop"])
    if fn == "mse":
        return ref.mse(xa, ya, reduction=red)
    if fn == "psnr":
        return ref.psnr(xa, ya, L, reduction=red)
    if fn == "l1":
        return ref.l1(xa, ya, reduction=red)
    if fn == "charbonnier":
        return ref.charbonnier(xa, ya, o["eps"], reduction=red)
    if fn == "huber":
        return ref.huber(xa, ya, o["delta"], reduction=red)
    if fn == "ssim":
        return ref.ssim(xa, ya, L, win_size=o["win_size"], reduction=red)
    if fn == "ms_ssim":
        return ref.ms_ssim(xa, ya, L, reduction=red)
    m, sd = ref.gmsd_stats_hp(xa, ya, L, downsample=o["downsample"])
    v = sd if fn == "gmsd" else m
    return v if red == "none" else float(v.mean())


def _call(cfg, x, y, L):
    fn, o = cfg["fn"], cfg["opts"]
    kw = dict(reduction=cfg["red"], luma=cfg["luma"], crop_border=cfg["crop"])
    if fn in ("psnr", "ssim", "ms_ssim", "gmsd", "gms"):
        kw["data_range"] = L
    if fn == "ssim":
        kw["win_size"] = o["win_size"]
    if fn in ("gmsd", "gms"):
        kw["downsample"] = o["downsample"]
    if fn == "charbonnier":
        kw["eps"] = o["eps"]
    if fn == "huber":
        kw["delta"] = o["delta"]
    return getattr(fa, fn)(x, y, **kw)


@pytest.mark.parametrize("i", range(144))
@pytest.mark.parametrize("where", ["cpu", pytest.param("cuda", marks=pytest.mark.gpu)])
def test_sweep_case(where, i, request):
    dev = request.getfixturevalue("gpu") if where == "cuda" else torch.device("cpu")
    cfg = _case(i)
    a, b, L = _inputs(cfg)
    dt = cfg["dt"]
    x = torch.as_tensor(a).to(dt).to(dev)
    y = torch.as_tensor(b).to(dt).to(dev)
    xa, ya = x.double().cpu().numpy(), y.double().cpu().numpy()
    if dt == torch.uint8:
        xa, ya = x.cpu().numpy(), y.cpu().numpy()
    want = np.atleast_1d(np.asarray(_oracle(cfg, xa, ya, L), dtype=np.float64))
    got = np.atleast_1d(_call(cfg, x, y, L).double().cpu().numpy())
    assert got.shape == want.shape, cfg
    fn = cfg["fn"]
    host_luma = where == "cpu" and cfg["luma"] is not None and dt != torch.float64
    if fn in ("mse", "l1") and dt == torch.uint8 and cfg["luma"] is None:
        assert np.array_equal(got, want), (cfg, got, want)
        return
    if fn == "psnr":
        assert np.abs(got - want).max() <= (1e-6 if host_luma else 1e-9), (cfg, got, want)
        return
    if fn in ("gmsd", "gms"):
        # relative on the spread (gmsd) and on 1 - q (gms)
        scale = np.abs(want) if fn == "gmsd" else np.abs(1.0 - want)
        tol = 1e-5 if host_luma else 1e-6  # a float32 luma plane shifts the gradients
        assert np.all(np.abs(got - want) <= tol * scale + 1e-15), (cfg, got, want)
        return
    if fn in ("ssim", "ms_ssim"):
        tol = 1e-9 if dt == torch.float64 else 1e-6
        assert np.abs(got - want).max() <= tol, (cfg, got, want)
        return
    f32_terms = (fn == "charbonnier" and dt != torch.float64) or (
        fn == "huber" and dt == torch.uint8 and where == "cuda" and cfg["luma"] is None)
    tol = 1e-6 if f32_terms or host_luma else 1e-9
    assert np.all(np.abs(got - want) <= tol * np.abs(want)), (cfg, got, want)
