"""StreamingMetrics: every metric captured into one HIP graph and replayed.

The kernels behind the C ABI allocate nothing and never synchronise, so the
whole scorer captures.  Replays are checked one by one against eager calls,
with eager work and synchronisations between them.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import frame_analytics_amd as fa
from oracle import reference as ref
from tests.conftest import u8_pair

pytestmark = pytest.mark.gpu


def test_streaming_matches_functional(gpu):
    a = torch.randint(0, 256, (1, 3, 240, 320), dtype=torch.uint8)
    b = (a.float() + 9).clamp(0, 255).to(torch.uint8)
    sm = fa.StreamingMetrics((1, 3, 240, 320), device="cuda", dtype=torch.uint8,
                             data_range=255.0)
    assert sm.graph_captured
    out = sm.update(a, b)
    ac, bc = a.cuda(), b.cuda()
    assert abs(out["ssim"] - float(fa.ssim(ac, bc, data_range=255.0))) < 1e-12
    assert abs(out["psnr"] - float(fa.psnr(ac, bc, data_range=255.0))) < 1e-12
    assert abs(out["mse"] - float(fa.mse(ac, bc))) < 1e-12


def test_streaming_replays_every_metric(gpu):
    metrics = ("mse", "psnr", "ssim", "ms_ssim", "gmsd", "gms", "l1", "charbonnier", "huber")
    shape = (2, 3, 192, 208)
    sm = fa.StreamingMetrics(shape, device="cuda", dtype=torch.uint8, data_range=255.0,
                             metrics=metrics)
    assert sm.graph_captured
    for seed in range(4):
        a, b = u8_pair(shape, 6.0 + 4 * seed, seed=100 + seed)
        got = sm.update(a, b)
        # eager work and a sync between replays
        ta, tb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
        want = {
            "mse": float(fa.mse(ta, tb)), "psnr": float(fa.psnr(ta, tb, data_range=255.0)),
            "ssim": float(fa.ssim(ta, tb, data_range=255.0)),
            "ms_ssim": float(fa.ms_ssim(ta, tb, data_range=255.0)),
            "gmsd": float(fa.gmsd(ta, tb, data_range=255.0)),
            "gms": float(fa.gms(ta, tb, data_range=255.0)),
            "l1": float(fa.l1(ta, tb)), "charbonnier": float(fa.charbonnier(ta, tb)),
            "huber": float(fa.huber(ta, tb)),
        }
        torch.cuda.synchronize()
        for k in metrics:
            assert abs(got[k] - want[k]) <= 1e-12 * max(1.0, abs(want[k])), (seed, k, got[k], want[k])
        assert got["mse"] == ref.mse(a, b)
        assert abs(got["ssim"] - ref.ssim(a, b, 255.0)) <= 1e-6 * got["ssim"]


def test_streaming_from_device_tensors(gpu):
    shape = (1, 1, 128, 160)
    sm = fa.StreamingMetrics(shape, device="cuda", dtype=torch.uint8, data_range=255.0)
    a, b = u8_pair(shape, 10.0, seed=3)
    ta, tb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    out = sm.update(ta, tb, as_float=False)
    assert isinstance(out["ssim"], torch.Tensor)
    assert float(out["mse"]) == ref.mse(a, b)


def test_streaming_graph_finishes_in_its_launches(gpu):
    """At 1080p RGB every captured metric takes its one-launch form (the pixel
    sweep's, the matrix-core SSIM's, GMSD's, MS-SSIM's three launches) on the
    graph's own accumulators: replays match eager calls made between them (on
    the stream's shared accumulators) to 1e-12, and every private accumulator
    is zero after each replay."""
    from frame_analytics_amd import backend

    metrics = ("mse", "psnr", "ssim", "ms_ssim", "gmsd")
    shape = (1, 3, 1080, 1920)
    sm = fa.StreamingMetrics(shape, device="cuda", dtype=torch.uint8, data_range=255.0,
                             metrics=metrics)
    assert sm.graph_captured
    assert {k[0] for k in sm._accs} == {"pixel", "ssim", "gmsd", "ms"}
    for seed in range(3):
        a, b = u8_pair(shape, 5.0 + 3 * seed, seed=200 + seed)
        got = sm.update(a, b)
        torch.cuda.synchronize()
        assert not any(bool(t.any()) for t in sm._accs.values()), seed
        ta, tb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
        want = {"mse": float(fa.mse(ta, tb)), "psnr": float(fa.psnr(ta, tb, data_range=255.0)),
                "ssim": float(fa.ssim(ta, tb, data_range=255.0)),
                "ms_ssim": float(fa.ms_ssim(ta, tb, data_range=255.0)),
                "gmsd": float(fa.gmsd(ta, tb, data_range=255.0))}
        for k in metrics:
            assert abs(got[k] - want[k]) <= 1e-12 * max(1.0, abs(want[k])), (seed, k, got[k], want[k])
        assert got["mse"] == ref.mse(a, b)
    shared = list(backend._stream_acc.values())
    assert not any(t is u for t in sm._accs.values() for u in shared)
