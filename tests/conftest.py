"""Shared test setup: import path, the `gpu` marker, seeded input generators."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")
    config.addinivalue_line(
        "markers", "portable_ok: a gpu test that runs the portable PyTorch path on GPU "
        "tensors on purpose (exempt from the native-dispatch check)")


@pytest.hookimpl(hookwrapper=True)
def pytest_runtest_makereport(item, call):
    outcome = yield
    rep = outcome.get_result()
    setattr(item, "rep_" + rep.when, rep)


@pytest.fixture(autouse=True)
def _served_by_gfx950_kernels(request):
    """A passing ``gpu`` test must have been served by the HIP kernels: at
    least one entry point of libfa_gpu.so ran during it (counted by
    ``backend.call_gpu``), and the portable PyTorch path computed nothing on a
    GPU tensor (``backend.portable_calls``).  So a ``try_*`` that quietly
    returned None -- which would let eager PyTorch meet the same numerical
    bars -- fails the suite."""
    if request.node.get_closest_marker("gpu") is None:
        yield
        return
    from frame_analytics_amd import backend

    ran0 = sum(backend.native_calls.values())
    portable0 = dict(backend.portable_calls)
    yield
    rep = getattr(request.node, "rep_call", None)
    if rep is None or not rep.passed or request.node.get_closest_marker("portable_ok"):
        return
    ran = sum(backend.native_calls.values()) - ran0
    portable = {k: v - portable0.get(k, 0) for k, v in backend.portable_calls.items()
                if v != portable0.get(k, 0)}
    assert ran > 0, "no gfx950 entry point ran in this GPU test"
    assert not portable, f"the portable PyTorch path ran on GPU tensors: {portable}"


def u8_pair(shape, sigma, seed):
    """BASELINE.json generator: a ~ U{0..255}; b = clip(a + round(N(0, sigma)), 0, 255)."""
    rng = np.random.default_rng(seed)
    a = rng.integers(0, 256, shape, dtype=np.uint8)
    noise = np.round(rng.normal(0.0, sigma, shape)).astype(np.int32)
    b = np.clip(a.astype(np.int32) + noise, 0, 255).astype(np.uint8)
    return a, b


def natural_pair(h, w, noise=8.0, seed=0, kind="natural"):
    """A photograph-like plane pair (smooth base + texture), rounded to integers,
    in the style of the reference's validate.make_pair (validate.py:44-64)."""
    rng = np.random.default_rng(seed)
    if kind == "natural":
        yy, xx = np.mgrid[0:h, 0:w].astype(np.float64)
        base = (110 + 60 * np.sin(xx / 37.0) * np.cos(yy / 53.0)
                + 40 * np.sin((xx + yy) / 17.0) + 25 * rng.standard_normal((h, w)))
        base = np.clip(base, 0, 255)
    elif kind == "uniform":
        base = rng.integers(0, 256, (h, w)).astype(np.float64)
    elif kind == "flat":
        base = np.full((h, w), 128.0)
    else:
        raise ValueError(kind)
    dist = np.clip(base + noise * rng.standard_normal((h, w)), 0, 255)
    return base.round(), dist.round()


def float_pair(shape, sigma=0.05, seed=0):
    """configs[3] generator: x ~ U[0,1), y = clip(x + N(0, sigma), 0, 1), float32."""
    rng = np.random.default_rng(seed)
    x = rng.random(shape, dtype=np.float32)
    y = np.clip(x + rng.normal(0.0, sigma, shape), 0, 1).astype(np.float32)
    return x, y


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")
    from frame_analytics_amd import backend

    ext = backend.load()
    assert ext is not None and ext.has_gpu, "gfx950 kernel library did not load"
    return torch.device("cuda:0")
