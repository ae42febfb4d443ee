"""Stateful wrappers around :mod:`frame_analytics_amd.functional`.

Counterparts of the reference's ``frame_analytics/modules.py`` for the metrics
on this build's path: ``MSE``, ``PSNR``, ``SSIM``, ``MSSSIM``, ``GMSD``,
``L1``, ``Charbonnier``, ``Huber`` and ``StreamingMetrics``.  LPIPS and
SSIMULACRA 2 are not part of this build.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import torch
import torch.nn as nn

from .functional import (
    MS_SSIM_WEIGHTS,
    _infer_data_range,
    charbonnier,
    gms,
    gmsd,
    huber,
    l1,
    ms_ssim,
    mse,
    psnr,
    ssim,
)

__all__ = ["MSE", "PSNR", "SSIM", "MSSSIM", "GMSD", "L1", "Charbonnier", "Huber",
           "StreamingMetrics"]


class MSE(nn.Module):
    def __init__(self, reduction: str = "mean", dtype: Optional[torch.dtype] = None,
                 out_dtype: torch.dtype = torch.float64, luma=None, crop_border: int = 0):
        super().__init__()
        self.reduction = reduction
        self.dtype_ = dtype
        self.out_dtype = out_dtype
        self.luma = luma
        self.crop_border = crop_border

    def forward(self, x, y):
        return mse(x, y, reduction=self.reduction, dtype=self.dtype_,
                   out_dtype=self.out_dtype, luma=self.luma, crop_border=self.crop_border)


class PSNR(nn.Module):
    """``PSNR(luma="matlab", crop_border=scale)`` is the super-resolution Y-PSNR."""

    def __init__(self, data_range: Optional[float] = None, reduction: str = "mean",
                 dtype: Optional[torch.dtype] = None, out_dtype: torch.dtype = torch.float64,
                 eps: float = 0.0, luma=None, crop_border: int = 0):
        super().__init__()
        self.data_range = data_range
        self.reduction = reduction
        self.dtype_ = dtype
        self.out_dtype = out_dtype
        self.eps = eps
        self.luma = luma
        self.crop_border = crop_border

    def forward(self, x, y):
        return psnr(x, y, data_range=self.data_range, reduction=self.reduction,
                    dtype=self.dtype_, out_dtype=self.out_dtype, eps=self.eps,
                    luma=self.luma, crop_border=self.crop_border)


class SSIM(nn.Module):
    """SSIM; ``.loss()`` is ``1 - SSIM`` and differentiates through the fused
    gfx950 backward when the inputs are float32 on the GPU."""

    def __init__(self, data_range: Optional[float] = None, win_size: int = 11,
                 sigma: float = 1.5, K: Sequence[float] = (0.01, 0.03),
                 reduction: str = "mean", return_map: bool = False,
                 dtype: Optional[torch.dtype] = None, downsample: bool = False,
                 luma=None, crop_border: int = 0):
        super().__init__()
        self.data_range = data_range
        self.win_size = win_size
        self.sigma = sigma
        self.K = tuple(K)
        self.reduction = reduction
        self.return_map = return_map
        self.dtype_ = dtype
        self.downsample = downsample
        self.luma = luma
        self.crop_border = crop_border

    def forward(self, x, y):
        return ssim(x, y, data_range=self.data_range, win_size=self.win_size,
                    sigma=self.sigma, K=self.K, reduction=self.reduction,
                    return_map=self.return_map, dtype=self.dtype_,
                    downsample=self.downsample, luma=self.luma, crop_border=self.crop_border)

    def loss(self, x, y):
        return 1.0 - self.forward(x, y)


class MSSSIM(nn.Module):
    """Multi-scale SSIM; ``.loss()`` is ``1 - MS-SSIM``."""

    def __init__(self, data_range: Optional[float] = None, win_size: int = 11,
                 sigma: float = 1.5, K: Sequence[float] = (0.01, 0.03),
                 weights: Optional[Sequence[float]] = None, reduction: str = "mean",
                 dtype: Optional[torch.dtype] = None, luma=None, crop_border: int = 0):
        super().__init__()
        self.data_range = data_range
        self.win_size = win_size
        self.sigma = sigma
        self.K = tuple(K)
        self.weights = tuple(weights) if weights is not None else MS_SSIM_WEIGHTS
        self.reduction = reduction
        self.dtype_ = dtype
        self.luma = luma
        self.crop_border = crop_border

    def forward(self, x, y):
        return ms_ssim(x, y, data_range=self.data_range, win_size=self.win_size,
                       sigma=self.sigma, K=self.K, weights=self.weights,
                       reduction=self.reduction, dtype=self.dtype_, luma=self.luma,
                       crop_border=self.crop_border)

    def loss(self, x, y):
        return 1.0 - self.forward(x, y)


class GMSD(nn.Module):
    """GMSD; ``forward`` is the deviation, ``.loss()`` is ``1 - mean(GMS)``."""

    def __init__(self, data_range: Optional[float] = None, T: Optional[float] = None,
                 eps: Optional[float] = None, downsample: bool = True,
                 reduction: str = "mean", dtype: Optional[torch.dtype] = None, luma=None,
                 crop_border: int = 0):
        super().__init__()
        self.data_range = data_range
        self.T = T
        self.eps = eps
        self.downsample = downsample
        self.reduction = reduction
        self.dtype_ = dtype
        self.luma = luma
        self.crop_border = crop_border

    def _kwargs(self):
        return dict(data_range=self.data_range, T=self.T, eps=self.eps,
                    downsample=self.downsample, reduction=self.reduction, dtype=self.dtype_,
                    luma=self.luma, crop_border=self.crop_border)

    def forward(self, x, y):
        return gmsd(x, y, **self._kwargs())

    def loss(self, x, y):
        return 1.0 - gms(x, y, **self._kwargs())


class _PixelLoss(nn.Module):
    _fn = None

    def __init__(self, reduction: str = "mean", dtype: Optional[torch.dtype] = None,
                 out_dtype: torch.dtype = torch.float64, luma=None, crop_border: int = 0):
        super().__init__()
        self.reduction = reduction
        self.dtype_ = dtype
        self.out_dtype = out_dtype
        self.luma = luma
        self.crop_border = crop_border
        self.extra = {}

    def forward(self, x, y):
        return type(self)._fn(x, y, reduction=self.reduction, dtype=self.dtype_,
                              out_dtype=self.out_dtype, luma=self.luma,
                              crop_border=self.crop_border, **self.extra)

    def loss(self, x, y):
        return self.forward(x, y)


class L1(_PixelLoss):
    """Mean absolute error."""

    _fn = staticmethod(l1)


class Charbonnier(_PixelLoss):
    """Charbonnier penalty; ``eps`` is the width of the quadratic region."""

    _fn = staticmethod(charbonnier)

    def __init__(self, eps: float = 1e-3, **kwargs):
        super().__init__(**kwargs)
        self.extra = {"eps": float(eps)}


class Huber(_PixelLoss):
    """Huber loss, matching ``torch.nn.HuberLoss``."""

    _fn = staticmethod(huber)

    def __init__(self, delta: float = 1.0, **kwargs):
        super().__init__(**kwargs)
        self.extra = {"delta": float(delta)}


class StreamingMetrics:
    """Fixed-shape frame scorer: every requested metric captured into one HIP
    graph, replayed per frame pair (reference modules.py:316-455).

    The kernels behind the C ABI allocate nothing and never synchronise, and
    every buffer they need comes from torch's allocator, so a warm-up pass
    followed by capture is all it takes.
    """

    _KNOWN = ("mse", "psnr", "ssim", "ms_ssim", "gmsd", "gms", "l1", "charbonnier", "huber")

    def __init__(self, shape, device="cuda", dtype=torch.uint8,
                 data_range: Optional[float] = None, metrics=("mse", "psnr", "ssim"),
                 use_cuda_graph: bool = True, pinned_staging: bool = True):
        self.device = torch.device(device)
        self.dtype = dtype
        self.shape = tuple(shape)
        self.metrics = tuple(metrics)
        unknown = [m for m in self.metrics if m not in self._KNOWN]
        if unknown:
            raise ValueError(f"unknown metric(s) {unknown}; expected any of {list(self._KNOWN)}")
        self.ref = torch.empty(self.shape, dtype=dtype, device=self.device)
        self.dist = torch.empty(self.shape, dtype=dtype, device=self.device)
        self._L = float(data_range) if data_range is not None else _infer_data_range(self.ref)
        self._host = None
        if pinned_staging and self.device.type == "cuda":
            self._host = (torch.empty(self.shape, dtype=dtype, pin_memory=True),
                          torch.empty(self.shape, dtype=dtype, pin_memory=True))
        self._graph = None
        self._static_out = None
        if use_cuda_graph and self.device.type == "cuda":
            self._try_capture()

    def _compute(self):
        out = {}
        if "mse" in self.metrics or "psnr" in self.metrics:
            m = mse(self.ref, self.dist)
            if "mse" in self.metrics:
                out["mse"] = m
            if "psnr" in self.metrics:
                out["psnr"] = math.log10(self._L ** 2) * 10.0 - 10.0 * torch.log10(m)
        if "ssim" in self.metrics:
            out["ssim"] = ssim(self.ref, self.dist, data_range=self._L)
        if "ms_ssim" in self.metrics:
            out["ms_ssim"] = ms_ssim(self.ref, self.dist, data_range=self._L)
        if "gmsd" in self.metrics:
            out["gmsd"] = gmsd(self.ref, self.dist, data_range=self._L)
        if "gms" in self.metrics:
            out["gms"] = gms(self.ref, self.dist, data_range=self._L)
        for name, fn in (("l1", l1), ("charbonnier", charbonnier), ("huber", huber)):
            if name in self.metrics:
                out[name] = fn(self.ref, self.dist)
        return out

    def _try_capture(self):
        try:
            self.ref.zero_()
            self.dist.zero_()
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(3):  # warm the allocator and the workspace caches
                    self._compute()
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._static_out = self._compute()
            self._graph = g
        except Exception:
            self._graph = None
            self._static_out = None

    def _stage(self, buf: torch.Tensor, src, slot: int) -> None:
        if not torch.is_tensor(src):
            src = torch.from_numpy(src)
        if src.shape != self.shape:
            src = src.reshape(self.shape)
        if src.is_cuda:
            buf.copy_(src, non_blocking=True)
        elif self._host is not None:
            self._host[slot].copy_(src)
            buf.copy_(self._host[slot], non_blocking=True)
        else:
            buf.copy_(src)

    def update(self, ref, dist, *, as_float: bool = True):
        """Score one frame pair; returns ``{metric: value}``."""
        self._stage(self.ref, ref, 0)
        self._stage(self.dist, dist, 1)
        if self._graph is not None:
            self._graph.replay()
            out = self._static_out
        else:
            out = self._compute()
        if as_float:
            return {k: float(v) for k, v in out.items()}
        return {k: v.clone() for k, v in out.items()}

    @property
    def graph_captured(self) -> bool:
        return self._graph is not None
