"""Stateful wrappers around :mod:`frame_analytics_amd.functional`.

Counterparts of the reference's ``frame_analytics/modules.py`` for the metrics
on this build's path: ``MSE``, ``PSNR``, ``SSIM``, ``MSSSIM``, ``GMSD``,
``L1``, ``Charbonnier``, ``Huber`` and ``StreamingMetrics``.  The constructor
signatures and the attribute names are the reference's (``modules.py:45-455``);
LPIPS and SSIMULACRA 2 are not part of this build.

Every metric module is a :class:`_Scorer`: it holds the functional keyword
arguments of one metric in a dict and forwards them on each call, so a module
and the function it wraps cannot drift apart.
"""

from __future__ import annotations

import math
from typing import Callable, Dict, Optional, Sequence

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

# attribute names the reference's modules expose -> functional keyword
_ATTR_TO_KW = {"dtype_": "dtype"}


class _Scorer(nn.Module):
    """One metric with fixed keyword arguments.

    ``self.kwargs`` is what every call passes to the functional form; the
    reference's attribute names (``module.reduction``, ``module.dtype_``, ...)
    read and write the same dict.
    """

    _metric: Callable = None  # the functional form, set by each subclass

    def __init__(self, **kwargs):
        super().__init__()
        self.__dict__["kwargs"] = dict(kwargs)

    def __getattr__(self, name):
        kw = self.__dict__.get("kwargs", {})
        key = _ATTR_TO_KW.get(name, name)
        if key in kw:
            return kw[key]
        return super().__getattr__(name)

    def __setattr__(self, name, value):
        kw = self.__dict__.get("kwargs")
        key = _ATTR_TO_KW.get(name, name)
        if kw is not None and key in kw:
            kw[key] = value
        else:
            super().__setattr__(name, value)

    def forward(self, x, y):
        return type(self)._metric(x, y, **self.kwargs)

    def extra_repr(self) -> str:
        return ", ".join(f"{k}={v!r}" for k, v in self.kwargs.items())


class _SimilarityLoss(_Scorer):
    """A similarity in [0, 1] whose loss is ``1 - value``."""

    def loss(self, x, y):
        return 1.0 - self.forward(x, y)


class MSE(_Scorer):
    """Mean squared error (exact integer sums for uint8 on the GPU)."""

    _metric = staticmethod(mse)

    def __init__(self, reduction: str = "mean", dtype: Optional[torch.dtype] = None,
                 out_dtype: torch.dtype = torch.float64, luma=None, crop_border: int = 0):
        super().__init__(reduction=reduction, dtype=dtype, out_dtype=out_dtype, luma=luma,
                         crop_border=crop_border)


class PSNR(_Scorer):
    """Peak signal-to-noise ratio; ``PSNR(luma="matlab", crop_border=scale)``
    is the Y-PSNR the super-resolution literature reports."""

    _metric = staticmethod(psnr)

    def __init__(self, data_range: Optional[float] = None, reduction: str = "mean",
                 dtype: Optional[torch.dtype] = None, out_dtype: torch.dtype = torch.float64,
                 eps: float = 0.0, luma=None, crop_border: int = 0):
        super().__init__(data_range=data_range, reduction=reduction, dtype=dtype,
                         out_dtype=out_dtype, eps=eps, luma=luma, crop_border=crop_border)


class SSIM(_SimilarityLoss):
    """SSIM; ``.loss()`` is ``1 - SSIM`` and differentiates through the fused
    gfx950 backward when the inputs are float32 on the GPU."""

    _metric = staticmethod(ssim)

    def __init__(self, data_range: Optional[float] = None, win_size: int = 11,
                 sigma: float = 1.5, K: Sequence[float] = (0.01, 0.03),
                 reduction: str = "mean", return_map: bool = False,
                 dtype: Optional[torch.dtype] = None, downsample: bool = False,
                 luma=None, crop_border: int = 0):
        super().__init__(data_range=data_range, win_size=win_size, sigma=sigma, K=tuple(K),
                         reduction=reduction, return_map=return_map, dtype=dtype,
                         downsample=downsample, luma=luma, crop_border=crop_border)


class MSSSIM(_SimilarityLoss):
    """Multi-scale SSIM; ``.loss()`` is ``1 - MS-SSIM`` (fused pyramid
    backward on the GPU)."""

    _metric = staticmethod(ms_ssim)

    def __init__(self, data_range: Optional[float] = None, win_size: int = 11,
                 sigma: float = 1.5, K: Sequence[float] = (0.01, 0.03),
                 weights: Optional[Sequence[float]] = None, reduction: str = "mean",
                 dtype: Optional[torch.dtype] = None, luma=None, crop_border: int = 0):
        super().__init__(data_range=data_range, win_size=win_size, sigma=sigma, K=tuple(K),
                         weights=MS_SSIM_WEIGHTS if weights is None else tuple(weights),
                         reduction=reduction, dtype=dtype, luma=luma, crop_border=crop_border)


class GMSD(_Scorer):
    """GMSD (lower is better); ``.loss()`` is ``1 - mean(GMS)``, whose
    gradient the gfx950 backward computes in float64."""

    _metric = staticmethod(gmsd)

    def __init__(self, data_range: Optional[float] = None, T: Optional[float] = None,
                 eps: Optional[float] = None, downsample: bool = True,
                 reduction: str = "mean", dtype: Optional[torch.dtype] = None, luma=None,
                 crop_border: int = 0):
        super().__init__(data_range=data_range, T=T, eps=eps, downsample=downsample,
                         reduction=reduction, dtype=dtype, luma=luma, crop_border=crop_border)

    def loss(self, x, y):
        return 1.0 - gms(x, y, **self.kwargs)


class _PixelScorer(_Scorer):
    """A per-pixel penalty; the loss is the value itself."""

    def __init__(self, reduction="mean", dtype=None, out_dtype=torch.float64, luma=None,
                 crop_border=0, **param):
        super().__init__(reduction=reduction, dtype=dtype, out_dtype=out_dtype, luma=luma,
                         crop_border=crop_border, **param)

    def loss(self, x, y):
        return self.forward(x, y)


class L1(_PixelScorer):
    """Mean absolute error, in the input's own units."""

    _metric = staticmethod(l1)

    def __init__(self, reduction: str = "mean", dtype: Optional[torch.dtype] = None,
                 out_dtype: torch.dtype = torch.float64, luma=None, crop_border: int = 0):
        super().__init__(reduction, dtype, out_dtype, luma, crop_border)


class Charbonnier(_PixelScorer):
    """``mean sqrt(d^2 + eps^2)``: L1 with a quadratic core of width ``eps``."""

    _metric = staticmethod(charbonnier)

    def __init__(self, eps: float = 1e-3, reduction: str = "mean",
                 dtype: Optional[torch.dtype] = None, out_dtype: torch.dtype = torch.float64,
                 luma=None, crop_border: int = 0):
        super().__init__(reduction, dtype, out_dtype, luma, crop_border, eps=float(eps))


class Huber(_PixelScorer):
    """Huber loss, term for term ``torch.nn.HuberLoss``."""

    _metric = staticmethod(huber)

    def __init__(self, delta: float = 1.0, reduction: str = "mean",
                 dtype: Optional[torch.dtype] = None, out_dtype: torch.dtype = torch.float64,
                 luma=None, crop_border: int = 0):
        super().__init__(reduction, dtype, out_dtype, luma, crop_border, delta=float(delta))


# --------------------------------------------------------------------------- #
# StreamingMetrics
# --------------------------------------------------------------------------- #


def _metric_table(L: float) -> Dict[str, Callable]:
    """name -> f(ref, dist, results so far) for every metric StreamingMetrics
    knows.  PSNR reuses the MSE already computed when both are asked for (a
    host constant minus one device op: no H2D copy, so it captures)."""
    bias = 10.0 * math.log10(L * L)

    def _psnr(a, b, done):
        if "mse" in done:
            return bias - 10.0 * torch.log10(done["mse"])
        return psnr(a, b, data_range=L)

    return {
        "mse": lambda a, b, done: mse(a, b),
        "psnr": _psnr,
        "ssim": lambda a, b, done: ssim(a, b, data_range=L),
        "ms_ssim": lambda a, b, done: ms_ssim(a, b, data_range=L),
        "gmsd": lambda a, b, done: gmsd(a, b, data_range=L),
        "gms": lambda a, b, done: gms(a, b, data_range=L),
        "l1": lambda a, b, done: l1(a, b),
        "charbonnier": lambda a, b, done: charbonnier(a, b),
        "huber": lambda a, b, done: huber(a, b),
    }


_ORDER = ("mse", "psnr", "ssim", "ms_ssim", "gmsd", "gms", "l1", "charbonnier", "huber")


class StreamingMetrics:
    """Scores a stream of fixed-shape frame pairs with one graph replay each.

    Same constructor and ``update`` as the reference's (``modules.py:316-455``).
    The design here:

    * The frame pair lives in two device buffers.  Every requested metric is
      captured, in one HIP graph, as a function of those buffers; the metrics
      are also gathered into one float64 vector inside the graph, so
      ``update(..., as_float=True)`` costs one device-to-host copy and one
      synchronisation whatever the number of metrics.
    * Host frames are staged through two pairs of pinned buffers used in turn.
      A pinned buffer is written only after the copy that last read it has
      finished (an event recorded behind each copy), so a frame never
      overwrites one that is still in flight, with ``as_float=False`` too.
    * The kernels behind the C ABI allocate nothing and never synchronise, so
      one eager warm-up pass (which fills the allocator pool and the workspace
      caches) and a capture are all it takes.  If capture fails the scorer
      runs eagerly; ``capture_error`` says why.
    """

    _KNOWN = _ORDER

    def __init__(self, shape, device="cuda", dtype=torch.uint8,
                 data_range: Optional[float] = None, metrics=("mse", "psnr", "ssim"),
                 use_cuda_graph: bool = True, pinned_staging: bool = True):
        names = tuple(metrics)
        unknown = [m for m in names if m not in _ORDER]
        if unknown:
            raise ValueError(f"unknown metric(s) {unknown}; expected any of {list(_ORDER)}")
        self.device = torch.device(device)
        self.dtype = dtype
        self.shape = tuple(shape)
        self.metrics = names
        self.data_range = data_range
        self.ref = torch.empty(self.shape, dtype=dtype, device=self.device)
        self.dist = torch.empty(self.shape, dtype=dtype, device=self.device)
        self._L = float(data_range) if data_range is not None else _infer_data_range(self.ref)
        table = _metric_table(self._L)
        # evaluation order: mse before psnr, whatever order the caller listed
        self._plan = [(m, table[m]) for m in _ORDER if m in names]
        on_gpu = self.device.type == "cuda"
        self._slots = None
        if pinned_staging and on_gpu:
            self._slots = [[torch.empty(self.shape, dtype=dtype, pin_memory=True)
                            for _ in range(2)] for _ in range(2)]
            self._slot_done = [[None, None], [None, None]]
        self._turn = 0
        self._graph = None
        self._outs = None
        self.capture_error: Optional[str] = None
        if use_cuda_graph and on_gpu:
            self._capture()

    # -- evaluation ---------------------------------------------------------- #

    def _evaluate(self):
        done: Dict[str, torch.Tensor] = {}
        for name, fn in self._plan:
            done[name] = fn(self.ref, self.dist, done)
        values = torch.stack([done[n].to(torch.float64).reshape(()) for n in self.metrics])
        return done, values

    def _capture(self) -> None:
        from . import backend

        side = torch.cuda.Stream(self.device)
        # the graph's own accumulators: only its replays use them, so the
        # captured metrics finish in their one launch (made in the warm-up)
        self._accs: dict = {}
        try:
            with torch.cuda.device(self.device), backend.private_accumulators(self._accs):
                self.ref.zero_()
                self.dist.zero_()
                side.wait_stream(torch.cuda.current_stream(self.device))
                with torch.cuda.stream(side):
                    self._evaluate()  # pool, workspace, window caches, accumulators
                side.synchronize()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=side):
                    outs = self._evaluate()
                torch.cuda.current_stream(self.device).wait_stream(side)
            self._graph, self._outs = graph, outs
        except Exception as exc:  # an eager scorer still works
            self._graph = self._outs = None
            self._accs = {}
            self.capture_error = f"{type(exc).__name__}: {exc}"

    # -- staging ------------------------------------------------------------- #

    def _put(self, which: int, src) -> None:
        dst = self.ref if which == 0 else self.dist
        t = src if torch.is_tensor(src) else torch.from_numpy(src)
        if tuple(t.shape) != self.shape:
            t = t.reshape(self.shape)
        if t.device.type != "cpu" or self._slots is None:
            dst.copy_(t, non_blocking=t.device.type != "cpu")
            return
        slot = self._turn
        pending = self._slot_done[which][slot]
        if pending is not None:
            pending.synchronize()  # the copy that last read this buffer is over
        host = self._slots[which][slot]
        host.copy_(t)
        dst.copy_(host, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        self._slot_done[which][slot] = ev

    # -- API ----------------------------------------------------------------- #

    def update(self, ref, dist, *, as_float: bool = True):
        """Score one frame pair (numpy arrays, CPU or device tensors of the
        configured shape).  Returns ``{metric: float}``, or ``{metric: 0-d
        tensor}`` on the device with ``as_float=False``."""
        self._put(0, ref)
        self._put(1, dist)
        self._turn ^= 1
        if self._graph is not None:
            self._graph.replay()
            done, values = self._outs
        else:
            done, values = self._evaluate()
        if as_float:
            return dict(zip(self.metrics, values.tolist()))
        return {n: done[n].clone() for n in self.metrics}

    @property
    def graph_captured(self) -> bool:
        return self._graph is not None
