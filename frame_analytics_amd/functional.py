"""MSE / PSNR / SSIM / MS-SSIM / GMSD / pixel losses -- the public functions.

Same names, signatures, defaults and error behaviour as the reference's
``frame_analytics/functional.py``; ``import frame_analytics_amd as fa`` is a
drop-in for ``import frame_analytics as fa`` on these entry points.

Routing for a GPU tensor: the gfx950 kernels behind ``include/fa_abi.h``
(through :mod:`frame_analytics_amd.backend`).  The portable PyTorch path below
runs only where the reference runs it too -- CPU tensors,
``backend_hint="torch"``, a window width without a kernel, the GMS map, a
float64 working dtype for GMSD, and pixel losses that need a gradient -- and
it is plain eager PyTorch: no ``torch.compile`` (on ROCm that would emit
Triton).  ``backend_hint="native"`` raises instead of taking it.
"""

from __future__ import annotations

import functools
import math
from typing import Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

__all__ = [
    "mse",
    "psnr",
    "ssim",
    "ms_ssim",
    "gmsd",
    "gms",
    "l1",
    "charbonnier",
    "huber",
    "rgb_to_luma",
    "gaussian_window_1d",
    "set_compile_enabled",
    "MS_SSIM_WEIGHTS",
]

def set_compile_enabled(flag: bool) -> None:
    """Kept for API compatibility (reference functional.py:55-59).

    This build never compiles the portable path -- on ROCm ``torch.compile``
    lowers to Triton -- so the flag changes nothing.
    """
    del flag


# --------------------------------------------------------------------------- #
# input handling (reference functional.py:141-271)
# --------------------------------------------------------------------------- #


def _infer_data_range(t: torch.Tensor) -> float:
    if t.dtype == torch.uint8:
        return 255.0
    if t.dtype in (torch.int16, torch.int32) or t.dtype == getattr(torch, "uint16", None):
        return 65535.0
    return 1.0


def _as_nchw(t: torch.Tensor) -> torch.Tensor:
    """(H,W), (C,H,W) or (N,C,H,W) -> 4-D view."""
    if t.ndim == 4:
        return t
    if t.ndim == 3:
        return t.unsqueeze(0)
    if t.ndim == 2:
        return t.unsqueeze(0).unsqueeze(0)
    raise ValueError(f"expected 2/3/4-D tensor, got shape {tuple(t.shape)}")


def _check_pair(x: torch.Tensor, y: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    if x.shape != y.shape:
        raise ValueError(f"shape mismatch: {tuple(x.shape)} vs {tuple(y.shape)}")
    if x.device != y.device:
        raise ValueError(f"device mismatch: {x.device} vs {y.device}")
    return _as_nchw(x), _as_nchw(y)


def _work_dtype(x: torch.Tensor, dtype: Optional[torch.dtype]) -> torch.dtype:
    if dtype is not None:
        return dtype
    return torch.float64 if x.dtype == torch.float64 else torch.float32


# (r, g, b, offset as a fraction of the data range)
LUMA_COEFFS = {
    "bt601": (0.299, 0.587, 0.114, 0.0),
    "bt709": (0.2126, 0.7152, 0.0722, 0.0),
    "matlab": (65.481 / 255.0, 128.553 / 255.0, 24.966 / 255.0, 16.0 / 255.0),
}


def _resolve_luma(luma) -> Optional[str]:
    if luma is None or luma is False:
        return None
    if luma is True:
        return "bt601"
    if isinstance(luma, str):
        if luma not in LUMA_COEFFS:
            raise ValueError(f"unknown luma mode {luma!r}; expected one of {sorted(LUMA_COEFFS)}")
        return luma
    raise TypeError(f"luma must be None, a bool or a string, got {type(luma).__name__}")


def rgb_to_luma(t: torch.Tensor, mode: str = "bt601", *,
                data_range: Optional[float] = None,
                dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """``(N,3,H,W)`` RGB -> ``(N,1,H,W)`` luma in the input's own units."""
    t4 = _as_nchw(t)
    if t4.shape[1] != 3:
        raise ValueError(f"luma needs a 3-channel image, got {t4.shape[1]} channels")
    m = _resolve_luma(mode)
    if m is None:
        raise ValueError("rgb_to_luma needs a luma convention, not None/False")
    kr, kg, kb, off = LUMA_COEFFS[m]
    L = float(data_range) if data_range is not None else _infer_data_range(t4)
    v = t4.to(_work_dtype(t4, dtype))
    out = kr * v[:, 0:1] + kg * v[:, 1:2] + kb * v[:, 2:3]
    return out + off * L if off else out


def _crop_border(t: torch.Tensor, b: int) -> torch.Tensor:
    if not b:
        return t
    if b < 0:
        raise ValueError(f"crop_border must be >= 0, got {b}")
    h, w = t.shape[-2], t.shape[-1]
    if h <= 2 * b or w <= 2 * b:
        raise ValueError(f"crop_border={b} removes the whole {h}x{w} image")
    return t[..., b:h - b, b:w - b]


def _prep(x, y, luma, crop_border: int, data_range: Optional[float]):
    """Shape check, data range, luma mode, border crop (a view)."""
    x4, y4 = _check_pair(x, y)
    L = float(data_range) if data_range is not None else _infer_data_range(x4)
    mode = _resolve_luma(luma)
    return _crop_border(x4, crop_border), _crop_border(y4, crop_border), L, mode


def _luma_tuple(mode, L):
    """(kr, kg, kb, offset in data units) of a luma convention, for the kernels."""
    kr, kg, kb, off = LUMA_COEFFS[mode]
    return (kr, kg, kb, off * L)


def _luma_arg_checked(x4, mode, L):
    """The kernels' luma tuple for a pixel reduction, after the channel check."""
    if mode is None:
        return None
    if x4.shape[1] != 3:
        raise ValueError(f"luma needs a 3-channel image, got {x4.shape[1]} channels")
    return _luma_tuple(mode, L)


def _apply_luma(x4, y4, mode, L, dtype):
    if mode is None:
        return x4, y4
    return (rgb_to_luma(x4, mode, data_range=L, dtype=dtype),
            rgb_to_luma(y4, mode, data_range=L, dtype=dtype))


def _no_autocast(t: torch.Tensor):
    """Convolutions of the portable path run at the tensor's own dtype."""
    return torch.autocast(device_type=t.device.type, enabled=False)


def _check_reduction(reduction: str) -> None:
    if reduction not in ("mean", "none"):
        raise ValueError(f"reduction must be 'mean' or 'none', got {reduction!r}")


# --------------------------------------------------------------------------- #
# MSE / PSNR
# --------------------------------------------------------------------------- #


def _sum_sq(x, y, dtype, per_image):
    from . import backend

    backend.note_portable("mse", x)
    d = x.to(dtype) - y.to(dtype)
    if per_image:
        return (d * d).sum(dim=(1, 2, 3), dtype=torch.float64) / d[0].numel()
    return (d * d).sum(dtype=torch.float64) / d.numel()


def mse(x: torch.Tensor, y: torch.Tensor, *, reduction: str = "mean",
        dtype: Optional[torch.dtype] = None, out_dtype: torch.dtype = torch.float64,
        luma=None, crop_border: int = 0) -> torch.Tensor:
    """Mean squared error; ``reduction="none"`` gives one value per image.

    uint8 pairs are reduced in exact integer arithmetic on the GPU.
    """
    x4, y4, L, mode = _prep(x, y, luma, crop_border, None)
    wdt = _work_dtype(x4, dtype)
    _check_reduction(reduction)
    per_image = reduction == "none"
    from . import backend

    # luma is formed inside the kernel and crops are read in place
    fast = backend.try_mse(x4, y4, per_image=per_image, dtype=out_dtype,
                           luma=_luma_arg_checked(x4, mode, L))
    if fast is not None:
        return fast
    x4, y4 = _apply_luma(x4, y4, mode, L, wdt)
    if mode is not None:  # the host kernels take the luma plane formed here
        fast = backend.try_mse(x4, y4, per_image=per_image, dtype=out_dtype)
        if fast is not None:
            return fast
    return _sum_sq(x4, y4, wdt, per_image).to(out_dtype)


def psnr(x: torch.Tensor, y: torch.Tensor, *, data_range: Optional[float] = None,
         reduction: str = "mean", dtype: Optional[torch.dtype] = None,
         out_dtype: torch.dtype = torch.float64, eps: float = 0.0, luma=None,
         crop_border: int = 0) -> torch.Tensor:
    """Peak signal-to-noise ratio in dB; identical inputs give ``+inf`` unless ``eps``."""
    _check_reduction(reduction)
    x4, y4, L, mode = _prep(x, y, luma, crop_border, data_range)
    bias = 10.0 * math.log10(L * L)
    from . import backend

    if not eps:
        # the dB conversion happens inside the reduction's finalize kernel, the
        # luma plane inside the reduction, and crops are read in place
        fast = backend.try_mse(x4, y4, per_image=reduction == "none", dtype=out_dtype,
                               psnr_bias=bias, luma=_luma_arg_checked(x4, mode, L))
        if fast is not None:
            return fast
    x4, y4 = _apply_luma(x4, y4, mode, L, _work_dtype(x4, dtype))
    m = mse(x4, y4, reduction=reduction, dtype=dtype, out_dtype=out_dtype)
    if eps:
        m = m.clamp_min(eps)
    # a host constant minus a device term: no H2D copy, capture-safe
    return bias - 10.0 * torch.log10(m)


# --------------------------------------------------------------------------- #
# SSIM
# --------------------------------------------------------------------------- #

_window_cache: dict = {}


def gaussian_window_1d(win_size: int = 11, sigma: float = 1.5, *, device=None,
                       dtype=torch.float32) -> torch.Tensor:
    """1-D factor of MATLAB's ``fspecial('gaussian', win_size, sigma)``.

    Normalised in float64, then cast; its outer product with itself is the
    normalised 2-D window.  Cached per (size, sigma, device, dtype) so that no
    call after the first performs a host-to-device copy.
    """
    key = (int(win_size), float(sigma), str(device), dtype)
    w = _window_cache.get(key)
    if w is None:
        half = (win_size - 1) / 2.0
        t = torch.arange(win_size, dtype=torch.float64) - half
        g = torch.exp(-(t * t) / (2.0 * sigma * sigma))
        w = (g / g.sum()).to(device=device, dtype=dtype)
        _window_cache[key] = w
    return w


def _f32_window(win: torch.Tensor) -> torch.Tensor:
    """The float32 window the kernels take, for a window of any dtype: the
    cached float32 copy when ``win`` came from :func:`gaussian_window_1d`."""
    if win.dtype == torch.float32:
        return win
    return win.to(torch.float32).contiguous()


def _moments_filtered(x4, y4, win, wdt, shift):
    """Separable 'valid' Gaussian of [x', y', x'^2, y'^2, x'y'], x' = x - shift.

    Returns a tuple of five (N, C, H-K+1, W-K+1) tensors.
    """
    from . import backend

    backend.note_portable("ssim_moments", x4)
    xs = x4.to(wdt) - shift
    ys = y4.to(wdt) - shift
    planes = torch.stack([xs, ys, xs * xs, ys * ys, xs * ys])  # (5, N, C, H, W)
    five, n, c, h, w = planes.shape
    k = win.numel()
    flat = planes.reshape(five * n * c, 1, h, w)
    wv = win.to(wdt)
    with _no_autocast(flat):
        flat = F.conv2d(flat, wv.view(1, 1, 1, k))
        flat = F.conv2d(flat, wv.view(1, 1, k, 1))
    return tuple(flat.reshape(five, n, c, h - k + 1, w - k + 1).unbind(0))


def _ssim_and_cs_maps(mom, shift, C1, C2):
    ux, uy, exx, eyy, exy = mom
    mx, my = ux + shift, uy + shift
    sxx = exx - ux * ux
    syy = eyy - uy * uy
    sxy = exy - ux * uy
    cs = (2.0 * sxy + C2) / (sxx + syy + C2)
    lum = (2.0 * mx * my + C1) / (mx * mx + my * my + C1)
    return lum * cs, cs


def _reject_double_backward() -> None:
    """The fused backward is a kernel, not an autograd graph: refuse
    ``create_graph=True`` instead of returning a silently-zero second
    derivative (reference functional.py:496-518)."""
    if torch.is_grad_enabled():
        raise RuntimeError(
            "frame_analytics_amd's fused SSIM backward is not twice differentiable, "
            "so create_graph=True (gradient penalties, Hessian-vector products, "
            "torch.func.hessian, MAML-style inner loops) cannot use it. For a "
            "second derivative use the portable path:\n"
            "    ...(x, y, backend_hint='torch')")


class _NativeSSIM(torch.autograd.Function):
    """Differentiable SSIM statistics from the gfx950 kernels, one class for
    every form the public functions need (``form``):

    * ``"mean"``: the batch-mean SSIM (``fa_gpu_ssim``).  The backward hands
      the upstream gradient to the kernel as a 1-element device tensor, so it
      never synchronises.
    * ``"map"``: the float32 SSIM map; the backward takes the map's gradient.
    * ``"cs"``: MS-SSIM's per-plane means ``(ssim, cs)`` (``fa_gpu_ssim_cs``).
    * ``"cs+pool"``: the same plus the next pyramid level ``(px, py)`` from
      the same pass (``fa_gpu_ssim_cs_ex``); the backward spreads a quarter of
      the level's gradient over each 2x2 block inside the scatter of the
      (ssim, cs) gradient (``fa_gpu_ssim_cs_backward_ex``), so a scale costs
      one forward and two backward launches whatever reaches it.

    x, y and the window are kept and the backward recomputes the moments from
    them (the reference keeps the same memory profile, functional.py:521-572
    and :749-783) -- except where the caller says which plane mean its loss
    reads (``use``, "s" or "cs": MS-SSIM reads cs below its coarsest scale and
    SSIM there) and the input is float32 or float64.  Then the forward runs in
    float64 and also writes the backward's coefficient maps for a unit
    gradient of that mean (``fa_gpu_ssim_cs_coef``, 3 float32 per output
    pixel, 4 when y needs a gradient, kept until the backward), and the
    backward is the scatter alone, each plane scaled by its upstream gradient
    (``fa_gpu_ssim_cs_scatter``); a backward that receives the other mean's
    gradient too recomputes, as without ``use``.  ``consts`` is (shift, C1,
    C2).
    """

    @staticmethod
    def forward(ctx, x, y, win, consts, form, pool_dtype, use=None):
        from . import backend

        shift, C1, C2 = consts
        ctx.set_materialize_grads(False)
        ctx.save_for_backward(x, y, win)
        ctx.consts, ctx.form, ctx.aux, ctx.use = consts, form, None, use
        if form in ("mean", "map"):
            res = backend.ssim_fused(x, y, win, shift, C1, C2, form == "map")
            return res[2] if form == "map" else res[1]
        need_dx, need_dy = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if (use is not None and (need_dx or need_dy)
                and x.dtype in (torch.float32, torch.float64)):
            s, cs, px, py, ctx.aux = backend.ssim_cs_coef_forward(
                x, y, win, shift, C1, C2, use == "s",
                pool_dtype if form == "cs+pool" else None, need_dy)
            if form == "cs":
                return s, cs
        elif form == "cs":
            return backend.ssim_cs_forward(x, y, win, shift, C1, C2)
        else:
            s, cs, px, py = backend.ssim_cs_forward(x, y, win, shift, C1, C2, pool_dtype)
        # a level of an input that needs no gradient needs none either: without
        # this the next scale would compute (and this one spread) its gradient
        for level, wanted in ((px, ctx.needs_input_grad[0]), (py, ctx.needs_input_grad[1])):
            if not wanted:
                ctx.mark_non_differentiable(level)
        return s, cs, px, py

    @staticmethod
    def backward(ctx, *grads):
        from . import backend

        _reject_double_backward()
        need_dx, need_dy = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        nothing = (None,) * 7
        if not (need_dx or need_dy) or all(g is None for g in grads):
            return nothing
        x, y, win = ctx.saved_tensors
        shift, C1, C2 = ctx.consts
        if ctx.form in ("mean", "map"):
            g = grads[0]
            dmap = g if ctx.form == "map" else None
            gscalar = None if ctx.form == "map" else g.reshape(1)
            dx, dy = backend.ssim_backward(x, y, dmap, gscalar, win, shift, C1, C2,
                                           need_dx, need_dy)
        else:
            planes = x.shape[0] * x.shape[1]
            g_px, g_py = grads[2:4] if ctx.form == "cs+pool" else (None, None)
            g_used, g_other = (grads[0], grads[1]) if ctx.use == "s" else (grads[1], grads[0])
            if ctx.aux is not None and g_other is None:
                if g_used is None:
                    g_used = x.new_zeros(planes, dtype=torch.float32)
                dx, dy = backend.ssim_cs_scatter(x, y, g_used, ctx.aux, win, shift, need_dx,
                                                 need_dy, g_px, g_py)
                ctx.aux = None
                return (dx if need_dx else None, dy if need_dy else None) + nothing[2:]
            g_s, g_cs = (g if g is not None else x.new_zeros(planes, dtype=torch.float32)
                         for g in grads[:2])
            dx, dy = backend.ssim_cs_backward(x, y, g_s, g_cs, win, shift, C1, C2,
                                              need_dx, need_dy, g_px, g_py)
        return (dx if need_dx else None, dy if need_dy else None) + nothing[2:]


def _matlab_downsample(x: torch.Tensor, f: int) -> torch.Tensor:
    """MATLAB ``ssim.m``'s automatic f x f box downsample (replicate padding,
    every f-th sample), reference functional.py:575-586."""
    if f <= 1:
        return x
    n, c, h, w = x.shape
    pad = f // 2
    xp = F.pad(x.reshape(n * c, 1, h, w), (pad, pad, pad, pad), mode="replicate")
    ker = x.new_full((1, 1, f, f), 1.0 / (f * f))
    with _no_autocast(xp):
        lp = F.conv2d(xp, ker)
    return lp.reshape(n, c, lp.shape[-2], lp.shape[-1])[:, :, ::f, ::f].contiguous()


def ssim(x: torch.Tensor, y: torch.Tensor, *, data_range: Optional[float] = None,
         win_size: int = 11, sigma: float = 1.5, K: Sequence[float] = (0.01, 0.03),
         reduction: str = "mean", return_map: bool = False,
         dtype: Optional[torch.dtype] = None, downsample: bool = False,
         backend_hint: str = "auto", luma=None, crop_border: int = 0) -> torch.Tensor:
    """Structural similarity (Wang et al. 2004), ``ssim_index.m`` defaults:
    11x11 Gaussian window, sigma 1.5, K = (0.01, 0.03), 'valid' support."""
    _check_reduction(reduction)
    x4, y4, L, mode = _prep(x, y, luma, crop_border, data_range)
    wdt = _work_dtype(x4, dtype)
    C1 = (float(K[0]) * L) ** 2
    C2 = (float(K[1]) * L) ** 2
    from . import backend

    # Inference on the GPU: the kernel forms the luma plane and reads crops in
    # place, so neither is materialised first.
    grad = torch.is_grad_enabled() and (x4.requires_grad or y4.requires_grad)
    if (backend_hint != "torch" and not grad and not downsample and mode is not None
            and x4.shape[-2] >= win_size and x4.shape[-1] >= win_size):
        if x4.shape[1] != 3:
            raise ValueError(f"luma needs a 3-channel image, got {x4.shape[1]} channels")
        fast = backend.try_ssim(x4, y4, win_size=win_size, sigma=sigma, shift=0.5 * L,
                                C1=C1, C2=C2, reduction=reduction, return_map=return_map,
                                dtype=wdt, luma=_luma_tuple(mode, L))
        if fast is not None:
            return fast
    x4, y4 = _apply_luma(x4, y4, mode, L, wdt)
    if downsample:
        f = max(1, int(round(min(x4.shape[-2], x4.shape[-1]) / 256.0)))
        if f > 1:
            x4 = _matlab_downsample(x4.to(wdt), f)
            y4 = _matlab_downsample(y4.to(wdt), f)
    if x4.shape[-2] < win_size or x4.shape[-1] < win_size:
        raise ValueError(f"image {tuple(x4.shape[-2:])} smaller than window {win_size}x{win_size}")
    shift = 0.5 * L

    if (backend_hint != "torch" and (x4.requires_grad or y4.requires_grad)
            and torch.is_grad_enabled() and reduction == "mean" and not downsample
            and backend.ssim_autograd_available(x4, y4, win_size)):
        win = gaussian_window_1d(win_size, sigma, device=x4.device, dtype=torch.float32)
        return _NativeSSIM.apply(x4, y4, win, (shift, C1, C2),
                                 "map" if return_map else "mean", None)

    if backend_hint != "torch":
        fast = backend.try_ssim(x4, y4, win_size=win_size, sigma=sigma, shift=shift,
                                C1=C1, C2=C2, reduction=reduction, return_map=return_map,
                                dtype=wdt)
        if fast is not None:
            return fast
        if backend_hint == "native":
            raise RuntimeError("native SSIM backend unavailable for these inputs")

    win = gaussian_window_1d(win_size, sigma, device=x4.device, dtype=wdt)
    smap, _ = _ssim_and_cs_maps(_moments_filtered(x4, y4, win, wdt, shift), shift, C1, C2)
    if return_map:
        return smap
    if reduction == "none":
        return smap.mean(dim=(1, 2, 3), dtype=torch.float64)
    return smap.mean(dtype=torch.float64)


# --------------------------------------------------------------------------- #
# MS-SSIM
# --------------------------------------------------------------------------- #

# Wang et al. 2003, table 1
MS_SSIM_WEIGHTS = (0.0448, 0.2856, 0.3001, 0.2363, 0.1333)

@functools.lru_cache(maxsize=64)
def _scale_exponents(weights: Tuple[float, ...], device: str) -> torch.Tensor:
    """MS-SSIM's scale weights as an ``(M, 1, 1)`` float64 tensor on ``device``,
    built once per (weights, device): a fresh tensor per call would be a
    host-to-device copy, which a graph capture cannot hold."""
    return torch.tensor(weights, dtype=torch.float64).view(-1, 1, 1).to(torch.device(device))


@functools.lru_cache(maxsize=16)
def _cofactor_mask(m: int, device: str) -> torch.Tensor:
    """``(m, m, 1, 1)`` bool, true on the diagonal: row k masks factor k."""
    return torch.eye(m, dtype=torch.bool).view(m, m, 1, 1).to(torch.device(device))


class _CombineScales(torch.autograd.Function):
    """The product of :func:`_combine_scales` with a backward that never waits
    for the host.  torch's ``prod`` backward counts the zero factors with a
    device-to-host read, so a training step would stop there until the device
    caught up and issue every later launch of its backward behind the host;
    here each factor's gradient takes the product of the other factors (a
    masked product, exact where factors are zero) and the derivatives of the
    clamp and the power as torch forms them: no gradient where t < 0 or the
    exponent is 0, inf for a zero factor under a fractional exponent.  The
    backward recomputes from the saved input, so its operations differentiate
    again under ``create_graph``."""

    @staticmethod
    def forward(ctx, stacked, expo):
        ctx.save_for_backward(stacked, expo)
        return stacked.clamp_min(0.0).pow(expo).prod(dim=0)

    @staticmethod
    def backward(ctx, g):
        stacked, expo = ctx.saved_tensors
        t = stacked.clamp_min(0.0)
        p = t.pow(expo)
        m = p.shape[0]
        others = p.unsqueeze(0).expand(m, *p.shape).masked_fill(
            _cofactor_mask(m, str(p.device)), 1.0).prod(dim=1)
        dpow = torch.where(expo == 0.0, 0.0, expo * t.pow(expo - 1.0))
        grad = torch.where(stacked >= 0.0, (g * others) * dpow, 0.0)
        return grad.to(stacked.dtype), None


class _MsHead(torch.autograd.Function):
    """MS-SSIM's head over the scales' ``(N, C)`` plane means on the GPU: the
    scale product, the channel mean and (``per_image`` false) the batch mean
    in one launch (``fa_gpu_ms_ssim_head``), and every scale's gradient in
    one launch back (``fa_gpu_ms_ssim_head_backward``), where the same torch
    expression (:func:`_combine_scales`, then the means) takes about six
    launches forward and twenty back per training step.  The derivatives are
    torch's (the clamp, the power, the product, the means); like the scales'
    fused backward it is not twice differentiable."""

    @staticmethod
    def forward(ctx, weights, per_image, *terms):
        from . import backend

        ctx.save_for_backward(*terms)
        ctx.weights, ctx.per_image = weights, per_image
        ctx.set_materialize_grads(False)
        return backend.ms_head(terms, weights, per_image)

    @staticmethod
    def backward(ctx, g):
        from . import backend

        _reject_double_backward()
        terms = ctx.saved_tensors
        needs = ctx.needs_input_grad[2:]
        if g is None or not any(needs):
            return (None, None) + (None,) * len(terms)
        grads = backend.ms_head_backward(terms, ctx.weights, ctx.per_image, g, needs)
        return (None, None, *grads)


def _combine_scales(terms, weights, device) -> torch.Tensor:
    """Per plane: prod_j max(t_j, 0)^w_j over the stacked ``(N, C)`` terms (a
    fractional power of a negative factor is not real, hence the clamp)."""
    expo = _scale_exponents(tuple(weights), str(device))
    stacked = torch.stack(terms)
    if torch.is_grad_enabled() and stacked.requires_grad:
        return _CombineScales.apply(stacked, expo)
    return stacked.clamp_min(0.0).pow(expo).prod(dim=0)


def _ssim_cs_pair(x4, y4, win, wdt, shift, C1, C2, backend_hint):
    """``(ssim, cs)`` plane means, each ``(N, C)``."""
    from . import backend

    n, c = x4.shape[0], x4.shape[1]
    if (backend_hint != "torch" and (x4.requires_grad or y4.requires_grad)
            and torch.is_grad_enabled()
            and backend.ssim_cs_autograd_available(x4, y4, win.numel())):
        s, cs = _NativeSSIM.apply(x4, y4, _f32_window(win), (shift, C1, C2), "cs", None)
        return s.view(n, c), cs.view(n, c)
    if backend_hint != "torch":
        fast = backend.try_ssim_cs(x4, y4, win=win, shift=shift, C1=C1, C2=C2)
        if fast is not None:
            return fast
        if backend_hint == "native":
            raise RuntimeError("native SSIM/CS backend unavailable for these inputs")
    smap, cs = _ssim_and_cs_maps(_moments_filtered(x4, y4, win, wdt, shift), shift, C1, C2)
    return (smap.mean(dim=(2, 3), dtype=torch.float64),
            cs.mean(dim=(2, 3), dtype=torch.float64))


def ms_ssim(x: torch.Tensor, y: torch.Tensor, *, data_range: Optional[float] = None,
            win_size: int = 11, sigma: float = 1.5, K: Sequence[float] = (0.01, 0.03),
            weights: Optional[Sequence[float]] = None, reduction: str = "mean",
            dtype: Optional[torch.dtype] = None, backend_hint: str = "auto",
            luma=None, crop_border: int = 0) -> torch.Tensor:
    """Multi-scale SSIM (Wang, Simoncelli, Bovik 2003).

    ``prod_j cs_j^{w_j}`` with the full SSIM at the coarsest scale, scales
    separated by a non-overlapping 2x2 mean (odd trailing row/column dropped),
    factors clamped at zero, channels averaged after the product.  Needs
    ``win_size * 2**(scales-1)`` pixels on a side.
    """
    _check_reduction(reduction)
    w = tuple(float(v) for v in (weights if weights is not None else MS_SSIM_WEIGHTS))
    if not w:
        raise ValueError("weights must not be empty")
    x4, y4, L, mode = _prep(x, y, luma, crop_border, data_range)
    wdt = _work_dtype(x4, dtype)
    C1 = (float(K[0]) * L) ** 2
    C2 = (float(K[1]) * L) ** 2
    shift = 0.5 * L
    scales = len(w)
    need = win_size * (1 << (scales - 1))
    if min(x4.shape[-2], x4.shape[-1]) < need:
        raise ValueError(
            f"image {tuple(x4.shape[-2:])} is too small for {scales} scales with a "
            f"{win_size}x{win_size} window; needs at least {need} px on a side")

    from . import backend

    win = gaussian_window_1d(win_size, sigma, device=x4.device, dtype=wdt)
    terms = []
    grad = torch.is_grad_enabled() and (x4.requires_grad or y4.requires_grad)
    native = (backend_hint != "torch"
              and backend.ssim_cs_pool_available(x4, y4, win_size)
              and not (grad and torch.cuda.is_current_stream_capturing()))
    # without a gradient the first scale forms the luma plane itself (its
    # pyramid is float64); with one, luma is an autograd op in front
    lw = None
    if mode is not None:
        if x4.shape[1] != 3:
            raise ValueError(f"luma needs a 3-channel image, got {x4.shape[1]} channels")
        if native and not grad:
            lw = _luma_tuple(mode, L)
        else:
            x4, y4 = _apply_luma(x4, y4, mode, L, wdt)
    n, c = x4.shape[0], (1 if lw is not None else x4.shape[1])
    if native:
        # On the GPU every scale is one fused pass that also writes the next
        # pyramid level, held exactly (the coarse scales amplify a rounded
        # level ~100x in the gradient): float32 below uint8, float64 below
        # floating input.  float16 / bfloat16 widen exactly to float32 when a
        # gradient is wanted, and a float64 working dtype widens the input.
        if wdt == torch.float64 and x4.dtype != torch.float64:
            x4, y4 = x4.double(), y4.double()
        elif grad and x4.dtype in (torch.float16, torch.bfloat16):
            x4, y4 = x4.float(), y4.float()
        pdt = torch.float64 if lw is not None else backend.pyramid_dtype(x4.dtype)
        win32 = _f32_window(win)
        consts = (shift, C1, C2)
        cx, cy = x4, y4
        if not grad and len(w) <= 8:
            # inference: one library call runs every scale's fused pass (cs
            # sums, the SSIM sums at the coarsest scale, the next exact level:
            # float16 for the first level and float32 below it under uint8,
            # float64 otherwise) and the reduction (plane terms, product,
            # channel and batch means), with no host work between launches
            return backend.ms_ssim_fused(x4, y4, win32, shift, C1, C2, w, luma=lw,
                                         per_image=reduction == "none")
        for i in range(scales):
            last = i == scales - 1
            if grad:
                # the loss reads the SSIM means at the coarsest scale, cs below
                keep = backend.ms_ssim_keeps_coefficients()
                if last:
                    s, cs = _NativeSSIM.apply(cx, cy, win32, consts, "cs", None,
                                              "s" if keep else None)
                else:
                    s, cs, cx, cy = _NativeSSIM.apply(cx, cy, win32, consts, "cs+pool", pdt,
                                                      "cs" if keep else None)
            else:
                out = backend.ssim_cs_pool(cx, cy, win32, shift, C1, C2,
                                           None if last else pdt, luma=lw if i == 0 else None)
                s, cs = out[0], out[1]
                if not last:
                    cx, cy = out[2], out[3]
            terms.append((s if last else cs).view(n, c))
    else:
        # the portable path pools at the working dtype, as the reference does
        backend.note_portable("ms_ssim_pyramid", x4)
        cx, cy = x4, y4
        for i in range(scales):
            if i:
                cx = F.avg_pool2d(cx.to(wdt), 2)
                cy = F.avg_pool2d(cy.to(wdt), 2)
            s, cs = _ssim_cs_pair(cx, cy, win, wdt, shift, C1, C2, backend_hint)
            terms.append(s if i == scales - 1 else cs)
    if native and grad and backend.ms_head_available(terms):
        return _MsHead.apply(w, reduction == "none", *terms)
    per_image = _combine_scales(terms, w, x4.device).mean(dim=1)  # channels after the product
    return per_image if reduction == "none" else per_image.mean()


# --------------------------------------------------------------------------- #
# GMSD / GMS
# --------------------------------------------------------------------------- #

@functools.lru_cache(maxsize=16)
def _prewitt_bank(device: str, dtype: torch.dtype) -> torch.Tensor:
    """``(2, 1, 3, 3)``: the x and y Prewitt kernels with taps +-1/3, as one
    convolution bank, built once per (device, dtype)."""
    ramp = torch.tensor([1.0, 0.0, -1.0], dtype=torch.float64) / 3.0
    flat = torch.ones(3, dtype=torch.float64)
    bank = torch.stack([torch.outer(flat, ramp), torch.outer(ramp, flat)])
    return bank.unsqueeze(1).to(device=torch.device(device), dtype=dtype)


def _gms_map(x4, y4, wdt, T, eps, downsample):
    from . import backend

    backend.note_portable("gms_map", x4)
    xf, yf = x4.to(wdt), y4.to(wdt)
    if downsample:
        xf, yf = F.avg_pool2d(xf, 2), F.avg_pool2d(yf, 2)
    n, c, h, w = xf.shape
    if h < 3 or w < 3:
        raise ValueError(f"image {h}x{w} is smaller than the 3x3 Prewitt window")
    both = torch.cat([xf, yf], dim=0).reshape(2 * n * c, 1, h, w)
    with _no_autocast(both):
        g = F.conv2d(both, _prewitt_bank(str(xf.device), wdt))  # (2NC, 2, H-2, W-2)
    g1 = torch.sqrt((g[: n * c] ** 2).sum(dim=1) + eps)
    g2 = torch.sqrt((g[n * c:] ** 2).sum(dim=1) + eps)
    q = (2.0 * g1 * g2 + T) / (g1 * g1 + g2 * g2 + T)
    return q.reshape(n, c, h - 2, w - 2)


class _FusedGMSD(torch.autograd.Function):
    """Differentiable native per-image ``(mean q, std q)`` of the GMS map
    (``fa_gpu_gmsd`` forward, ``fa_gpu_gmsd_backward`` in float64)."""

    @staticmethod
    def forward(ctx, x, y, T, eps, downsample):
        from . import backend

        mean, std = backend.gmsd_stats_fwd(x, y, T, eps, downsample)
        ctx.save_for_backward(x, y, mean, std)
        ctx.consts = (T, eps, downsample)
        ctx.set_materialize_grads(False)
        return mean, std

    @staticmethod
    def backward(ctx, g_mean, g_std):
        from . import backend

        _reject_double_backward()
        x, y, mean, std = ctx.saved_tensors
        T, eps, downsample = ctx.consts
        need_dx, need_dy = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if not (need_dx or need_dy) or (g_mean is None and g_std is None):
            return (None,) * 5
        dx, dy = backend.gmsd_stats_bwd(x, y, mean, std, g_mean, g_std, T, eps, downsample,
                                        need_dx, need_dy)
        return dx if need_dx else None, dy if need_dy else None, None, None, None


def _gmsd_common(x, y, data_range, T, eps, downsample, dtype, luma, crop_border,
                 reduction, return_map, backend_hint):
    """``(map, None)`` or ``(None, (gms_mean, gmsd))`` per image."""
    _check_reduction(reduction)
    x4, y4, L, mode = _prep(x, y, luma, crop_border, data_range)
    wdt = _work_dtype(x4, dtype)
    Tv = float(T) if T is not None else 170.0 * (L / 255.0) ** 2
    ev = float(eps) if eps is not None else (1e-6 * L) ** 2
    grad = torch.is_grad_enabled() and (x4.requires_grad or y4.requires_grad)
    if backend_hint != "torch" and grad and not return_map:
        # training: luma (if any) is an autograd op in front, then the native
        # statistics with a float64 backward
        from . import backend

        xl, yl = _apply_luma(x4, y4, mode, L, wdt)
        if xl.dtype in (torch.float16, torch.bfloat16):
            xl, yl = xl.float(), yl.float()
        if backend.gmsd_autograd_available(xl, yl):
            return None, _FusedGMSD.apply(xl, yl, Tv, ev, downsample)
    if backend_hint != "torch":
        from . import backend

        # The kernel forms the luma plane itself (its offset cancels out of
        # every gradient) and reads crops in place; its statistics are
        # float64-accurate, so a float64 working dtype needs no other path.
        # Its map is float32, so a float64 map takes the portable path.
        if mode is not None and x4.shape[1] != 3:
            raise ValueError(f"luma needs a 3-channel image, got {x4.shape[1]} channels")
        lw = LUMA_COEFFS[mode][:3] if mode is not None else None
        fast = None
        if not (return_map and wdt == torch.float64):
            fast = backend.try_gmsd(x4, y4, T=Tv, eps=ev, downsample=downsample, luma=lw,
                                    want_map=return_map)
        if fast is not None:
            if return_map:
                return (fast[2] if wdt == torch.float32 else fast[2].to(wdt)), None
            return None, fast
        if backend_hint == "native":
            raise RuntimeError("native GMSD backend unavailable for these inputs")
    x4, y4 = _apply_luma(x4, y4, mode, L, wdt)
    if mode is not None and backend_hint != "torch" and not return_map:
        from . import backend  # host kernels: luma formed here

        fast = backend.try_gmsd(x4, y4, T=Tv, eps=ev, downsample=downsample)
        if fast is not None:
            return None, fast
    q = _gms_map(x4, y4, wdt, Tv, ev, downsample)
    if return_map:
        return q, None
    # widen before the variance: q sits within ~1e-3 of 1 on a good match
    f = q.reshape(q.shape[0], -1).double()
    return None, (f.mean(dim=1), f.var(dim=1, correction=0).clamp_min(0.0).sqrt())


def gms(x: torch.Tensor, y: torch.Tensor, *, data_range: Optional[float] = None,
        T: Optional[float] = None, eps: Optional[float] = None, downsample: bool = True,
        reduction: str = "mean", return_map: bool = False,
        dtype: Optional[torch.dtype] = None, luma=None, crop_border: int = 0,
        backend_hint: str = "auto") -> torch.Tensor:
    """Mean gradient-magnitude similarity; higher is better, 1.0 is identical."""
    q, stats = _gmsd_common(x, y, data_range, T, eps, downsample, dtype, luma,
                            crop_border, reduction, return_map, backend_hint)
    if q is not None:
        return q
    if reduction == "none":
        return stats[0]
    # the native statistics come with their batch means, formed in the kernel
    return stats[2][0] if len(stats) > 2 and stats[2] is not None else stats[0].mean()


def gmsd(x: torch.Tensor, y: torch.Tensor, *, data_range: Optional[float] = None,
         T: Optional[float] = None, eps: Optional[float] = None, downsample: bool = True,
         reduction: str = "mean", return_map: bool = False,
         dtype: Optional[torch.dtype] = None, luma=None, crop_border: int = 0,
         backend_hint: str = "auto") -> torch.Tensor:
    """Gradient magnitude similarity deviation (Xue et al. 2014); lower is better."""
    q, stats = _gmsd_common(x, y, data_range, T, eps, downsample, dtype, luma,
                            crop_border, reduction, return_map, backend_hint)
    if q is not None:
        return q
    if reduction == "none":
        return stats[1]
    return stats[2][1] if len(stats) > 2 and stats[2] is not None else stats[1].mean()


# --------------------------------------------------------------------------- #
# pixel losses
# --------------------------------------------------------------------------- #

# op codes of include/fa_abi.h
_OP_MSE = 0
_OP_L1 = 1
_OP_CHARB = 2
_OP_HUBER = 3


def _pixel_terms(name, d, param):
    if name == "l1":
        return d.abs()
    if name == "charbonnier":
        return torch.sqrt(d * d + param)
    a = d.abs()
    return torch.where(a <= param, 0.5 * a * a, param * (a - 0.5 * param))


_PIXEL_OPS = {"l1": _OP_L1, "charbonnier": _OP_CHARB, "huber": _OP_HUBER}


def _pixel_loss(name, x, y, param, reduction, dtype, out_dtype, luma, crop_border,
                backend_hint):
    _check_reduction(reduction)
    x4, y4, L, mode = _prep(x, y, luma, crop_border, None)
    wdt = _work_dtype(x4, dtype)
    per_image = reduction == "none"
    from . import backend

    if backend_hint != "torch":
        fast = backend.try_pixel(x4, y4, op=_PIXEL_OPS[name], param=param,
                                 per_image=per_image, dtype=out_dtype,
                                 luma=_luma_arg_checked(x4, mode, L))
        if fast is not None:
            return fast
        if backend_hint == "native":
            raise RuntimeError(f"native {name} backend unavailable for these inputs")
    x4, y4 = _apply_luma(x4, y4, mode, L, wdt)
    if mode is not None and backend_hint != "torch":  # host kernels: luma formed here
        fast = backend.try_pixel(x4, y4, op=_PIXEL_OPS[name], param=param,
                                 per_image=per_image, dtype=out_dtype)
        if fast is not None:
            return fast
    backend.note_portable(name, x4)
    t = _pixel_terms(name, x4.to(wdt) - y4.to(wdt), param)
    if per_image:
        out = t.sum(dim=(1, 2, 3), dtype=torch.float64) / t[0].numel()
    else:
        out = t.sum(dtype=torch.float64) / t.numel()
    return out.to(out_dtype)


def l1(x: torch.Tensor, y: torch.Tensor, *, reduction: str = "mean",
       dtype: Optional[torch.dtype] = None, out_dtype: torch.dtype = torch.float64,
       luma=None, crop_border: int = 0, backend_hint: str = "auto") -> torch.Tensor:
    """Mean absolute error, in the input's own units."""
    return _pixel_loss("l1", x, y, 0.0, reduction, dtype, out_dtype, luma, crop_border,
                       backend_hint)


def charbonnier(x: torch.Tensor, y: torch.Tensor, *, eps: float = 1e-3,
                reduction: str = "mean", dtype: Optional[torch.dtype] = None,
                out_dtype: torch.dtype = torch.float64, luma=None, crop_border: int = 0,
                backend_hint: str = "auto") -> torch.Tensor:
    """``mean sqrt((x - y)^2 + eps^2)``; ``eps`` has the units of the residual."""
    return _pixel_loss("charbonnier", x, y, float(eps) ** 2, reduction, dtype, out_dtype,
                       luma, crop_border, backend_hint)


def huber(x: torch.Tensor, y: torch.Tensor, *, delta: float = 1.0, reduction: str = "mean",
          dtype: Optional[torch.dtype] = None, out_dtype: torch.dtype = torch.float64,
          luma=None, crop_border: int = 0, backend_hint: str = "auto") -> torch.Tensor:
    """Huber loss, term for term ``torch.nn.HuberLoss``."""
    if delta <= 0:
        raise ValueError(f"delta must be > 0, got {delta}")
    return _pixel_loss("huber", x, y, float(delta), reduction, dtype, out_dtype, luma,
                       crop_border, backend_hint)
