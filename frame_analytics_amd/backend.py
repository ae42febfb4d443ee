"""Dispatch to the gfx950 kernels: tensors in, raw pointers across the C ABI.

Counterpart of the reference's ``frame_analytics/backend.py``.  Shapes and
dtypes become ints, tensors become device pointers, and every buffer the
kernels write -- scratch included -- is allocated here through torch's caching
allocator, so no call ever allocates inside the library and every call stays
legal inside a HIP graph capture (reference backend.py:145-153).

Failure policy (deliberately stricter than the reference, which warns once and
falls back to PyTorch, backend.py:215-224):

* on a machine with a GPU the kernel library must load; if it cannot, the
  first call raises.  ``FA_NATIVE=0`` is the explicit opt-out.
* a kernel that returns a non-zero status raises :class:`KernelError`; there is
  no silent retry on another path.
* ``try_*`` return ``None`` only when the native path does not apply to the
  call by design (a gradient that the kernel cannot give, a window width
  without a kernel, a CPU tensor on a host without the CPU library); the
  caller then takes the portable path, exactly where the reference would.

CPU tensors go to the host kernel library ``libfa_cpu.so``
(``include/fa_cpu_abi.h``) for inference calls, as in the reference
(backend.py:318-328, 505-515, 615-622, 656-662).  That library is optional:
without it (or on a CPU without AVX2 + FMA) CPU tensors take the portable
path, which is the reference's own behaviour on such hosts.
"""

from __future__ import annotations

import ctypes
import os
from typing import Any, Optional

import torch

from ._cabi import KernelError, status_text  # noqa: F401

_SUPPORTED = (torch.uint8, torch.float16, torch.bfloat16, torch.float32, torch.float64)

# mirrors the dtype codes of include/fa_abi.h (reference backend.py:37-43)
_DTYPE_CODE = {
    torch.uint8: 0,
    torch.float16: 1,
    torch.bfloat16: 2,
    torch.float32: 3,
    torch.float64: 4,
}
# include/fa_abi.h: OR-ed into FA_F32 for the float32 levels of a uint8 pyramid
FA_DTYPE_U8_PYRAMID = 0x100

_PSNR_NONE = -1.0e300
_OP_MSE = 0
_WINDOWS = (3, 5, 7, 9, 11)


class _Native:
    """What :func:`load` hands back: the kernel library and where it came from."""

    def __init__(self) -> None:
        self.gpu: Any = None
        self.gpu_origin: Optional[str] = None
        self.gpu_error: Optional[str] = None

    @property
    def has_gpu(self) -> bool:
        return self.gpu is not None


_ext: Optional[_Native] = None
_load_error: Optional[str] = None


def _disabled() -> bool:
    return os.environ.get("FA_NATIVE", "auto").lower() in ("0", "off", "false", "no")


def load(force: bool = False) -> Optional[_Native]:
    """Load the kernel library (building it in-tree first if it is missing).

    Returns ``None`` when native kernels are disabled (``FA_NATIVE=0``) or when
    the machine has no GPU.  On a machine with a GPU a library that will not
    load raises: a GPU call must never quietly run somewhere else.
    """
    global _ext, _load_error
    if _ext is not None and not force:
        return _ext
    if _disabled():
        _load_error = "disabled via FA_NATIVE"
        return None
    if not torch.cuda.is_available():
        _load_error = "no GPU visible"
        return None
    from . import _cabi

    native = _Native()
    try:
        native.gpu, native.gpu_origin = _cabi.load_gpu()
    except Exception as exc:
        _load_error = f"{type(exc).__name__}: {exc}"
        raise RuntimeError(
            "frame_analytics_amd: the gfx950 kernel library failed to load "
            f"({_load_error}); set FA_NATIVE=0 to run the portable PyTorch "
            "path on purpose") from exc
    _load_error = None
    _ext = native
    return _ext


_cpu: Any = None
_cpu_state: Optional[str] = None  # None: not tried yet; "" loaded; else why not


def load_cpu() -> Any:
    """The host kernel library, or ``None`` (``FA_NATIVE=0``, a CPU without
    AVX2 + FMA, or a library that cannot be built here).  Its pool is sized
    to ``torch.get_num_threads()`` on first load (reference backend.py:94-97)."""
    global _cpu, _cpu_state
    if _cpu_state is not None:
        return _cpu
    if _disabled():
        _cpu_state = "disabled via FA_NATIVE"
        return None
    from . import _cabi

    try:
        lib, why = _cabi.load_cpu()
    except Exception as exc:  # no compiler / no library: the portable path serves
        lib, why = None, f"{type(exc).__name__}: {exc}"
    if lib is not None:
        lib.fa_cpu_set_num_threads(int(torch.get_num_threads()))
        why = ""
    _cpu, _cpu_state = lib, why
    return _cpu


def _cpu_ready(x: torch.Tensor, y: torch.Tensor) -> Any:
    """The host library when an inference call on CPU tensors can use it."""
    if x.is_cuda or y.is_cuda or x.device.type != "cpu" or not _usable(x, y):
        return None
    if x.dim() != 4 or x.shape != y.shape or x.numel() == 0:
        return None
    return load_cpu()


def _check_cpu(code: int) -> None:
    if code != 0:
        raise KernelError(f"host kernel returned status {code}")


def status() -> dict:
    try:
        ext = load()
    except RuntimeError:
        ext = None
    path = None
    if ext is not None:
        from . import _build

        path = str(_build.library_path())
    return {
        "available": ext is not None,
        "gpu": bool(ext is not None and ext.has_gpu),
        "error": _load_error,
        "gpu_source": None if ext is None else ext.gpu_origin,
        "gpu_library": path,
        "cpu": load_cpu() is not None,
        "cpu_error": _cpu_state or None,
    }


# --------------------------------------------------------------------------- #
# marshalling helpers
# --------------------------------------------------------------------------- #


def _f64(device, *shape) -> torch.Tensor:
    return torch.empty(shape, device=device, dtype=torch.float64)


def _contig(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() else t.contiguous()


def _view_strides(t: torch.Tensor):
    """``(tensor, strides)``: a unit-column-stride view passes its (image,
    channel, row) strides as an int64[3] host array; anything else is copied
    contiguous and passes null."""
    if t.is_contiguous():
        return t, None
    if t.stride(-1) != 1 or min(t.stride()) < 0:
        return t.contiguous(), None
    return t, (ctypes.c_int64 * 3)(t.stride(0), t.stride(1), t.stride(2))


def _luma_arg(luma: Optional[tuple]):
    """{kr, kg, kb, offset} as a double[4] host array, or None."""
    if luma is None:
        return None
    kr, kg, kb, off = (tuple(luma) + (0.0,))[:4]
    return (ctypes.c_double * 4)(float(kr), float(kg), float(kb), float(off))


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _dev(t: torch.Tensor) -> int:
    i = t.device.index
    return torch.cuda.current_device() if i is None else int(i)


def _stream(t: torch.Tensor):
    return torch.cuda.current_stream(t.device).cuda_stream


def _check(code: int, ext: _Native) -> None:
    if code != 0:
        raise KernelError(status_text(code, ext.gpu))


_win_cache: dict = {}


def _win_f32(win: torch.Tensor) -> torch.Tensor:
    """The window as contiguous float32, cast once per cached window."""
    if win.dtype == torch.float32:
        return _contig(win)
    key = (id(win), str(win.device))
    hit = _win_cache.get(key)
    if hit is not None and hit[0] is win:
        return hit[1]
    w = win.to(torch.float32).contiguous()
    _win_cache[key] = (win, w)
    return w


def _usable(x: torch.Tensor, y: torch.Tensor) -> bool:
    """Inference-only kernels serve a call unless a gradient is actually wanted
    (reference backend.py:227-244)."""
    grad_wanted = torch.is_grad_enabled() and (x.requires_grad or y.requires_grad)
    return x.dtype in _SUPPORTED and x.dtype == y.dtype and not grad_wanted


def _gpu_ext(x: torch.Tensor) -> Optional[_Native]:
    """The loaded library when ``x`` lives on the GPU, else ``None``."""
    if not x.is_cuda:
        return None
    ext = load()
    if ext is None or not ext.has_gpu:
        return None
    return ext


# Workspace sizes depend on the shape only; caching them keeps the runtime
# query out of graph capture (reference backend.py:247-286).
_ws_cache: dict = {}


def _pixel_workspace(ext: _Native, n_images: int, n_per_image: int, dev: int) -> int:
    key = ("pix", n_images, n_per_image, dev)
    hit = _ws_cache.get(key)
    if hit is None:
        out = ctypes.c_int(0)
        _check(ext.gpu.fa_gpu_pixel_workspace(n_images, n_per_image, dev, ctypes.byref(out)), ext)
        hit = _ws_cache[key] = int(out.value)
    return hit


def _ssim_workspace(ext: _Native, h: int, w: int, k: int) -> int:
    key = ("ssim", h, w, k)
    hit = _ws_cache.get(key)
    if hit is None:
        out = ctypes.c_int(0)
        _check(ext.gpu.fa_gpu_ssim_workspace(h, w, k, ctypes.byref(out)), ext)
        hit = _ws_cache[key] = int(out.value)
    return hit


def _gmsd_workspace(ext: _Native, h: int, w: int, downsample: bool) -> int:
    key = ("gmsd", h, w, bool(downsample))
    hit = _ws_cache.get(key)
    if hit is None:
        out = ctypes.c_int(0)
        _check(ext.gpu.fa_gpu_gmsd_workspace(h, w, int(downsample), ctypes.byref(out)), ext)
        hit = _ws_cache[key] = int(out.value)
    return hit


# --------------------------------------------------------------------------- #
# pixel losses
# --------------------------------------------------------------------------- #


def pixel_gpu(ext: _Native, x: torch.Tensor, y: torch.Tensor, *, op: int,
              param: float, per_image: bool, psnr_bias: float,
              luma: Optional[tuple] = None) -> torch.Tensor:
    """One fused reduction; exactly one output tensor is allocated.  Strided
    (cropped) views and ``luma`` = (kr, kg, kb, offset) go through
    ``fa_gpu_pixel_reduce_ex``, which reads them in place."""
    n, c, h, w = (int(v) for v in x.shape)
    x, xs = _view_strides(x)
    y, ys = _view_strides(y)
    per = c * h * w
    dev = _dev(x)
    bpi = _pixel_workspace(ext, n, per, dev)
    partial = _f64(x.device, n, bpi)
    want_psnr = psnr_bias != _PSNR_NONE
    out = _f64(x.device, n) if per_image else _f64(x.device)
    sinks: list = [None, None, None, None]
    sinks[(2 if want_psnr else 0) + (0 if per_image else 1)] = out
    if luma is None and xs is None and ys is None:
        _check(ext.gpu.fa_gpu_pixel_reduce(
            _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, per, op, float(param),
            float(psnr_bias), _ptr(partial), bpi,
            _ptr(sinks[0]), _ptr(sinks[1]), _ptr(sinks[2]), _ptr(sinks[3]),
            dev, _stream(x)), ext)
    else:
        _check(ext.gpu.fa_gpu_pixel_reduce_ex(
            _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w, xs, ys, _luma_arg(luma),
            op, float(param), float(psnr_bias), _ptr(partial), bpi,
            _ptr(sinks[0]), _ptr(sinks[1]), _ptr(sinks[2]), _ptr(sinks[3]),
            dev, _stream(x)), ext)
    return out


def pixel_cpu(lib: Any, x: torch.Tensor, y: torch.Tensor, *, op: int, param: float,
              per_image: bool, psnr_bias: float) -> torch.Tensor:
    """One host reduction (``fa_cpu_pixel_reduce``) over contiguous copies."""
    x, y = _contig(x), _contig(y)
    n = int(x.shape[0])
    out = torch.empty((n,) if per_image else (), dtype=torch.float64)
    _check_cpu(lib.fa_cpu_pixel_reduce(
        _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, x.numel() // n, op, float(param),
        float(psnr_bias), int(per_image), _ptr(out)))
    return out


def try_mse(x: torch.Tensor, y: torch.Tensor, *, per_image: bool,
            dtype: torch.dtype, psnr_bias: Optional[float] = None,
            luma: Optional[tuple] = None) -> Optional[torch.Tensor]:
    """Squared-error reduction, or PSNR when ``psnr_bias`` (= 10 log10 L^2) is given."""
    if not x.is_cuda:
        lib = _cpu_ready(x, y) if luma is None else None
        if lib is None:
            return None
        bias = psnr_bias if psnr_bias is not None else _PSNR_NONE
        out = pixel_cpu(lib, x, y, op=_OP_MSE, param=0.0, per_image=per_image, psnr_bias=bias)
        return out if dtype == torch.float64 else out.to(dtype)
    ext = _gpu_ext(x)
    if ext is None or not _usable(x, y) or x.dim() != 4 or x.shape != y.shape:
        return None
    if luma is not None and x.shape[1] != 3:
        return None
    bias = psnr_bias if psnr_bias is not None else _PSNR_NONE
    out = pixel_gpu(ext, x, y, op=_OP_MSE, param=0.0, per_image=per_image, psnr_bias=bias,
                    luma=luma)
    return out if dtype == torch.float64 else out.to(dtype)


def try_pixel(x: torch.Tensor, y: torch.Tensor, *, op: int, param: float,
              per_image: bool, dtype: torch.dtype,
              luma: Optional[tuple] = None) -> Optional[torch.Tensor]:
    """L1 / Charbonnier / Huber reduction; ``None`` if no kernel applies."""
    if not x.is_cuda:
        lib = _cpu_ready(x, y) if luma is None else None
        if lib is None:
            return None
        out = pixel_cpu(lib, x, y, op=op, param=param, per_image=per_image,
                        psnr_bias=_PSNR_NONE)
        return out if dtype == torch.float64 else out.to(dtype)
    ext = _gpu_ext(x)
    if ext is None or not _usable(x, y) or x.dim() != 4 or x.shape != y.shape:
        return None
    if luma is not None and x.shape[1] != 3:
        return None
    out = pixel_gpu(ext, x, y, op=op, param=param, per_image=per_image,
                    psnr_bias=_PSNR_NONE, luma=luma)
    return out if dtype == torch.float64 else out.to(dtype)


# --------------------------------------------------------------------------- #
# SSIM
# --------------------------------------------------------------------------- #


def ssim_autograd_available(x: torch.Tensor, y: torch.Tensor, win_size: int) -> bool:
    """Can the differentiable native SSIM path serve this call?"""
    return (
        x.is_cuda
        and x.dtype == torch.float32
        and y.dtype == torch.float32
        and x.shape == y.shape
        and x.dim() == 4
        and win_size in _WINDOWS
        and not torch.cuda.is_current_stream_capturing()
        and _gpu_ext(x) is not None
    )


def ssim_cs_autograd_available(x: torch.Tensor, y: torch.Tensor, win_size: int) -> bool:
    """Can the differentiable native MS-SSIM primitive serve this call?  float32
    levels and the float64 levels of the exact pyramid both can."""
    return (
        x.is_cuda
        and x.dtype in (torch.float32, torch.float64)
        and y.dtype == x.dtype
        and x.shape == y.shape
        and x.dim() == 4
        and win_size in _WINDOWS
        and not torch.cuda.is_current_stream_capturing()
        and _gpu_ext(x) is not None
    )


def ssim_fused(x: torch.Tensor, y: torch.Tensor, win: torch.Tensor,
               shift: float, C1: float, C2: float, want_map: bool):
    """Forward half of the differentiable SSIM: ``[per_image, total(, map)]``."""
    ext = load()
    x, y = _contig(x), _contig(y)
    winf = _win_f32(win)
    n, c, h, w = x.shape
    k = int(winf.numel())
    bpp = _ssim_workspace(ext, h, w, k)
    partial = _f64(x.device, n * c, bpp)
    per_image = _f64(x.device, n)
    total = _f64(x.device)
    smap = (torch.empty((n, c, h - k + 1, w - k + 1), device=x.device, dtype=torch.float32)
            if want_map else None)
    _check(ext.gpu.fa_gpu_ssim(
        _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w, _ptr(winf), k,
        float(shift), float(C1), float(C2), _ptr(smap), _ptr(partial), bpp,
        _ptr(per_image), _ptr(total), _dev(x), _stream(x)), ext)
    return [per_image, total, smap] if want_map else [per_image, total]


def ssim_backward(x, y, dL_dmap, grad_scalar, win, shift, C1, C2, need_dx, need_dy):
    ext = load()
    x, y = _contig(x), _contig(y)
    winf = _win_f32(win)
    n, c, h, w = x.shape
    k = int(winf.numel())
    hout, wout = h - k + 1, w - k + 1
    has_map = dL_dmap is not None and dL_dmap.numel() > 0
    dmap = dL_dmap.to(torch.float32).contiguous() if has_map else None
    gscalar = None if has_map else grad_scalar.to(torch.float32).contiguous().reshape(1)
    aux = torch.empty((4 if need_dy else 3, n * c, hout, wout), device=x.device,
                      dtype=torch.float32)
    dx = torch.empty_like(x) if need_dx else None
    dy = torch.empty_like(y) if need_dy else None
    _check(ext.gpu.fa_gpu_ssim_backward(
        _ptr(x), _ptr(y), _ptr(dmap), _ptr(gscalar), _ptr(winf), k, n, c, h, w,
        float(shift), float(C1), float(C2), _ptr(aux), _ptr(dx), _ptr(dy),
        _dev(x), _stream(x)), ext)
    return dx, dy


def _ssim_cpu(lib: Any, x, y, win_size, sigma, shift, C1, C2, reduction, return_map, dtype):
    from .functional import gaussian_window_1d

    x, y = _contig(x), _contig(y)
    n, c, h, w = (int(v) for v in x.shape)
    hout, wout = h - win_size + 1, w - win_size + 1
    win = gaussian_window_1d(win_size, sigma, device=x.device, dtype=torch.float32).contiguous()
    per_plane = torch.empty((n * c,), dtype=torch.float64)
    smap = torch.empty((n, c, hout, wout), dtype=torch.float32) if return_map else None
    _check_cpu(lib.fa_cpu_ssim(
        _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w, _ptr(win), win_size,
        float(shift), float(C1), float(C2), _ptr(smap), _ptr(per_plane)))
    if return_map:
        return smap if dtype == torch.float32 else smap.to(dtype)
    per_image = per_plane.view(n, c).sum(dim=1) / float(hout * wout * c)
    return per_image if reduction == "none" else per_image.mean()


def try_ssim(x: torch.Tensor, y: torch.Tensor, *, win_size: int, sigma: float,
             shift: float, C1: float, C2: float, reduction: str,
             return_map: bool, dtype: torch.dtype,
             luma: Optional[tuple] = None) -> Optional[torch.Tensor]:
    """SSIM on the GPU; ``None`` when the native path does not apply.

    Float64 input runs a float64 kernel.  A float64 *map* still takes the
    portable path, because the C ABI's map buffer is float32.  ``luma`` =
    (kr, kg, kb, offset) has the kernel form the luma plane of three-channel
    input itself; cropped views are read in place (``fa_gpu_ssim_ex``).
    CPU tensors run ``fa_cpu_ssim`` (float32 arithmetic, float64 for float64
    input), without luma or in-place crops.
    """
    if dtype == torch.float64 and (x.dtype != torch.float64 or return_map):
        return None
    if not x.is_cuda:
        lib = _cpu_ready(x, y) if luma is None and win_size in _WINDOWS else None
        if lib is None or x.shape[-2] < win_size or x.shape[-1] < win_size:
            return None
        return _ssim_cpu(lib, x, y, win_size, sigma, shift, C1, C2, reduction, return_map,
                         dtype)
    ext = _gpu_ext(x)
    if ext is None or not _usable(x, y) or win_size not in _WINDOWS:
        return None
    n, c = int(x.shape[0]), int(x.shape[1])
    if luma is not None and c != 3:
        return None
    from .functional import gaussian_window_1d

    win = _win_f32(gaussian_window_1d(win_size, sigma, device=x.device, dtype=torch.float32))
    h, w = int(x.shape[-2]), int(x.shape[-1])
    hout, wout = h - win_size + 1, w - win_size + 1
    x, xs = _view_strides(x)
    y, ys = _view_strides(y)
    cout = 1 if luma is not None else c
    bpp = _ssim_workspace(ext, h, w, win_size)
    partial = _f64(x.device, n * cout, bpp)
    smap = per_image = total = None
    if return_map:
        smap = torch.empty((n, cout, hout, wout), device=x.device, dtype=torch.float32)
    elif reduction == "none":
        per_image = _f64(x.device, n)
    else:
        total = _f64(x.device)
    if luma is None and xs is None and ys is None:
        _check(ext.gpu.fa_gpu_ssim(
            _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w, _ptr(win), win_size,
            float(shift), float(C1), float(C2), _ptr(smap), _ptr(partial), bpp,
            _ptr(per_image), _ptr(total), _dev(x), _stream(x)), ext)
    else:
        _check(ext.gpu.fa_gpu_ssim_ex(
            _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w, xs, ys, _luma_arg(luma),
            _ptr(win), win_size, float(shift), float(C1), float(C2), _ptr(smap),
            _ptr(partial), bpp, _ptr(per_image), _ptr(total), _dev(x), _stream(x)), ext)
    if return_map:
        return smap if dtype == torch.float32 else smap.to(dtype)
    return per_image if reduction == "none" else total


# --------------------------------------------------------------------------- #
# MS-SSIM's per-scale primitive
# --------------------------------------------------------------------------- #


def pyramid_dtype(dt: torch.dtype) -> torch.dtype:
    """Element type of the MS-SSIM pyramid levels below an input of type ``dt``:
    float32 holds the 2x2 means of uint8 levels exactly at every depth (a level
    k value is a multiple of 4^-k below 256), float64 those of every floating
    type."""
    return torch.float32 if dt == torch.uint8 else torch.float64


def _ssim_cs_gpu(ext: _Native, x, y, winf, shift, C1, C2, pool_dtype=None, luma=None):
    """``(s, cs)`` plane means, plus the next pyramid level ``(px, py)`` of
    ``pool_dtype`` when one is asked for (one fused pass).  x / y may be
    strided views; ``luma`` = (kr, kg, kb, offset) makes each image one plane."""
    n, c, h, w = x.shape
    k = int(winf.numel())
    cout = 1 if luma is not None else c
    planes = n * cout
    x, xs = _view_strides(x)
    y, ys = _view_strides(y)
    bpp = _ssim_workspace(ext, h, w, k)
    partial = _f64(x.device, planes, bpp)
    partial_cs = _f64(x.device, planes, bpp)
    out_s = _f64(x.device, planes)
    out_cs = _f64(x.device, planes)
    if pool_dtype is None and luma is None and xs is None and ys is None:
        _check(ext.gpu.fa_gpu_ssim_cs(
            _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w, _ptr(winf), k,
            float(shift), float(C1), float(C2), _ptr(partial), _ptr(partial_cs),
            bpp, _ptr(out_s), _ptr(out_cs), _dev(x), _stream(x)), ext)
        return out_s, out_cs
    px = py = None
    if pool_dtype is not None:
        px = torch.empty((n, cout, h // 2, w // 2), dtype=pool_dtype, device=x.device)
        py = torch.empty_like(px)
    pcode = _DTYPE_CODE[pool_dtype if pool_dtype is not None else torch.float64]
    _check(ext.gpu.fa_gpu_ssim_cs_ex(
        _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w, xs, ys, _luma_arg(luma),
        _ptr(winf), k, float(shift), float(C1), float(C2), _ptr(partial), _ptr(partial_cs),
        bpp, _ptr(out_s), _ptr(out_cs), None, _ptr(px), _ptr(py), pcode, _dev(x),
        _stream(x)), ext)
    return (out_s, out_cs) if pool_dtype is None else (out_s, out_cs, px, py)


def ssim_cs_partials(x, y, win, shift, C1, C2, pool_dtype, luma=None, u8_pyramid=False):
    """One inference MS-SSIM scale left unreduced: ``(partial, partial_cs,
    slots, npix, px, py)`` -- the per-plane partial sums of the SSIM and cs
    maps (``slots`` per plane, packed), the plane's output pixel count, and the
    next pyramid level (``None`` at the coarsest scale).  The partial sums go
    to :func:`ms_ssim_reduce`; nothing is synchronised.  ``u8_pyramid``: x and
    y are float32 levels of a uint8 pyramid (FA_DTYPE_U8_PYRAMID)."""
    ext = load()
    winf = _win_f32(win)
    n, c, h, w = x.shape
    k = int(winf.numel())
    cout = 1 if luma is not None else c
    x, xs = _view_strides(x)
    y, ys = _view_strides(y)
    bpp = _ssim_workspace(ext, h, w, k)
    partial = _f64(x.device, n * cout, bpp)
    partial_cs = _f64(x.device, n * cout, bpp)
    px = py = None
    if pool_dtype is not None:
        px = torch.empty((n, cout, h // 2, w // 2), dtype=pool_dtype, device=x.device)
        py = torch.empty_like(px)
    pcode = _DTYPE_CODE[pool_dtype if pool_dtype is not None else torch.float64]
    slots = ctypes.c_int(0)
    code = _DTYPE_CODE[x.dtype]
    if u8_pyramid:
        if x.dtype != torch.float32 or luma is not None:
            raise ValueError("u8_pyramid needs float32 levels without luma")
        code |= FA_DTYPE_U8_PYRAMID
    _check(ext.gpu.fa_gpu_ssim_cs_ex(
        _ptr(x), _ptr(y), code, n, c, h, w, xs, ys, _luma_arg(luma),
        _ptr(winf), k, float(shift), float(C1), float(C2), _ptr(partial), _ptr(partial_cs),
        bpp, None, None, ctypes.byref(slots), _ptr(px), _ptr(py), pcode, _dev(x),
        _stream(x)), ext)
    npix = float((h - k + 1) * (w - k + 1))
    return partial, partial_cs, int(slots.value), npix, px, py


def ssim_cs_forward(x, y, win, shift, C1, C2, pool_dtype=None):
    """``(ssim, cs)`` plane means from the differentiable native path, plus the
    next pyramid level when ``pool_dtype`` is given."""
    ext = load()
    return _ssim_cs_gpu(ext, _contig(x), _contig(y), _win_f32(win), shift, C1, C2,
                        pool_dtype)


def ssim_cs_backward(x, y, gs, gcs, win, shift, C1, C2, need_dx, need_dy,
                     gpx=None, gpy=None):
    """Gradients of the plane means (and of the pyramid level the forward
    pooled, ``gpx`` / ``gpy``) with respect to x and y."""
    ext = load()
    x, y = _contig(x), _contig(y)
    winf = _win_f32(win)
    n, c, h, w = x.shape
    k = int(winf.numel())
    hout, wout = h - k + 1, w - k + 1
    gsf = gs.to(torch.float32).contiguous().reshape(-1)
    gcsf = gcs.to(torch.float32).contiguous().reshape(-1)
    aux = torch.empty((4 if need_dy else 3, n * c, hout, wout), device=x.device,
                      dtype=torch.float32)
    dx = torch.empty_like(x) if need_dx else None
    dy = torch.empty_like(y) if need_dy else None
    gpx = _contig(gpx) if (gpx is not None and need_dx) else None
    gpy = _contig(gpy) if (gpy is not None and need_dy) else None
    if x.dtype == torch.float32 and gpx is None and gpy is None:
        _check(ext.gpu.fa_gpu_ssim_cs_backward(
            _ptr(x), _ptr(y), _ptr(gsf), _ptr(gcsf), _ptr(winf), k, n, c, h, w,
            float(shift), float(C1), float(C2), _ptr(aux), _ptr(dx), _ptr(dy),
            _dev(x), _stream(x)), ext)
    else:
        gp = gpx if gpx is not None else gpy
        gp_code = _DTYPE_CODE[gp.dtype] if gp is not None else _DTYPE_CODE[torch.float64]
        if gpx is not None and gpy is not None and gpx.dtype != gpy.dtype:
            gpy = gpy.to(gpx.dtype)
        _check(ext.gpu.fa_gpu_ssim_cs_backward_ex(
            _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], _ptr(gsf), _ptr(gcsf), _ptr(winf), k,
            n, c, h, w, float(shift), float(C1), float(C2), _ptr(gpx), _ptr(gpy), gp_code,
            _ptr(aux), _ptr(dx), _ptr(dy), _dev(x), _stream(x)), ext)
    return dx, dy


def ssim_cs_pool_available(x: torch.Tensor, y: torch.Tensor, win_size: int) -> bool:
    """Can the native MS-SSIM scale step (CS means + fused pyramid) serve x, y?"""
    return (x.is_cuda and x.dim() == 4 and x.dtype in _SUPPORTED and y.dtype == x.dtype
            and x.shape == y.shape and win_size in _WINDOWS
            and x.shape[-2] >= win_size and x.shape[-1] >= win_size
            and x.stride(-1) == 1 and y.stride(-1) == 1
            and _gpu_ext(x) is not None)


def ssim_cs_pool(x, y, win, shift, C1, C2, pool_dtype, luma=None):
    """Inference form of one MS-SSIM scale: ``(s, cs, px, py)``, or ``(s, cs)``
    when ``pool_dtype`` is None (the coarsest scale).  Views are read in place;
    ``luma`` forms the luma plane of three-channel input in the kernel."""
    ext = load()
    return _ssim_cs_gpu(ext, x, y, _win_f32(win), shift, C1, C2, pool_dtype, luma)


def try_ssim_cs(x: torch.Tensor, y: torch.Tensor, *, win: torch.Tensor,
                shift: float, C1: float, C2: float):
    """``(ssim, cs)`` per plane, shaped ``(N, C)``; ``None`` if unavailable."""
    k = int(win.numel())
    if not x.is_cuda:
        lib = _cpu_ready(x, y) if k in _WINDOWS else None
        if lib is None or x.shape[-2] < k or x.shape[-1] < k:
            return None
        x, y = _contig(x), _contig(y)
        n, c, h, w = (int(v) for v in x.shape)
        winf = win.to(torch.float32).contiguous()
        s = torch.empty((n * c,), dtype=torch.float64)
        cs = torch.empty((n * c,), dtype=torch.float64)
        _check_cpu(lib.fa_cpu_ssim_cs(
            _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w, _ptr(winf), k,
            float(shift), float(C1), float(C2), _ptr(s), _ptr(cs)))
        return s.view(n, c), cs.view(n, c)
    ext = _gpu_ext(x)
    if ext is None or not _usable(x, y):
        return None
    if k not in _WINDOWS or x.shape[-2] < k or x.shape[-1] < k:
        return None
    n, c = int(x.shape[0]), int(x.shape[1])
    s, cs = _ssim_cs_gpu(ext, _contig(x), _contig(y), _win_f32(win), shift, C1, C2)
    return s.view(n, c), cs.view(n, c)


# --------------------------------------------------------------------------- #
# GMSD
# --------------------------------------------------------------------------- #


def try_gmsd(x: torch.Tensor, y: torch.Tensor, *, T: float, eps: float, downsample: bool,
             luma: Optional[tuple] = None, want_map: bool = False):
    """``(gms_mean, gmsd)`` per image, float64 -- plus the float32 q map when
    ``want_map`` -- or ``None`` if unavailable.

    ``luma`` = (kr, kg, kb[, offset]) makes the kernel read the three channels
    and form the luma plane itself; cropped views are read in place through
    their strides (``fa_gpu_gmsd_ex``).  CPU tensors run ``fa_cpu_gmsd``
    (statistics only: no luma, no map).
    """
    if not x.is_cuda:
        lib = _cpu_ready(x, y) if luma is None and not want_map else None
        if lib is None:
            return None
        x, y = _contig(x), _contig(y)
        n, c, h, w = (int(v) for v in x.shape)
        hd, wd = (h // 2, w // 2) if downsample else (h, w)
        if hd < 3 or wd < 3:
            return None
        mean = torch.empty((n,), dtype=torch.float64)
        dev = torch.empty((n,), dtype=torch.float64)
        _check_cpu(lib.fa_cpu_gmsd(
            _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w, float(T), float(eps),
            int(downsample), _ptr(mean), _ptr(dev)))
        return mean, dev
    ext = _gpu_ext(x)
    if ext is None or not _usable(x, y):
        return None
    n, c = int(x.shape[0]), int(x.shape[1])
    h, w = int(x.shape[-2]), int(x.shape[-1])
    if luma is not None and c != 3:
        return None
    x, xs = _view_strides(x)
    y, ys = _view_strides(y)
    cout = 1 if luma is not None else c
    planes = n * cout
    bpp = _gmsd_workspace(ext, h, w, downsample)
    psum = _f64(x.device, planes, bpp)
    psumsq = _f64(x.device, planes, bpp)
    mean = _f64(x.device, n)
    dev = _f64(x.device, n)
    qmap = None
    if want_map:
        hd, wd = (h // 2, w // 2) if downsample else (h, w)
        qmap = torch.empty((n, cout, hd - 2, wd - 2), dtype=torch.float32, device=x.device)
    if luma is None and xs is None and ys is None and qmap is None:
        _check(ext.gpu.fa_gpu_gmsd(
            _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w, float(T), float(eps),
            int(downsample), _ptr(psum), _ptr(psumsq), bpp, _ptr(mean), _ptr(dev),
            _dev(x), _stream(x)), ext)
    else:
        _check(ext.gpu.fa_gpu_gmsd_ex(
            _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w, xs, ys, _luma_arg(luma),
            float(T), float(eps), int(downsample), _ptr(qmap), _ptr(psum), _ptr(psumsq), bpp,
            _ptr(mean), _ptr(dev), _dev(x), _stream(x)), ext)
    return (mean, dev, qmap) if want_map else (mean, dev)


def gmsd_autograd_available(x: torch.Tensor, y: torch.Tensor) -> bool:
    """Can the differentiable native GMS / GMSD path serve this call?"""
    return (x.is_cuda and x.dim() == 4 and x.dtype in (torch.float32, torch.float64)
            and y.dtype == x.dtype and x.shape == y.shape
            and not torch.cuda.is_current_stream_capturing() and _gpu_ext(x) is not None)


def gmsd_stats_fwd(x, y, T, eps, downsample):
    """Forward half of the differentiable GMS / GMSD: ``(mean, std)`` per image."""
    ext = load()
    x, y = _contig(x), _contig(y)
    n, c, h, w = x.shape
    bpp = _gmsd_workspace(ext, h, w, downsample)
    psum = _f64(x.device, n * c, bpp)
    psumsq = _f64(x.device, n * c, bpp)
    mean = _f64(x.device, n)
    dev = _f64(x.device, n)
    _check(ext.gpu.fa_gpu_gmsd(
        _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w, float(T), float(eps),
        int(downsample), _ptr(psum), _ptr(psumsq), bpp, _ptr(mean), _ptr(dev),
        _dev(x), _stream(x)), ext)
    return mean, dev


def gmsd_stats_bwd(x, y, mean, std, g_mean, g_std, T, eps, downsample, need_dx, need_dy):
    ext = load()
    x, y = _contig(x), _contig(y)
    n, c, h, w = x.shape
    hd, wd = (h // 2, w // 2) if downsample else (h, w)
    aux = torch.empty((4, n * c, hd - 2, wd - 2), dtype=torch.float64, device=x.device)
    gm = g_mean.to(torch.float64).contiguous() if g_mean is not None else None
    gs = g_std.to(torch.float64).contiguous() if g_std is not None else None
    dx = torch.empty_like(x) if need_dx else None
    dy = torch.empty_like(y) if need_dy else None
    _check(ext.gpu.fa_gpu_gmsd_backward(
        _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w, float(T), float(eps),
        int(downsample), _ptr(mean), _ptr(std), _ptr(gm), _ptr(gs), _ptr(aux), _ptr(dx),
        _ptr(dy), _dev(x), _stream(x)), ext)
    return dx, dy


def ms_ssim_reduce(partials, slots, npix, weights, n: int, c: int, per_image: bool):
    """MS-SSIM's per-scale plane reductions, clamp / power / product and the
    channel and batch means in two launches (``fa_gpu_ms_ssim_reduce``) from
    the partial sums of :func:`ssim_cs_partials`."""
    ext = load()
    dev = partials[0].device
    m = len(partials)
    arr = (ctypes.c_void_p * m)(*[t.data_ptr() for t in partials])
    sl = (ctypes.c_int * m)(*[int(v) for v in slots])
    npx = (ctypes.c_double * m)(*[float(v) for v in npix])
    w = (ctypes.c_double * m)(*[float(v) for v in weights])
    scratch = _f64(dev, m * n * c)
    out = _f64(dev, n) if per_image else _f64(dev)
    _check(ext.gpu.fa_gpu_ms_ssim_reduce(
        arr, sl, npx, w, m, n, c, _ptr(scratch), _ptr(out) if per_image else None,
        None if per_image else _ptr(out), _dev(partials[0]), _stream(partials[0])), ext)
    return out