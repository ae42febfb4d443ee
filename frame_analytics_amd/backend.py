"""Dispatch to the gfx950 kernels: tensors in, raw pointers across the C ABI.

Counterpart of the reference's ``frame_analytics/backend.py``.  Shapes and
dtypes become ints, tensors become device pointers, and every buffer the
kernels write -- scratch included -- is allocated here through torch's caching
allocator, so no call ever allocates inside the library and every call stays
legal inside a HIP graph capture (reference backend.py:145-153).

Failure policy:

* on a machine with a GPU the kernel library must load; if it cannot, the
  first call raises (the reference would quietly run PyTorch instead).
  ``FA_NATIVE=0`` is the explicit opt-out.
* a kernel that declines an inference call (a non-zero status, raised as
  :class:`KernelError`) makes its ``try_*`` warn once per distinct message
  and return ``None``, so the call takes the portable path -- the reference's
  behaviour (backend.py:213-224).  The differentiable entry points
  (``ssim_fused``, ``ssim_cs_forward``, the backward passes) raise instead,
  as the reference's do.
* ``try_*`` also return ``None`` where the native path does not apply to the
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

import contextlib
import ctypes
import functools
import os
import threading
import warnings
from collections import Counter
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


# --------------------------------------------------------------------------- #
# calling into libfa_gpu.so
# --------------------------------------------------------------------------- #

#: entry point name -> calls made through :func:`call_gpu` in this process.
#: Tests read it to show that a GPU call was served by the gfx950 kernels.
native_calls: Counter = Counter()
#: functional helper -> evaluations of the portable PyTorch path on GPU tensors
portable_calls: Counter = Counter()


def note_portable(what: str, t: torch.Tensor) -> None:
    """Record that the portable path computed ``what`` on a GPU tensor."""
    if t.is_cuda:
        portable_calls[what] += 1


def call_gpu(name: str, *args) -> int:
    """Call one entry point of ``include/fa_abi.h`` and return its status.

    Every GPU launch of this package goes through here, so
    :data:`native_calls` counts them."""
    ext = load()
    if ext is None or not ext.has_gpu:
        raise RuntimeError(f"{name}: the gfx950 kernel library is not loaded")
    code = getattr(ext.gpu, name)(*args)
    native_calls[name] += 1
    return int(code)


_FA_E_ARG = 5  # include/fa_abi.h: a refusal made before anything was launched


def _run_or_needs_workspace(name: str, args_without, args_with, acc=None) -> None:
    """Call a one-launch entry point without its workspace first (it is not
    read where the call finishes in its launch); when the library answers
    FA_E_ARG -- it refuses before launching anything -- call it again with the
    workspace that ``args_with()`` allocates.  Any other failure raises, and
    drops the stream's accumulator ``acc`` (:func:`_forget_acc`)."""
    code = call_gpu(name, *args_without)
    if code == 0:
        return
    if code == _FA_E_ARG:
        code = call_gpu(name, *args_with())
        if code == 0:
            return
    _forget_acc(acc)
    raise KernelError(f"{name}: " + status_text(code, _ext.gpu if _ext else None))


def _run_acc(name: str, acc, *args) -> None:
    """:func:`_run` for a call handed the stream's accumulator ``acc``: a
    failure drops it (:func:`_forget_acc`) before raising."""
    code = call_gpu(name, *args)
    if code:
        _forget_acc(acc)
        raise KernelError(f"{name}: " + status_text(code, _ext.gpu if _ext else None))


def _run(name: str, *args) -> None:
    """:func:`call_gpu`, raising :class:`KernelError` on a non-zero status."""
    code = call_gpu(name, *args)
    if code:
        raise KernelError(f"{name}: " + status_text(code, _ext.gpu if _ext else None))


_declined_seen: set = set()


def _declined(exc: KernelError) -> None:
    """Warn (once per distinct message) that a kernel refused a call, which
    then takes the portable path."""
    key = str(exc)
    if key in _declined_seen:
        return
    _declined_seen.add(key)
    warnings.warn(f"frame_analytics_amd: a native kernel declined this call ({key}); "
                  "computing it with the portable PyTorch path", RuntimeWarning, stacklevel=3)


def _site(t: torch.Tensor):
    """``(device ordinal, hipStream_t)`` of the caller's current stream on the
    device of ``t``: kernels are enqueued where torch would enqueue its own.
    The raw handle comes straight from torch's C layer: building a
    ``torch.cuda.Stream`` object per call costs ~3 us of host time, which is
    a tenth of a short call such as configs[4] GMSD."""
    idx = t.get_device()
    return idx, torch._C._cuda_getCurrentRawStream(idx)


def _win32(win: torch.Tensor) -> torch.Tensor:
    """The window as the ABI takes it: contiguous float32.  The functional
    layer hands over its cached float32 windows, so this is a no-op there."""
    if win.dtype != torch.float32:
        win = win.to(torch.float32)
    return _contig(win)


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


_WORKSPACE_QUERY = {
    "pixel": "fa_gpu_pixel_workspace",  # (n_images, n_per_image, device)
    "ssim": "fa_gpu_ssim_workspace",    # (H, W, K)
    "gmsd": "fa_gpu_gmsd_workspace",    # (H, W, downsample)
}


@functools.lru_cache(maxsize=None)
def workspace_slots(kind: str, a: int, b: int, c: int) -> int:
    """Partial-sum slots per image (``"pixel"``) or per plane (``"ssim"``,
    ``"gmsd"``) a launch of this shape needs; the arguments follow the
    entry point's.  The answer depends on the shape only, so each shape is
    asked once and a graph capture never issues the query (reference
    backend.py:247-286 keeps the same property)."""
    out = ctypes.c_int(0)
    _run(_WORKSPACE_QUERY[kind], int(a), int(b), int(c), ctypes.byref(out))
    return int(out.value)


# --------------------------------------------------------------------------- #
# pixel losses
# --------------------------------------------------------------------------- #


#: uint64 words of the one-launch entry points' accumulators
#: (FA_PIXEL_ACC_WORDS, FA_GMSD_ACC_WORDS, FA_SSIM_ACC_WORDS, FA_MS_SSIM_ACC_WORDS)
_ACC_WORDS = {"pixel": (32 + 1) * 16, "gmsd": (3 * 64 + 2) * 16, "ssim": (256 + 1) * 16,
              "ms": (8 * 256 + 1) * 16}
#: (kind, device, raw stream) -> that stream's accumulator, zero between calls
_stream_acc: dict = {}
#: per thread: (kind, device) -> accumulator of one HIP graph's calls alone
#: (see private_accumulators); unset outside such a scope
_private = threading.local()


@contextlib.contextmanager
def private_accumulators(store: dict):
    """Within this scope the one-launch entry points take their accumulators
    from ``store`` (made on first use, outside capture), in graph capture
    too.  For a graph whose replays share those buffers with nothing else
    (``StreamingMetrics``: its warm-up and its capture run in this scope, and
    then only its replays use them), so the captured calls can finish in their
    one launch; each replay leaves them zero, like an eager call.  The scope
    is the calling thread's: calls from other threads keep their streams'
    shared accumulators."""
    prev = getattr(_private, "store", None)
    _private.store = store
    try:
        yield store
    finally:
        _private.store = prev


def _acc_for(kind: str, device: torch.device, dev: int, stream: int) -> Optional[torch.Tensor]:
    """The zeroed accumulator that lets a reduction finish inside its one
    launch (``fa_gpu_pixel_reduce_once``, ``fa_gpu_gmsd_once``,
    ``fa_gpu_ssim_once``, ``fa_gpu_ms_ssim``).  Each call
    leaves it zero again, so one buffer serves every call on its stream, in
    stream order; calls on another stream get their own.  Under graph capture
    there is none (the call takes its two-launch form): a graph's replays
    could overlap eager calls of the stream that recorded it -- unless the
    capture runs in :func:`private_accumulators`, whose buffers are the
    graph's alone."""
    capturing = torch._C._cuda_isCurrentStreamCapturing()
    store = getattr(_private, "store", None)
    if store is not None:
        acc = store.get((kind, dev))
        if acc is None and not capturing:
            acc = torch.zeros(_ACC_WORDS[kind], dtype=torch.int64, device=device)
            store[(kind, dev)] = acc
        return acc
    if capturing:
        return None
    key = (kind, dev, stream)
    acc = _stream_acc.get(key)
    if acc is None:
        acc = torch.zeros(_ACC_WORDS[kind], dtype=torch.int64, device=device)
        _stream_acc[key] = acc
    return acc


def _forget_acc(acc: Optional[torch.Tensor]) -> None:
    """Drop a stream's accumulator after a call that failed with it: a call
    that stopped between two of its launches (MS-SSIM makes three) can leave
    words of it non-zero, and every later call on the stream counts from zero.
    The next call allocates a new, zeroed one."""
    if acc is None:
        return
    for store in (_stream_acc, getattr(_private, "store", None) or {}):
        for key, t in list(store.items()):
            if t is acc:
                del store[key]


def pixel_gpu(ext: _Native, x: torch.Tensor, y: torch.Tensor, *, op: int,
              param: float, per_image: bool, psnr_bias: float,
              luma: Optional[tuple] = None) -> torch.Tensor:
    """One fused reduction; exactly one output tensor is allocated.  Strided
    (cropped) views and ``luma`` = (kr, kg, kb, offset) go through
    ``fa_gpu_pixel_reduce_ex``, which reads them in place."""
    del ext  # the library is reached through call_gpu
    n, c, h, w = (int(v) for v in x.shape)
    x, xs = _view_strides(x)
    y, ys = _view_strides(y)
    per = c * h * w
    dev, stream = _site(x)
    bpi = workspace_slots("pixel", n, per, dev)
    out = _f64(x.device, n) if per_image else _f64(x.device)
    # the four ABI sinks, in order: mean per image, mean total, dB per image,
    # dB total; exactly one is written
    slot = (2 if psnr_bias != _PSNR_NONE else 0) + (0 if per_image else 1)
    sinks = [_ptr(out) if i == slot else None for i in range(4)]
    if luma is None and xs is None and ys is None:
        acc = _acc_for("pixel", x.device, dev, stream) if x.dtype == torch.uint8 else None

        def args(partial):
            return (_ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, per, op, float(param),
                    float(psnr_bias), partial, bpi, _ptr(acc), *sinks, dev, stream)

        if acc is None:
            _run("fa_gpu_pixel_reduce_once", *args(_ptr(_f64(x.device, n, bpi))))
        else:
            _run_or_needs_workspace("fa_gpu_pixel_reduce_once", args(None),
                                    lambda: args(_ptr(_f64(x.device, n, bpi))), acc)
    else:
        partial = _f64(x.device, n, bpi)
        _run("fa_gpu_pixel_reduce_ex", _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w,
             xs, ys, _luma_arg(luma), op, float(param), float(psnr_bias), _ptr(partial), bpi,
             *sinks, dev, stream)
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
    return try_pixel(x, y, op=_OP_MSE, param=0.0, per_image=per_image, dtype=dtype,
                     luma=luma, psnr_bias=psnr_bias)


def try_pixel(x: torch.Tensor, y: torch.Tensor, *, op: int, param: float,
              per_image: bool, dtype: torch.dtype,
              luma: Optional[tuple] = None,
              psnr_bias: Optional[float] = None) -> Optional[torch.Tensor]:
    """MSE / L1 / Charbonnier / Huber reduction (PSNR with ``psnr_bias``);
    ``None`` if no kernel applies."""
    bias = _PSNR_NONE if psnr_bias is None else float(psnr_bias)
    try:
        if not x.is_cuda:
            lib = _cpu_ready(x, y) if luma is None else None
            if lib is None:
                return None
            out = pixel_cpu(lib, x, y, op=op, param=param, per_image=per_image, psnr_bias=bias)
        else:
            ext = _gpu_ext(x)
            if ext is None or not _usable(x, y) or x.dim() != 4 or x.shape != y.shape:
                return None
            if luma is not None and x.shape[1] != 3:
                return None
            out = pixel_gpu(ext, x, y, op=op, param=param, per_image=per_image,
                            psnr_bias=bias, luma=luma)
    except KernelError as exc:
        _declined(exc)
        return None
    return out if dtype == torch.float64 else out.to(dtype)


# --------------------------------------------------------------------------- #
# SSIM
# --------------------------------------------------------------------------- #


def _autograd_ok(x: torch.Tensor, y: torch.Tensor, dtypes) -> bool:
    return (x.is_cuda and x.dim() == 4 and x.dtype in dtypes and y.dtype == x.dtype
            and x.shape == y.shape and not torch.cuda.is_current_stream_capturing()
            and _gpu_ext(x) is not None)


def ssim_autograd_available(x: torch.Tensor, y: torch.Tensor, win_size: int) -> bool:
    """Can the differentiable native SSIM path serve this call?"""
    return win_size in _WINDOWS and _autograd_ok(x, y, (torch.float32,))


def ssim_cs_autograd_available(x: torch.Tensor, y: torch.Tensor, win_size: int) -> bool:
    """Can the differentiable native MS-SSIM primitive serve this call?  float32
    levels and the float64 levels of the exact pyramid both can."""
    return win_size in _WINDOWS and _autograd_ok(x, y, (torch.float32, torch.float64))


def ssim_fused(x: torch.Tensor, y: torch.Tensor, win: torch.Tensor,
               shift: float, C1: float, C2: float, want_map: bool):
    """Forward half of the differentiable SSIM: ``[per_image, total(, map)]``."""
    x, y, win = _contig(x), _contig(y), _win32(win)
    n, c, h, w = (int(v) for v in x.shape)
    k = int(win.numel())
    bpp = workspace_slots("ssim", h, w, k)
    dev, stream = _site(x)
    per_image, total = _f64(x.device, n), _f64(x.device)
    if not want_map:
        # the means finished in the forward's launch where it can (the stream's
        # accumulator; none under graph capture)
        acc = _acc_for("ssim", x.device, dev, stream)

        def args(partial):
            return (_ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w, None, None, None,
                    _ptr(win), k, float(shift), float(C1), float(C2), None, partial, bpp,
                    _ptr(acc), _ptr(per_image), _ptr(total), dev, stream)

        if acc is None:
            _run("fa_gpu_ssim_once", *args(_ptr(_f64(x.device, n * c, bpp))))
        else:
            _run_or_needs_workspace("fa_gpu_ssim_once", args(None),
                                    lambda: args(_ptr(_f64(x.device, n * c, bpp))), acc)
        return [per_image, total]
    partial = _f64(x.device, n * c, bpp)
    smap = torch.empty((n, c, h - k + 1, w - k + 1), device=x.device, dtype=torch.float32)
    _run("fa_gpu_ssim", _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w, _ptr(win), k,
         float(shift), float(C1), float(C2), _ptr(smap), _ptr(partial), bpp,
         _ptr(per_image), _ptr(total), dev, stream)
    return [per_image, total, smap]


def _grad_buffers(x, y, k, need_dx, need_dy):
    """The backward's float32 coefficient maps (3, or 4 with dy, per output
    pixel: the ABI's ``aux``) and its outputs."""
    n, c, h, w = (int(v) for v in x.shape)
    aux = torch.empty((4 if need_dy else 3, n * c, h - k + 1, w - k + 1), device=x.device,
                      dtype=torch.float32)
    return (aux, torch.empty_like(x) if need_dx else None,
            torch.empty_like(y) if need_dy else None)


def ssim_backward(x, y, dL_dmap, grad_scalar, win, shift, C1, C2, need_dx, need_dy):
    """dL/dx, dL/dy of the SSIM map (``dL_dmap``) or of the batch mean
    (``grad_scalar``, a 1-element device tensor read by the kernel)."""
    x, y, win = _contig(x), _contig(y), _win32(win)
    n, c, h, w = (int(v) for v in x.shape)
    k = int(win.numel())
    if dL_dmap is not None and dL_dmap.numel() > 0:
        dmap, gscalar = dL_dmap.to(torch.float32).contiguous(), None
    else:
        dmap, gscalar = None, grad_scalar.to(torch.float32).contiguous().reshape(1)
    aux, dx, dy = _grad_buffers(x, y, k, need_dx, need_dy)
    dev, stream = _site(x)
    _run("fa_gpu_ssim_backward", _ptr(x), _ptr(y), _ptr(dmap), _ptr(gscalar), _ptr(win), k,
         n, c, h, w, float(shift), float(C1), float(C2), _ptr(aux), _ptr(dx), _ptr(dy),
         dev, stream)
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
    """SSIM on the GPU (or the host library); ``None`` when the native path does
    not apply or a kernel declined the call (warned once)."""
    try:
        return _ssim_native(x, y, win_size=win_size, sigma=sigma, shift=shift, C1=C1, C2=C2,
                            reduction=reduction, return_map=return_map, dtype=dtype, luma=luma)
    except KernelError as exc:
        _declined(exc)
        return None


def _ssim_native(x: torch.Tensor, y: torch.Tensor, *, win_size: int, sigma: float,
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
    n, c, h, w = (int(v) for v in x.shape)
    if luma is not None and c != 3:
        return None
    from .functional import gaussian_window_1d

    win = gaussian_window_1d(win_size, sigma, device=x.device, dtype=torch.float32)
    x, xs = _view_strides(x)
    y, ys = _view_strides(y)
    planes = n * (1 if luma is not None else c)
    bpp = workspace_slots("ssim", h, w, win_size)
    dev, stream = _site(x)
    # one sink: the float32 map, the per-image means or the batch mean
    smap = per_image = total = None
    if return_map:
        smap = torch.empty((n, planes // n, h - win_size + 1, w - win_size + 1),
                           device=x.device, dtype=torch.float32)
    elif reduction == "none":
        per_image = _f64(x.device, n)
    else:
        total = _f64(x.device)
    head = (_ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w)

    def tail(partial):
        return (_ptr(win), win_size, float(shift), float(C1), float(C2), _ptr(smap), partial,
                bpp, _ptr(per_image), _ptr(total), dev, stream)

    if smap is None:
        acc = _acc_for("ssim", x.device, dev, stream)
        lw = _luma_arg(luma)

        def args(partial):
            t = tail(partial)
            return (*head, xs, ys, lw, *t[:8], _ptr(acc), *t[8:])

        if acc is None:
            _run("fa_gpu_ssim_once", *args(_ptr(_f64(x.device, planes, bpp))))
        else:
            _run_or_needs_workspace("fa_gpu_ssim_once", args(None),
                                    lambda: args(_ptr(_f64(x.device, planes, bpp))), acc)
        return per_image if reduction == "none" else total
    partial = _ptr(_f64(x.device, planes, bpp))
    if luma is None and xs is None and ys is None:
        _run("fa_gpu_ssim", *head, *tail(partial))
    else:
        _run("fa_gpu_ssim_ex", *head, xs, ys, _luma_arg(luma), *tail(partial))
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


def _cs_launch(x, y, win, shift, C1, C2, *, pool_dtype=None, luma=None, reduce=True,
               u8_pyramid=False, ssim_sums=True):
    """One CS pass (``fa_gpu_ssim_cs_ex``, or ``fa_gpu_ssim_cs`` for a plain
    contiguous call): the (ssim, cs) partial sums per plane, their plane means
    when ``reduce``, and the next pyramid level of ``pool_dtype`` if given.
    Without ``reduce`` and ``ssim_sums`` the pass forms the cs sums alone.

    Returns ``(s, cs, partial, partial_cs, slots, px, py)``; ``s``/``cs`` are
    ``None`` without ``reduce``, ``partial`` without the SSIM sums, and
    ``slots`` is what the launch reports (``-1`` when it was not asked)."""
    win = _win32(win)
    n, c, h, w = (int(v) for v in x.shape)
    k = int(win.numel())
    planes = n * (1 if luma is not None else c)
    x, xs = _view_strides(x)
    y, ys = _view_strides(y)
    bpp = workspace_slots("ssim", h, w, k)
    dev, stream = _site(x)
    partial = _f64(x.device, planes, bpp) if reduce or ssim_sums else None
    partial_cs = _f64(x.device, planes, bpp)
    s = cs = px = py = None
    if reduce:
        s, cs = _f64(x.device, planes), _f64(x.device, planes)
    if pool_dtype is not None:
        px = torch.empty((n, planes // n, h // 2, w // 2), dtype=pool_dtype, device=x.device)
        py = torch.empty_like(px)
    code = _DTYPE_CODE[x.dtype]
    if u8_pyramid:
        if x.dtype not in (torch.float32, torch.float16) or luma is not None:
            raise ValueError("u8_pyramid needs float32 (or first-level float16) levels "
                             "without luma")
        code |= FA_DTYPE_U8_PYRAMID
    head = (_ptr(x), _ptr(y), code, n, c, h, w)
    consts = (_ptr(win), k, float(shift), float(C1), float(C2), _ptr(partial),
              _ptr(partial_cs), bpp, _ptr(s), _ptr(cs))
    if (reduce and pool_dtype is None and luma is None and xs is None and ys is None
            and not u8_pyramid):
        _run("fa_gpu_ssim_cs", *head, *consts, dev, stream)
        return s, cs, partial, partial_cs, -1, None, None
    slots = ctypes.c_int(-1)
    pcode = _DTYPE_CODE[pool_dtype if pool_dtype is not None else torch.float64]
    _run("fa_gpu_ssim_cs_ex", *head, xs, ys, _luma_arg(luma), *consts,
         None if reduce else ctypes.byref(slots), _ptr(px), _ptr(py), pcode, dev, stream)
    return s, cs, partial, partial_cs, int(slots.value), px, py


def ssim_cs_partials(x, y, win, shift, C1, C2, pool_dtype, luma=None, u8_pyramid=False,
                     ssim_sums=True):
    """One inference MS-SSIM scale left unreduced: ``(partial, partial_cs,
    slots, npix, px, py)`` -- the per-plane partial sums of the SSIM map
    (``None`` unless ``ssim_sums``: MS-SSIM reads them only at its coarsest
    scale) and of the cs map (``slots`` per plane, packed), the plane's output
    pixel count, and the next pyramid level (``None`` at the coarsest scale).  The partial sums go
    to :func:`ms_ssim_reduce`; nothing is synchronised.  ``u8_pyramid``: x and
    y are levels of a uint8 pyramid (FA_DTYPE_U8_PYRAMID): float32, or the
    first level in float16, where its quarter samples are exact."""
    _, _, ps, pcs, slots, px, py = _cs_launch(x, y, win, shift, C1, C2, pool_dtype=pool_dtype,
                                              luma=luma, reduce=False, u8_pyramid=u8_pyramid,
                                              ssim_sums=ssim_sums)
    k = int(win.numel())
    npix = float((x.shape[-2] - k + 1) * (x.shape[-1] - k + 1))
    return ps, pcs, slots, npix, px, py


def ssim_cs_forward(x, y, win, shift, C1, C2, pool_dtype=None):
    """``(ssim, cs)`` plane means from the differentiable native path, plus the
    next pyramid level when ``pool_dtype`` is given."""
    s, cs, _, _, _, px, py = _cs_launch(_contig(x), _contig(y), win, shift, C1, C2,
                                        pool_dtype=pool_dtype)
    return (s, cs) if pool_dtype is None else (s, cs, px, py)


def ssim_cs_backward(x, y, gs, gcs, win, shift, C1, C2, need_dx, need_dy,
                     gpx=None, gpy=None):
    """Gradients of the plane means (and of the pyramid level the forward
    pooled, ``gpx`` / ``gpy``) with respect to x and y."""
    x, y, win = _contig(x), _contig(y), _win32(win)
    n, c, h, w = (int(v) for v in x.shape)
    k = int(win.numel())
    gsf = gs.to(torch.float32).contiguous().reshape(-1)
    gcsf = gcs.to(torch.float32).contiguous().reshape(-1)
    aux, dx, dy = _grad_buffers(x, y, k, need_dx, need_dy)
    gpx = _contig(gpx) if (gpx is not None and need_dx) else None
    gpy = _contig(gpy) if (gpy is not None and need_dy) else None
    dev, stream = _site(x)
    consts = (_ptr(win), k, n, c, h, w, float(shift), float(C1), float(C2))
    if x.dtype == torch.float32 and gpx is None and gpy is None:
        _run("fa_gpu_ssim_cs_backward", _ptr(x), _ptr(y), _ptr(gsf), _ptr(gcsf), *consts,
             _ptr(aux), _ptr(dx), _ptr(dy), dev, stream)
        return dx, dy
    if gpx is not None and gpy is not None and gpx.dtype != gpy.dtype:
        gpy = gpy.to(gpx.dtype)
    gp = gpx if gpx is not None else gpy
    gp_code = _DTYPE_CODE[gp.dtype if gp is not None else torch.float64]
    _run("fa_gpu_ssim_cs_backward_ex", _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], _ptr(gsf),
         _ptr(gcsf), *consts, _ptr(gpx), _ptr(gpy), gp_code, _ptr(aux), _ptr(dx), _ptr(dy),
         dev, stream)
    return dx, dy


def ms_ssim_keeps_coefficients() -> bool:
    """Whether MS-SSIM's training forward writes the backward's coefficient
    maps and keeps them until the backward (faster; peak memory one set of
    float32 maps per scale higher).  ``FA_MS_SSIM_RECOMPUTE=1`` recomputes
    them in the backward instead, as the reference does."""
    return os.environ.get("FA_MS_SSIM_RECOMPUTE", "0").lower() not in ("1", "on", "true", "yes")


def ssim_cs_coef_forward(x, y, win, shift, C1, C2, unit_s, pool_dtype, need_dy):
    """A training step's CS pass in float64 (``fa_gpu_ssim_cs_coef``): the
    plane means ``(s, cs)``, the next pyramid level when ``pool_dtype`` is
    given, and the backward's coefficient maps for a unit gradient of the SSIM
    means (``unit_s``) or of the cs means, 3 (4 with ``need_dy``) float32 per
    output pixel.  Returns ``(s, cs, px, py, aux)``."""
    x, y, win = _contig(x), _contig(y), _win32(win)
    n, c, h, w = (int(v) for v in x.shape)
    k = int(win.numel())
    planes = n * c
    bpp = workspace_slots("ssim", h, w, k)
    partial, partial_cs = _f64(x.device, planes, bpp), _f64(x.device, planes, bpp)
    s, cs = _f64(x.device, planes), _f64(x.device, planes)
    px = py = None
    if pool_dtype is not None:
        px = torch.empty((n, c, h // 2, w // 2), dtype=pool_dtype, device=x.device)
        py = torch.empty_like(px)
    aux = torch.empty((4 if need_dy else 3, planes, h - k + 1, w - k + 1), device=x.device,
                      dtype=torch.float32)
    dev, stream = _site(x)
    pcode = _DTYPE_CODE[pool_dtype if pool_dtype is not None else torch.float64]
    _run("fa_gpu_ssim_cs_coef", _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w, _ptr(win), k,
         float(shift), float(C1), float(C2), int(bool(unit_s)), _ptr(partial), _ptr(partial_cs),
         bpp, _ptr(s), _ptr(cs), _ptr(px), _ptr(py), pcode, _ptr(aux), int(bool(need_dy)),
         dev, stream)
    return s, cs, px, py, aux


def ssim_cs_scatter(x, y, g, aux, win, shift, need_dx, need_dy, gpx=None, gpy=None):
    """Gradients from ``ssim_cs_coef_forward``'s maps: each plane's share times
    ``g[plane]`` (the upstream gradient of the plane mean the maps were made
    for), plus a quarter of the pyramid level's gradient ``gpx`` / ``gpy``."""
    x, y, win = _contig(x), _contig(y), _win32(win)
    n, c, h, w = (int(v) for v in x.shape)
    k = int(win.numel())
    gf = _contig(g.to(torch.float64)).reshape(-1)
    dx = torch.empty_like(x) if need_dx else None
    dy = torch.empty_like(y) if need_dy else None
    gpx = _contig(gpx) if (gpx is not None and need_dx) else None
    gpy = _contig(gpy) if (gpy is not None and need_dy) else None
    if gpx is not None and gpy is not None and gpx.dtype != gpy.dtype:
        gpy = gpy.to(gpx.dtype)
    gp = gpx if gpx is not None else gpy
    gp_code = _DTYPE_CODE[gp.dtype if gp is not None else torch.float64]
    dev, stream = _site(x)
    _run("fa_gpu_ssim_cs_scatter", _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], _ptr(gf), _ptr(win), k,
         n, c, h, w, float(shift), _ptr(aux), int(aux.shape[0] == 4), _ptr(gpx), _ptr(gpy),
         gp_code, _ptr(dx), _ptr(dy), dev, stream)
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
    s, cs, _, _, _, px, py = _cs_launch(x, y, win, shift, C1, C2, pool_dtype=pool_dtype,
                                        luma=luma)
    return (s, cs) if pool_dtype is None else (s, cs, px, py)


def try_ssim_cs(x: torch.Tensor, y: torch.Tensor, *, win: torch.Tensor,
                shift: float, C1: float, C2: float):
    """``(ssim, cs)`` per plane, shaped ``(N, C)``; ``None`` if unavailable or
    a kernel declined the call (warned once)."""
    try:
        return _ssim_cs_native(x, y, win=win, shift=shift, C1=C1, C2=C2)
    except KernelError as exc:
        _declined(exc)
        return None


def _ssim_cs_native(x: torch.Tensor, y: torch.Tensor, *, win: torch.Tensor,
                    shift: float, C1: float, C2: float):
    k = int(win.numel())
    if x.shape[-2] < k or x.shape[-1] < k or k not in _WINDOWS:
        return None
    n, c, h, w = (int(v) for v in x.shape)
    if not x.is_cuda:
        lib = _cpu_ready(x, y)
        if lib is None:
            return None
        x, y, win = _contig(x), _contig(y), _win32(win)
        s = torch.empty((n * c,), dtype=torch.float64)
        cs = torch.empty((n * c,), dtype=torch.float64)
        _check_cpu(lib.fa_cpu_ssim_cs(
            _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w, _ptr(win), k,
            float(shift), float(C1), float(C2), _ptr(s), _ptr(cs)))
        return s.view(n, c), cs.view(n, c)
    if _gpu_ext(x) is None or not _usable(x, y):
        return None
    s, cs, *_ = _cs_launch(_contig(x), _contig(y), win, shift, C1, C2)
    return s.view(n, c), cs.view(n, c)


# --------------------------------------------------------------------------- #
# GMSD
# --------------------------------------------------------------------------- #


def try_gmsd(x: torch.Tensor, y: torch.Tensor, *, T: float, eps: float, downsample: bool,
             luma: Optional[tuple] = None, want_map: bool = False):
    """:func:`_gmsd_native`, or ``None`` when a kernel declined the call
    (warned once)."""
    try:
        return _gmsd_native(x, y, T=T, eps=eps, downsample=downsample, luma=luma,
                            want_map=want_map)
    except KernelError as exc:
        _declined(exc)
        return None


def _gmsd_native(x: torch.Tensor, y: torch.Tensor, *, T: float, eps: float,
                 downsample: bool, luma: Optional[tuple] = None, want_map: bool = False):
    """``(gms_mean, gmsd)`` per image, float64 -- plus the float32 q map when
    ``want_map``, or else their two batch means as a third, (2,) tensor -- or
    ``None`` if unavailable.

    ``luma`` = (kr, kg, kb[, offset]) makes the kernel read the three channels
    and form the luma plane itself; cropped views are read in place through
    their strides (``fa_gpu_gmsd_ex`` / ``fa_gpu_gmsd_once``).  CPU tensors
    run ``fa_cpu_gmsd`` (statistics only: no luma, no map).
    """
    n, c, h, w = (int(v) for v in x.shape)
    hd, wd = (h // 2, w // 2) if downsample else (h, w)
    if not x.is_cuda:
        lib = _cpu_ready(x, y) if luma is None and not want_map else None
        if lib is None or hd < 3 or wd < 3:
            return None
        x, y = _contig(x), _contig(y)
        mean = torch.empty((n,), dtype=torch.float64)
        dev = torch.empty((n,), dtype=torch.float64)
        _check_cpu(lib.fa_cpu_gmsd(
            _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w, float(T), float(eps),
            int(downsample), _ptr(mean), _ptr(dev)))
        return mean, dev
    if _gpu_ext(x) is None or not _usable(x, y):
        return None
    if luma is not None and c != 3:
        return None
    x, xs = _view_strides(x)
    y, ys = _view_strides(y)
    planes = n * (1 if luma is not None else c)
    return _gmsd_launch(x, y, xs, ys, luma, T, eps, downsample, planes, want_map, hd, wd)


def _gmsd_launch(x, y, xs, ys, luma, T, eps, downsample, planes, want_map, hd, wd,
                 separate=False):
    """``(mean, std, qmap)`` with the map, else ``(mean, std, batch)``: the
    batch means of both.  Without the map the statistics come from
    ``fa_gpu_gmsd_once``, which finishes a uint8 call inside its one launch.
    ``separate``: mean and std in allocations of their own (autograd outputs),
    not views of one."""
    n, c, h, w = (int(v) for v in x.shape)
    bpp = workspace_slots("gmsd", h, w, int(bool(downsample)))
    dev, stream = _site(x)
    head = (_ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w)
    consts = (float(T), float(eps), int(bool(downsample)))

    def workspaces():
        # one allocation for both (each torch allocation is ~1.7 us of host time)
        ps, pss = _f64(x.device, 2, planes, bpp).unbind(0)
        return _ptr(ps), _ptr(pss)

    if want_map:
        psum, psumsq = workspaces()
        mean, std = _f64(x.device, 2, n).unbind(0)
        qmap = torch.empty((n, planes // n, hd - 2, wd - 2), dtype=torch.float32,
                           device=x.device)
        _run("fa_gpu_gmsd_ex", *head, xs, ys, _luma_arg(luma), *consts, _ptr(qmap),
             psum, psumsq, bpp, _ptr(mean), _ptr(std), dev, stream)
        return mean, std, qmap
    if separate:
        mean, std, batch = _f64(x.device, n), _f64(x.device, n), None
    else:
        out = _f64(x.device, 2 * n + 2)
        mean, std, batch = out[:n], out[n:2 * n], out[2 * n:]
    acc = _acc_for("gmsd", x.device, dev, stream)
    lw = _luma_arg(luma)

    def args(ws):
        return (*head, xs, ys, lw, *consts, *ws, bpp, _ptr(acc), _ptr(mean), _ptr(std),
                _ptr(batch), dev, stream)

    if acc is None:
        _run("fa_gpu_gmsd_once", *args(workspaces()))
    else:
        _run_or_needs_workspace("fa_gpu_gmsd_once", args((None, None)),
                                lambda: args(workspaces()), acc)
    return mean, std, batch


def gmsd_autograd_available(x: torch.Tensor, y: torch.Tensor) -> bool:
    """Can the differentiable native GMS / GMSD path serve this call?"""
    return _autograd_ok(x, y, (torch.float32, torch.float64))


def gmsd_stats_fwd(x, y, T, eps, downsample):
    """Forward half of the differentiable GMS / GMSD: ``(mean, std)`` per image."""
    x, y = _contig(x), _contig(y)
    n, c, h, w = (int(v) for v in x.shape)
    hd, wd = (h // 2, w // 2) if downsample else (h, w)
    mean, std, _ = _gmsd_launch(x, y, None, None, None, T, eps, downsample, n * c, False,
                                hd, wd, separate=True)
    return mean, std


def gmsd_stats_bwd(x, y, mean, std, g_mean, g_std, T, eps, downsample, need_dx, need_dy):
    """dL/dx, dL/dy of L = g_mean . mean + g_std . std (float64 arithmetic)."""
    x, y = _contig(x), _contig(y)
    n, c, h, w = (int(v) for v in x.shape)
    hd, wd = (h // 2, w // 2) if downsample else (h, w)
    aux = torch.empty((4, n * c, hd - 2, wd - 2), dtype=torch.float64, device=x.device)
    gm = None if g_mean is None else g_mean.to(torch.float64).contiguous()
    gs = None if g_std is None else g_std.to(torch.float64).contiguous()
    dx = torch.empty_like(x) if need_dx else None
    dy = torch.empty_like(y) if need_dy else None
    dev, stream = _site(x)
    _run("fa_gpu_gmsd_backward", _ptr(x), _ptr(y), _DTYPE_CODE[x.dtype], n, c, h, w,
         float(T), float(eps), int(bool(downsample)), _ptr(mean), _ptr(std), _ptr(gm),
         _ptr(gs), _ptr(aux), _ptr(dx), _ptr(dy), dev, stream)
    return dx, dy


@functools.lru_cache(maxsize=256)
def _ms_workspace_bytes(code: int, n: int, c: int, h: int, w: int, k: int, m: int,
                        luma: bool) -> int:
    """Bytes of fa_gpu_ms_ssim's workspace for one call shape (asked once per
    shape, so a graph capture never issues the query)."""
    out = ctypes.c_int64(0)
    _run("fa_gpu_ms_ssim_workspace", code, n, c, h, w, k, m, int(luma), ctypes.byref(out))
    return int(out.value)


def ms_ssim_fused(x, y, win, shift, C1, C2, weights, luma=None, per_image=False):
    """Inference MS-SSIM in one C-ABI call (``fa_gpu_ms_ssim``): every scale's
    fused pass and the reduction, launched back to back from the library, over
    one workspace allocation; per-image values (``per_image``) or their
    batch mean.  With the stream's accumulator (none under graph capture) a
    uint8 call whose scales all fit the matrix-core kernel runs in three
    launches, the reduction finished in the last."""
    win = _win32(win)
    n, c, h, w = (int(v) for v in x.shape)
    k = int(win.numel())
    m = len(weights)
    x, xs = _view_strides(x)
    y, ys = _view_strides(y)
    code = _DTYPE_CODE[x.dtype]
    nbytes = _ms_workspace_bytes(code, n, c, h, w, k, m, luma is not None)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    out = _f64(x.device, n) if per_image else _f64(x.device)
    wts = (ctypes.c_double * m)(*[float(v) for v in weights])
    dev, stream = _site(x)
    acc = _acc_for("ms", x.device, dev, stream) if x.dtype == torch.uint8 and luma is None \
        else None
    _run_acc("fa_gpu_ms_ssim", acc, _ptr(x), _ptr(y), code, n, c, h, w, xs, ys,
             _luma_arg(luma), _ptr(win), k, float(shift), float(C1), float(C2), wts, m,
             _ptr(ws), nbytes, _ptr(acc) if acc is not None else None,
             _ptr(out) if per_image else None, None if per_image else _ptr(out), dev, stream)
    return out


def ms_head_available(terms) -> bool:
    """Can ``fa_gpu_ms_ssim_head`` combine these ``(N, C)`` plane means?"""
    t0 = terms[0]
    return (0 < len(terms) <= 8 and t0.is_cuda and t0.dim() == 2
            and all(t.dtype == torch.float64 and t.is_contiguous() and t.shape == t0.shape
                    and t.device == t0.device for t in terms)
            and _gpu_ext(t0) is not None)


def ms_head(terms, weights, per_image: bool) -> torch.Tensor:
    """MS-SSIM's head over formed plane means (``fa_gpu_ms_ssim_head``): the
    per-image values ``(N,)`` or their batch mean (a 0-d tensor)."""
    m = len(terms)
    n, c = (int(v) for v in terms[0].shape)
    ptrs = (ctypes.c_void_p * m)(*[t.data_ptr() for t in terms])
    wts = (ctypes.c_double * m)(*[float(v) for v in weights])
    out = _f64(terms[0].device, n) if per_image else _f64(terms[0].device)
    dev, stream = _site(terms[0])
    _run("fa_gpu_ms_ssim_head", ptrs, m, n, c, wts, _ptr(out) if per_image else None,
         None if per_image else _ptr(out), dev, stream)
    return out


def ms_head_backward(terms, weights, per_image: bool, g, needs):
    """Each scale's gradient of its plane means from the upstream gradient
    ``g`` of :func:`ms_head`'s output (``fa_gpu_ms_ssim_head_backward``); None
    where ``needs`` says no."""
    m = len(terms)
    n, c = (int(v) for v in terms[0].shape)
    g = _contig(g.to(torch.float64))
    grads = [torch.empty_like(t) if need else None for t, need in zip(terms, needs)]
    ptrs = (ctypes.c_void_p * m)(*[t.data_ptr() for t in terms])
    gptrs = (ctypes.c_void_p * m)(*[_ptr(v) for v in grads])
    wts = (ctypes.c_double * m)(*[float(v) for v in weights])
    dev, stream = _site(terms[0])
    _run("fa_gpu_ms_ssim_head_backward", ptrs, m, n, c, wts, _ptr(g) if per_image else None,
         None if per_image else _ptr(g), gptrs, dev, stream)
    return grads


def ms_ssim_reduce(partials, slots, npix, weights, n: int, c: int, per_image: bool):
    """MS-SSIM's per-scale plane reductions, clamp / power / product and the
    channel and batch means in two launches (``fa_gpu_ms_ssim_reduce``) from
    the partial sums of :func:`ssim_cs_partials`."""
    m = len(partials)
    ref = partials[0]
    arr = (ctypes.c_void_p * m)(*[t.data_ptr() for t in partials])
    sl = (ctypes.c_int * m)(*[int(v) for v in slots])
    npx = (ctypes.c_double * m)(*[float(v) for v in npix])
    wts = (ctypes.c_double * m)(*[float(v) for v in weights])
    terms = _f64(ref.device, m * n * c)
    out = _f64(ref.device, n) if per_image else _f64(ref.device)
    dev, stream = _site(ref)
    _run("fa_gpu_ms_ssim_reduce", arr, sl, npx, wts, m, n, c, _ptr(terms),
         _ptr(out) if per_image else None, None if per_image else _ptr(out), dev, stream)
    return out
